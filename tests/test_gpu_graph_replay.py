"""HIP graph replay of the chunked matvecs' in-launch reduce.

The down matvec of a dense or SwiGLU FFN at these shapes (18176 and 11008
columns) splits its rows into column chunks that hand their partial sums to
reducer workgroups of the same launch through tagged slots; the reducers
zero the slots again, so a replayed graph needs no reset (and records no
memset).  A call is captured on the handle's stream after eager calls have
allocated the workspace and the slot area; the graph is then replayed with
new inputs in the captured buffer, with eager calls and synchronisations in
between, and every replay must equal the eager result to the bit."""
import ctypes

import numpy as np
import pytest
import torch

import llg
import llg.gguf as gg
from tests.helpers import normal

pytestmark = pytest.mark.gpu


def _bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _gpu_quant(shape, std, seed, t):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return gg.quantize(torch.randn(shape, generator=g, device="cuda") * std, t).cpu().numpy()


def _vp(t: torch.Tensor):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("kind,h,ff", [("dense", 4544, 18176), ("swiglu", 4096, 11008)])
def test_chunked_down_graph_replay(dev, rng, kind, h, ff):
    t = gg.Q4_0
    u = dev.upload_matrix(_gpu_quant((ff, h), 0.02, 71, t), t, ff, h)
    d = dev.upload_matrix(_gpu_quant((h, ff), 0.02, 72, t), t, h, ff)
    g = dev.upload_matrix(_gpu_quant((ff, h), 0.02, 73, t), t, ff, h)
    xd = torch.empty(h, device="cuda")
    outd = torch.empty(h, device="cuda")

    def call():
        if kind == "dense":
            dev.check(dev.lib.llg_hipd_ffn_dense(dev.h, u.id, d.id, _vp(xd), gg.ACT_RELU,
                                                 _vp(outd)), "ffn_dense")
        else:
            dev.check(dev.lib.llg_hipd_ffn_swiglu(dev.h, g.id, u.id, d.id, _vp(xd), _vp(outd)),
                      "ffn_swiglu")

    xs = [normal(rng, h, 1.0) for _ in range(4)]
    refs = []
    for x in xs:  # eager results (the first call allocates what the graph uses)
        xd.copy_(torch.from_numpy(x))
        torch.cuda.synchronize()
        call()
        dev.sync()
        refs.append(outd.cpu().numpy().copy())
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.ExternalStream(dev.stream)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        call()
    torch.cuda.synchronize()
    for _ in range(3):
        for x, ref in zip(xs, refs):
            xd.copy_(torch.from_numpy(x))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert np.array_equal(_bits(outd.cpu().numpy()), _bits(ref))
            call()  # eager work between the replays
            dev.sync()
            assert np.array_equal(_bits(outd.cpu().numpy()), _bits(ref))
    del graph
    for m in (u, d, g):
        m.release()
