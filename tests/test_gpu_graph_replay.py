"""HIP graph replay of the in-launch hand-offs.

The down matvec of a dense or SwiGLU FFN at these shapes (18176 and 11008
columns) splits its rows into column chunks that hand their partial sums to
reducer workgroups of the same launch through tagged slots, which the
reducers zero again; the fused sparse step hands the predictor's hidden
units to its tiles in slots tagged with an epoch that its reduce advances on
the device, as do the layers of the Falcon step.  So a replayed graph needs
no reset (and records no memset).  A
call is captured on the handle's stream after eager calls have allocated
what it uses; the graph is then replayed with new inputs in the captured
buffer, with eager calls and synchronisations in between, and every replay
must equal the eager result to the bit."""
import ctypes

import numpy as np
import pytest
import torch

import llg
import llg.gguf as gg
from oracle import refcpu as R
from tests.helpers import make_falcon, make_sparse_layer, normal, ref_falcon_f64, threshold_for

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


def test_fused_sparse_step_graph_replay(dev, rng):
    """ffnFlash path 2 at the Falcon-7B layer's shape: the predictor workgroups
    hand the hidden units to the tiles in slots tagged with the sync area's
    epoch, and k_tile_reduce advances the epoch word on the device, so a
    replay never accepts a slot from an earlier one.  Captured once, replayed
    12 times with new inputs and eager calls between: outputs and active
    lists equal the eager ones to the bit."""
    h, ff, rank = 4544, 18176, 128
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    wup, wout = normal(rng, (rank, h), 0.05), normal(rng, (ff, rank), 0.05)
    xs = [normal(rng, h, 1.0) for _ in range(4)]
    _, lg = R.predict(wup, wout, None, xs[0], 0.0)
    thr = threshold_for(lg, 909)
    p = llg.Predictor(dev, wup, wout, None, thr)
    b = dev.upload_bundle(up, dn, gg.Q4_0, h, ff)
    xd = torch.empty(h, device="cuda")
    outd = torch.empty(h, device="cuda")
    actd = torch.empty(ff, dtype=torch.int32, device="cuda")
    nd = torch.empty(1, dtype=torch.int32, device="cuda")

    def call():
        dev.check(dev.lib.llg_hipd_ffn_predict_sparse(
            dev.h, p.w_up.id, p.w_out.id, p.bias_id, b.id, _vp(xd), _vp(xd), ctypes.c_float(thr),
            gg.ACT_RELU, _vp(outd), _vp(actd), _vp(nd)), "ffn_predict_sparse")

    def result():
        k = int(nd.cpu()[0])
        return outd.cpu().numpy().copy(), actd[:k].cpu().numpy().copy()

    refs = []
    for x in xs:  # eager results (the first call allocates the workspace and sync area)
        xd.copy_(torch.from_numpy(x))
        torch.cuda.synchronize()
        call()
        dev.sync()
        refs.append(result())
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.ExternalStream(dev.stream)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        call()
    torch.cuda.synchronize()
    for _ in range(3):
        for x, (ro, ra) in zip(xs, refs):
            xd.copy_(torch.from_numpy(x))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            o, a = result()
            assert np.array_equal(_bits(o), _bits(ro)) and np.array_equal(a, ra)
            call()  # eager work between the replays
            dev.sync()
            o, a = result()
            assert np.array_equal(_bits(o), _bits(ro)) and np.array_equal(a, ra)
    del graph
    b.release()


FALCON = dict(n_layers=2, hidden=256, n_heads=4, n_kv=1, head_dim=64, ff=512, vocab=300,
              max_seq=64, rank=16, rope_base=10000.0, eps=1e-5)


def test_falcon_step_graph_replay(dev, rng):
    """One decode step of a Falcon model whose layers run Wo and the predictor
    in the tile launch (combiner slots, the sync area's epoch), captured at
    position 23 after an eager prefill of positions 0-22 and replayed with
    four different tokens, eager steps at the same position in between: the
    logits (copied out by the step) equal the eager ones to the bit and the
    next token is the same."""
    d = dict(FALCON)
    w = make_falcon(rng, d)
    prompt = rng.integers(0, d["vocab"], 24)
    _, _, thr = ref_falcon_f64(w, d, prompt)
    m = llg.FalconModel(dev, d, w, thr)
    toks = torch.tensor(prompt.astype(np.int32), device="cuda")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    pos = 23
    for s_ in range(pos):
        m.step_device(toks.data_ptr() + 4 * s_, s_, sink.data_ptr())
    dev.sync()
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    nxt = torch.zeros(1, dtype=torch.int32, device="cuda")
    lg = torch.empty(d["vocab"], device="cuda")
    cands = [int(c) for c in rng.integers(0, d["vocab"], 4)]

    def step():
        m.step_device(tok.data_ptr(), pos, nxt.data_ptr(), lg.data_ptr())

    refs = []
    for c in cands:
        tok.fill_(c)
        torch.cuda.synchronize()
        step()
        dev.sync()
        refs.append((lg.cpu().numpy().copy(), int(nxt.cpu()[0])))
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.ExternalStream(dev.stream)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        step()
    torch.cuda.synchronize()
    for _ in range(3):
        for c, (rl, rn) in zip(cands, refs):
            tok.fill_(c)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert np.array_equal(_bits(lg.cpu().numpy()), _bits(rl)) and int(nxt.cpu()[0]) == rn
            step()  # eager work between the replays
            dev.sync()
            assert np.array_equal(_bits(lg.cpu().numpy()), _bits(rl)) and int(nxt.cpu()[0]) == rn
    del graph
    m.release()
