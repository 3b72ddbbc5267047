"""The in-launch hand-offs' fallback paths, forced from the host.

A consumer of a tagged-slot hand-off (the chunked matvec's reducer
workgroups, the fused sparse step's tile workgroups, the Falcon tile launch's
tile workgroups, the window step's down workgroups) computes a value itself when its slot stays empty for the
poll bound, so that every wait ends.  In a working launch that never
happens.  A device created with LLG_CHECK_HANDOFF set makes every consumer,
after the usual wait, compute every handed-over value itself and use its own;
these tests require the results of such a device to equal, to the bit, those
of a normal device on the same inputs.  That pins the fallback's sums (the
same blocks, block sums and order as the producers) without any wait being
cut short, so no slot is left filled for a later launch."""
import os

import numpy as np
import pytest
import torch

import llg
import llg.gguf as gg
from oracle import refcpu as R
from tests.helpers import make_falcon, make_sparse_layer, max_rel_err, normal, ref_falcon_f64, \
    threshold_for, window_sets

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev_check():
    os.environ["LLG_CHECK_HANDOFF"] = "1"
    try:
        d = llg.Device()
    finally:
        del os.environ["LLG_CHECK_HANDOFF"]
    yield d
    d.close()


def _bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32).view(np.uint32)




def _gpu_quant(shape, std, seed, t):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return gg.quantize(torch.randn(shape, generator=g, device="cuda") * std, t).cpu().numpy()


@pytest.mark.parametrize("t,h,ff", [(gg.Q4_0, 4544, 18176), (gg.Q8_0, 4544, 18176),
                                    (gg.F16, 4544, 18176), (gg.F32, 1024, 8192)])
def test_dense_chunk_reduce_fallback_bit_identical(dev, dev_check, rng, t, h, ff):
    """Dense FFN and SwiGLU FFN: the down matvec's column chunks (4 for 18176
    columns, 2 for 8192) reduced from the slots, or every chunk sum computed
    by the reducer from x in memory.  Bit-identical for Q4_0, F16 and F32,
    whose block dots are explicit fused multiply-adds.  The Q8_0 block dot
    leaves the contraction of its products to the compiler (forcing it spills
    34-42 registers in the 1024-thread Q8_0 instances), and the reducer's
    inlined copy contracts them otherwise: its chunk sums differ in their
    last bits, so the outputs agree within 1e-6 of their largest magnitude
    (a few ulps of the largest; more ulps only where a sum cancels)."""
    up, down = _gpu_quant((ff, h), 0.02, 51, t), _gpu_quant((h, ff), 0.02, 52, t)
    gate = _gpu_quant((ff, h), 0.02, 53, t)
    x = normal(rng, h, 1.0)
    outs = []
    for dv in (dev, dev_check):
        u, d = dv.upload_matrix(up, t, ff, h), dv.upload_matrix(down, t, h, ff)
        g = dv.upload_matrix(gate, t, ff, h)
        outs.append((llg.ffn_dense(dv, u, d, x, gg.ACT_RELU), llg.ffn_swiglu(dv, g, u, d, x)))
        for m in (u, d, g):
            m.release()
    for a, b in zip(outs[0], outs[1]):
        if t == gg.Q8_0:
            assert np.max(np.abs(a - b)) <= 1e-6 * np.max(np.abs(a))
        else:
            assert np.array_equal(_bits(a), _bits(b))
    assert max_rel_err(outs[1][0], R.ffn_dense(up, down, t, h, ff, x)) <= 1e-3


def test_fused_sparse_fallback_bit_identical(dev, dev_check, rng):
    """ffnFlash path 2 at the Falcon-7B layer's shape with the predictor in the
    tile launch: the hidden units from the predictor workgroups' slots, or all
    128 computed by every tile workgroup itself."""
    h, ff, rank = 4544, 18176, 128
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    wup, wout = normal(rng, (rank, h), 0.05), normal(rng, (ff, rank), 0.05)
    x = normal(rng, h, 1.0)
    _, lg = R.predict(wup, wout, None, x, 0.0)
    res = []
    for dv in (dev, dev_check):
        p = llg.Predictor(dv, wup, wout, None, threshold_for(lg, 909))
        b = dv.upload_bundle(up, dn, gg.Q4_0, h, ff)
        res.append(llg.ffn_predict_sparse(dv, p, b, x, x))
        b.release()
    assert np.array_equal(_bits(res[0][0]), _bits(res[1][0]))
    assert np.array_equal(res[0][1], res[1][1])


FALCON = dict(n_layers=2, hidden=256, n_heads=4, n_kv=1, head_dim=64, ff=512, vocab=300,
              max_seq=64, rank=16, rope_base=10000.0, eps=1e-5)


def test_falcon_tile_launch_fallback_bit_identical(dev, dev_check, rng):
    """A Falcon decode whose layers run Wo and the predictor in the tile launch:
    the hidden units from the combiner workgroups' slots, or merged from the
    attention splits' products by every tile workgroup itself; logits equal
    to the bit at every one of 24 positions."""
    d = dict(FALCON)
    w = make_falcon(rng, d)
    prompt = rng.integers(0, d["vocab"], 24)
    _, _, thr = ref_falcon_f64(w, d, prompt)
    runs = []
    for dv in (dev, dev_check):
        m = llg.FalconModel(dv, d, w, thr)
        runs.append([m.forward(int(tk), s) for s, tk in enumerate(prompt)])
        m.release()
    for (l0, _, n0), (l1, _, n1) in zip(*runs):
        assert np.array_equal(_bits(l0), _bits(l1))
        assert np.array_equal(n0, n1)


@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16, gg.F32])
def test_window_step_fallback_bit_identical(dev, dev_check, rng, t):
    """Window steps (update + FFN in one launch, k = 3, 20 tokens of 120 active
    neurons, 60% carried over): each entry's activation from the up
    workgroups' slot, or computed by the down workgroup itself."""
    h, ff = 512, 1024
    up, dn = make_sparse_layer(rng, h, ff, t)
    sets = window_sets(rng, ff, 120, 20, 0.6)
    xs = [normal(rng, h, 1.0) for _ in sets]
    runs = []
    for dv in (dev, dev_check):
        b = dv.upload_bundle(up, dn, t, h, ff)
        nc = llg.NeuronCache(dv, b, 3)
        d_out = torch.empty(h, device="cuda")
        d_n = torch.empty(1, dtype=torch.int32, device="cuda")
        outs = []
        for a, x in zip(sets, xs):
            d_x = torch.from_numpy(x).cuda()
            d_a = torch.from_numpy(np.ascontiguousarray(a, np.int32)).cuda()
            d_n.fill_(a.size)
            torch.cuda.synchronize()
            nc.step_device(d_x.data_ptr(), d_a.data_ptr(), d_n.data_ptr(), d_out.data_ptr())
            dv.sync()
            outs.append(d_out.cpu().numpy())
        runs.append((outs, nc.resident()))
        nc.win.release()
        b.release()
    for o0, o1 in zip(runs[0][0], runs[1][0]):
        assert np.array_equal(_bits(o0), _bits(o1))
    assert np.array_equal(runs[0][1], runs[1][1])


def test_matvec_slot_area_grows(rng):
    """On a fresh handle, a chunked matvec of 512 rows (4 column chunks) and
    then one of 20000 rows: the second needs 4 x 20000 slots (640 KB), more
    than the first call's area (256 KB), so the area is replaced by a larger
    zeroed one between the calls.  Both against the oracle."""
    t = gg.Q4_0
    dv = llg.Device()
    try:
        for rows, cols in [(512, 18176), (20000, 18176)]:
            w = _gpu_quant((rows, cols), 0.02, 81 + rows, t)
            x = normal(rng, cols, 1.0)
            m = dv.upload_matrix(w, t, rows, cols)
            got = dv.matvec_q(m, x)
            ref = R.matmulvec(np.stack([R.dequantize(w[r], t) for r in range(rows)]), x)
            assert max_rel_err(got, ref) <= 1e-5, rows
            m.release()
    finally:
        dv.close()
