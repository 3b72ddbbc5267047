"""Run-to-run determinism: the same inputs give bit-identical outputs on every
call, as the reference's sequential CPU loops do (ffn_flash.go:273-298,
window.go:143-180, forward.go:106-314).  Every output element of these paths
is summed by one workgroup in a fixed order (no floating-point atomics), so
repeated calls, fresh device objects and fresh models must agree to the bit,
and so must greedy token streams."""
import numpy as np
import pytest
import torch

import llg
import llg.gguf as gg
from oracle import refcpu as R
from tests.helpers import make_falcon, make_sparse_layer, max_rel_err, normal, ref_falcon_f64, \
    threshold_for, window_sets

pytestmark = pytest.mark.gpu

REPEATS = 4


def _bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _same_bits(outs):
    for o in outs[1:]:
        assert np.array_equal(_bits(o), _bits(outs[0]))


@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16, gg.F32])
def test_sparse_ffn_repeats_bit_identical(dev, rng, t):
    """ffnSparseLoad at the Falcon-7B layer's shape with 909 neurons, repeated
    calls and a second upload of the same bundle."""
    h, ff = 4544, 18176
    up, dn = make_sparse_layer(rng, h, ff, t)
    x = normal(rng, h, 1.0)
    active = np.sort(rng.choice(ff, 909, replace=False)).astype(np.int32)
    b1 = dev.upload_bundle(up, dn, t, h, ff)
    b2 = dev.upload_bundle(up, dn, t, h, ff)
    outs = [llg.ffn_sparse_load(dev, b, x, active) for b in [b1, b2] * (REPEATS // 2)]
    _same_bits(outs)
    assert max_rel_err(outs[0], R.ffn_sparse_load(up, dn, t, h, ff, x, active)) <= 1e-3
    b1.release()
    b2.release()


def test_predict_sparse_repeats_bit_identical(dev, rng):
    """ffnFlash path 2 (predictor, selection, gathered FFN) at the Falcon-7B
    layer's shape: repeated calls give the same active set and output bits."""
    h, ff, rank = 4544, 18176, 128
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    wup, wout = normal(rng, (rank, h), 0.05), normal(rng, (ff, rank), 0.05)
    x = normal(rng, h, 1.0)
    _, lg = R.predict(wup, wout, None, x, 0.0)
    p = llg.Predictor(dev, wup, wout, None, threshold_for(lg, 909))
    b = dev.upload_bundle(up, dn, gg.Q4_0, h, ff)
    res = [llg.ffn_predict_sparse(dev, p, b, x, x) for _ in range(REPEATS)]
    _same_bits([r[0] for r in res])
    for r in res[1:]:
        assert np.array_equal(r[1], res[0][1])
    b.release()


def test_window_sequence_bit_identical(dev, rng):
    """Two sliding windows over the same bundle and the same 24-token active
    sets (k = 5, 70% carry-over) give bit-identical outputs token by token."""
    h, ff, n_act = 1024, 4096, 205
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    b = dev.upload_bundle(up, dn, gg.Q4_0, h, ff)
    sets = window_sets(rng, ff, n_act, 24, 0.7)
    xs = [normal(rng, h, 1.0) for _ in sets]
    runs = []
    for _ in range(2):
        nc = llg.NeuronCache(dev, b, 5)
        outs = []
        for a, x in zip(sets, xs):
            nc.update(a)
            outs.append(nc.ffn_forward(x, a))
        runs.append(outs)
        nc.win.release()
    for o0, o1 in zip(*runs):
        assert np.array_equal(_bits(o0), _bits(o1))
    b.release()


FALCON = dict(n_layers=2, hidden=256, n_heads=4, n_kv=1, head_dim=64, ff=512, vocab=300,
              max_seq=64, rank=16, rope_base=10000.0, eps=1e-5)


def test_falcon_decode_bit_identical(dev, rng):
    """Two models built from the same weights decode the same 40 tokens (the
    prompt through ForwardFlash, then the device greedy loop): logits equal to
    the bit at every position and the greedy streams equal."""
    d = dict(FALCON)
    w = make_falcon(rng, d)
    prompt = rng.integers(0, d["vocab"], 24)
    _, _, thr = ref_falcon_f64(w, d, prompt)
    runs = []
    for _ in range(2):
        m = llg.FalconModel(dev, d, w, thr)
        logits = [m.forward(int(tk), s)[0] for s, tk in enumerate(prompt)]
        gen = torch.zeros(17, dtype=torch.int32, device="cuda")
        gen[0] = int(np.argmax(logits[-1]))
        torch.cuda.synchronize()
        for i in range(16):
            m.step_device(gen.data_ptr() + 4 * i, len(prompt) + i, gen.data_ptr() + 4 * (i + 1))
        dev.sync()
        runs.append((logits, gen.cpu().numpy()))
        m.release()
    for l0, l1 in zip(runs[0][0], runs[1][0]):
        assert np.array_equal(_bits(l0), _bits(l1))
    assert np.array_equal(runs[0][1], runs[1][1])


def _gpu_quant(shape, std, seed, t):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return gg.quantize(torch.randn(shape, generator=g, device="cuda") * std, t).cpu().numpy()


@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0])
def test_dense_ffn_repeats_bit_identical(dev, rng, t):
    """The dense FFN at the Falcon-7B layer's shape: its down matvec splits the
    18176-wide rows into column chunks whose partial sums are added in chunk
    order, so repeated calls agree to the bit."""
    h, ff = 4544, 18176
    up, down = _gpu_quant((ff, h), 0.02, 41, t), _gpu_quant((h, ff), 0.02, 42, t)
    u, d = dev.upload_matrix(up, t, ff, h), dev.upload_matrix(down, t, h, ff)
    x = normal(rng, h, 1.0)
    outs = [llg.ffn_dense(dev, u, d, x, gg.ACT_RELU) for _ in range(REPEATS)]
    _same_bits(outs)
    assert max_rel_err(outs[0], R.ffn_dense(up, down, t, h, ff, x)) <= 1e-3
    gate = _gpu_quant((ff, h), 0.02, 43, t)
    gt = dev.upload_matrix(gate, t, ff, h)
    _same_bits([llg.ffn_swiglu(dev, gt, u, d, x) for _ in range(REPEATS)])
    for m in (u, d, gt):
        m.release()


@pytest.mark.parametrize("n_tok", [1, 3, 77])
def test_moe_repeats_bit_identical(dev, rng, n_tok):
    """moeFFN at the Mixtral layer's shape: decode batches (per-token expert
    kernels, partial dot products added in chunk then slot order) and a
    grouped-GEMM batch give bit-identical outputs, ids and weights."""
    d, eff, E, k = 4096, 14336, 8, 2
    router = normal(rng, (E, d), 0.02)
    gate = _gpu_quant((E * eff, d), 0.02, 51, gg.Q4_0)
    up = _gpu_quant((E * eff, d), 0.02, 52, gg.Q4_0)
    down = _gpu_quant((E * d, eff), 0.02, 53, gg.Q4_0)
    hs = [dev.upload_f32(router), dev.upload_matrix(gate, gg.Q4_0, E * eff, d),
          dev.upload_matrix(up, gg.Q4_0, E * eff, d), dev.upload_matrix(down, gg.Q4_0, E * d, eff)]
    x = normal(rng, (n_tok, d), 1.0)
    res = [llg.moe_ffn(dev, *hs, E, k, x) for _ in range(REPEATS)]
    _same_bits([r[0] for r in res])
    for r in res[1:]:
        assert np.array_equal(r[1], res[0][1]) and np.array_equal(_bits(r[2]), _bits(res[0][2]))
    for hnd in hs:
        hnd.release()
