"""GPU parity: the gfx950 library (through the C ABI) against the CPU oracle
on the same seeded inputs.

Bars (from the hot-path contract):
  - dequantized values, active index sets and MoE expert ids: bit-exact;
  - FFN outputs: max |gpu - oracle| <= 1e-3 * max |oracle| (fp32 accumulation);
  - predictor logits: fp32 reordering only (max rel 1e-5 of max |logit|).
Sizes are the configs' real shapes where the oracle finishes in seconds, and
tiny/ragged shapes for the edge cases.
"""
import ctypes

import numpy as np
import pytest
import torch

import llg
import llg.gguf as gg
from oracle import refcpu as R
from tests.helpers import (make_falcon, make_sparse_layer, max_rel_err, normal, quant,
                           ref_falcon_f64, threshold_for, window_sets)

pytestmark = pytest.mark.gpu

TOL = 1e-3  # FFN output tolerance relative to the output's max-abs


def gpu_normal(shape, std, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return torch.randn(shape, generator=g, device="cuda", dtype=torch.float32) * std


def gpu_quant(shape, std, seed, t) -> np.ndarray:
    """Big weights: drawn and quantized on the GPU, bytes returned to the host."""
    return gg.quantize(gpu_normal(shape, std, seed), t).cpu().numpy()


# ---------------------------------------------------------------- dequant
@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16, gg.F32])
def test_dequant_bit_exact(dev, rng, t):
    rows, cols = 37, 4544
    raw = quant(normal(rng, (rows, cols), 0.02), t)
    if t in (gg.Q4_0, gg.Q8_0):
        bs = 18 if t == gg.Q4_0 else 34
        specials = [0x0001, 0x03FF, 0x7C00, 0xFC00, 0x7E01, 0xFE00, 0x8000, 0x0000, 0x7BFF]
        for i, hb in enumerate(specials):  # f16 scale specials, incl. NaN payloads
            raw[i, 0:2] = [hb & 0xFF, hb >> 8]
            raw[i, bs:bs + 2] = [hb & 0xFF, hb >> 8]
    elif t == gg.F16:
        raw[0, :8] = np.array([0x0001, 0x7E01, 0xFC00, 0x8000], np.uint16).view(np.uint8)
    m = dev.upload_matrix(raw, t, rows, cols)
    got = dev.dequant(m, 0, rows)
    ref = np.stack([R.dequantize(raw[r], t) for r in range(rows)])
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    part = dev.dequant(m, 5, 3)
    assert np.array_equal(part.view(np.uint32), ref[5:8].view(np.uint32))
    m.release()


def test_dequant_bundle_rows(dev, rng):
    h, ff = 256, 50
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    b = dev.upload_bundle(up, dn, gg.Q4_0, h, ff)
    got = dev.dequant(b, 10, 4)
    for i in range(4):
        assert np.array_equal(got[i, :h], R.dequantize(up[10 + i], gg.Q4_0))
        assert np.array_equal(got[i, h:], R.dequantize(dn[10 + i], gg.Q4_0))
    b.release()


# ---------------------------------------------------------------- selection
@pytest.mark.parametrize("ff", [1, 63, 64, 65, 1000, 18176, 100003])
def test_select_bit_exact(dev, rng, ff):
    lg = normal(rng, ff, 1.0)
    lg[rng.choice(ff, min(ff, 5), replace=False)] = 0.25  # ties exactly at the threshold
    for thr in (0.25, 1.645, -10.0, 10.0):
        assert np.array_equal(dev.select(lg, thr), R.select(lg, thr))


# ---------------------------------------------------------------- predictor
@pytest.mark.parametrize("h,rank,ff,bias", [(64, 16, 256, True), (4544, 128, 18176, False),
                                            (4544, 128, 18176, True), (96, 20, 300, False)])
def test_predict(dev, rng, h, rank, ff, bias):
    wup, wout = normal(rng, (rank, h), 0.05), normal(rng, (ff, rank), 0.05)
    b = normal(rng, ff, 0.01) if bias else None
    a = normal(rng, h, 1.0)
    _, ref_lg = R.predict(wup, wout, b, a, 0.0)
    n_target = max(1, int(round(0.05 * ff)))
    thr = threshold_for(ref_lg, n_target)
    ref_act, _ = R.predict(wup, wout, b, a, thr)
    assert ref_act.size == n_target
    p = llg.Predictor(dev, wup, wout, b, thr)
    act, lg = p.predict(a, return_logits=True)
    assert np.max(np.abs(lg - ref_lg)) <= 1e-5 * np.max(np.abs(ref_lg))
    assert np.array_equal(act, ref_act)
    # selection on the oracle's own logits is bit-exact by construction of the hook
    assert np.array_equal(dev.select(ref_lg, thr), ref_act)


# ---------------------------------------------------------------- sparse FFN
@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16, gg.F32])
@pytest.mark.parametrize("h,ff,n", [(64, 64, 1), (128, 512, 40), (256, 333, 333)])
def test_ffn_sparse_small(dev, rng, t, h, ff, n):
    up, dn = make_sparse_layer(rng, h, ff, t)
    x = normal(rng, h, 1.0)
    active = np.sort(rng.choice(ff, n, replace=False)).astype(np.int32)
    b = dev.upload_bundle(up, dn, t, h, ff)
    for act in (gg.ACT_RELU, gg.ACT_SILU, gg.ACT_GELU):
        got = llg.ffn_sparse_load(dev, b, x, active, act)
        ref = R.ffn_sparse_load(up, dn, t, h, ff, x, active, act)
        assert max_rel_err(got, ref) <= TOL, (t, h, ff, n, act)
    b.release()


@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16])
def test_ffn_sparse_config0(dev, rng, t):
    """Falcon-7B-shaped layer, d=4544, F=18176, 909 active neurons."""
    h, ff = 4544, 18176
    up = gpu_quant((ff, h), 0.02, 11, t)
    dn = gpu_quant((ff, h), 0.02, 12, t)
    x = normal(rng, h, 1.0)
    active = np.sort(rng.choice(ff, 909, replace=False)).astype(np.int32)
    b = dev.upload_bundle(up, dn, t, h, ff)
    got = llg.ffn_sparse_load(dev, b, x, active)
    ref = R.ffn_sparse_load(up, dn, t, h, ff, x, active)
    assert max_rel_err(got, ref) <= TOL
    # unsorted indices are accepted like the reference's []int, and a
    # repeated index adds its neuron once per occurrence (ffn_flash.go:262-298
    # reads and accumulates every listed row)
    perm = active[::-1].copy()
    assert max_rel_err(llg.ffn_sparse_load(dev, b, x, perm),
                       R.ffn_sparse_load(up, dn, t, h, ff, x, perm)) <= TOL
    rep = np.concatenate([active[:300], active[100:200], active[:50], active[300:]])
    rep = rep[rng.permutation(rep.size)].astype(np.int32)
    got = llg.ffn_sparse_load(dev, b, x, rep)
    ref_rep = R.ffn_sparse_load(up, dn, t, h, ff, x, rep)
    assert max_rel_err(got, ref_rep) <= TOL
    assert max_rel_err(ref_rep, ref) > 10 * TOL  # the repeats do count
    b.release()


def test_ffn_sparse_edge_cases(dev, rng):
    h, ff = 64, 64
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    b = dev.upload_bundle(up, dn, gg.Q4_0, h, ff)
    x = normal(rng, h, 1.0)
    assert np.all(llg.ffn_sparse_load(dev, b, x, np.array([], np.int32)) == 0)
    with pytest.raises(llg.LlgError) as e:
        llg.ffn_sparse_load(dev, b, x, np.array([3, 64], np.int32))
    assert e.value.code == llg.LLG_E_RANGE
    with pytest.raises(llg.LlgError) as e:
        llg.ffn_sparse_load(dev, b, x, np.array([-1], np.int32))
    assert e.value.code == llg.LLG_E_RANGE
    allact = np.arange(ff, dtype=np.int32)
    assert max_rel_err(llg.ffn_sparse_load(dev, b, x, allact),
                       R.ffn_sparse_load(up, dn, gg.Q4_0, h, ff, x, allact)) <= TOL
    b.release()


@pytest.mark.parametrize("t,bias", [(gg.Q4_0, False), (gg.Q4_0, True), (gg.F16, False),
                                    (gg.F16, True), (gg.F32, False)])
def test_ffn_predict_sparse_config0(dev, rng, t, bias):
    """Path 2 of ffnFlash (ffn_flash.go:225-231): predictor + selection +
    gathered FFN in one call at the config-0 shape with exactly 909 active
    neurons.  Q4_0 rows are the config's; F16 and F32 bundles take the
    fused kernel's wide-row layout (dtype.go:12-38 dequant).  With a bias the
    logits are B.(A.x) + bias (predictor.go:69-73)."""
    h, ff, rank = 4544, 18176, 128
    up = gpu_quant((ff, h), 0.02, 21, t)
    dn = gpu_quant((ff, h), 0.02, 22, t)
    wup, wout = normal(rng, (rank, h), 0.05), normal(rng, (ff, rank), 0.05)
    bv = normal(rng, ff, 0.05) if bias else None
    x = normal(rng, h, 1.0)
    _, lg = R.predict(wup, wout, bv, x, 0.0)
    thr = threshold_for(lg, 909)
    ref_act, _ = R.predict(wup, wout, bv, x, thr)
    assert ref_act.size == 909
    ref = R.ffn_sparse_load(up, dn, t, h, ff, x, ref_act)
    b = dev.upload_bundle(up, dn, t, h, ff)
    p = llg.Predictor(dev, wup, wout, bv, thr)
    out, act = llg.ffn_predict_sparse(dev, p, b, x, x)
    assert np.array_equal(act, ref_act)
    assert max_rel_err(out, ref) <= TOL
    b.release()


@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16, gg.F32])
@pytest.mark.parametrize("h,ff,rank", [(256, 1024, 32), (160, 1000, 20), (4544, 2048, 128)])
@pytest.mark.parametrize("bias", [False, True])
def test_ffn_predict_sparse_densities(dev, rng, t, h, ff, rank, bias):
    """The fused predictor -> selection -> gathered FFN at the extremes of
    density: no neuron (a zero output), about half of them (tiles with more
    active neurons than one round of up rows covers) and every neuron; the
    second shape has a partial last tile and a hidden size of 5 blocks, the
    third the config-0 hidden size (F16/F32: two passes of the down loop).
    With a bias vector the logits carry it (predictor.go:69-73)."""
    up, dn = make_sparse_layer(rng, h, ff, t)
    wup, wout = normal(rng, (rank, h), 0.05), normal(rng, (ff, rank), 0.05)
    bv = normal(rng, ff, 0.05) if bias else None
    x, a = normal(rng, h, 1.0), normal(rng, h, 1.0)
    _, lg = R.predict(wup, wout, bv, a, 0.0)
    b = dev.upload_bundle(up, dn, t, h, ff)
    for n_target in (0, ff // 2, ff):
        thr = float(np.max(lg)) + 1.0 if n_target == 0 else (
            float(np.min(lg)) - 1.0 if n_target == ff else threshold_for(lg, n_target))
        ref_act, _ = R.predict(wup, wout, bv, a, thr)
        assert ref_act.size == n_target
        p = llg.Predictor(dev, wup, wout, bv, thr)
        out, act = llg.ffn_predict_sparse(dev, p, b, a, x)
        assert np.array_equal(act, ref_act), n_target
        ref = R.ffn_sparse_load(up, dn, t, h, ff, x, ref_act)
        if n_target == 0:
            assert np.all(out == 0)
        else:
            assert max_rel_err(out, ref) <= TOL, n_target
    b.release()


# ---------------------------------------------------------------- dense path
@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16, gg.F32])
def test_matvec_q_small(dev, rng, t):
    rows, cols = 77, 320
    w = quant(normal(rng, (rows, cols), 0.02), t)
    x = normal(rng, cols, 1.0)
    m = dev.upload_matrix(w, t, rows, cols)
    ref = R.matmulvec(np.stack([R.dequantize(w[r], t) for r in range(rows)]), x)
    assert max_rel_err(dev.matvec_q(m, x), ref) <= 1e-5
    m.release()


@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16, gg.F32])
@pytest.mark.parametrize("cols", [6400, 25600])
def test_matvec_q_chunked_ragged(dev, rng, t, cols):
    """Rows wider than one workgroup's staged x: 6400 columns (2 column chunks,
    reduced inside the launch by one reducer workgroup whose threads past row
    77 idle) and 25600 columns (5 chunks: partial sums added by k_chunk_sum);
    77 rows, so the last 8-row tile is partial."""
    rows = 77
    w = quant(normal(rng, (rows, cols), 0.02), t)
    x = normal(rng, cols, 1.0)
    m = dev.upload_matrix(w, t, rows, cols)
    ref = R.matmulvec(np.stack([R.dequantize(w[r], t) for r in range(rows)]), x)
    for _ in range(2):  # the second call finds the slots zeroed by the first
        assert max_rel_err(dev.matvec_q(m, x), ref) <= 1e-5
    m.release()


@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16])
@pytest.mark.parametrize("act", [gg.ACT_RELU, gg.ACT_GELU])
def test_ffn_dense_config1(dev, rng, t, act):
    """Dense naive path (window=0): full up matvec, the activation, full down
    matvec; ReLU (ffnReLU, forward.go:342-353) and GELU (ffnGELU, :355-366,
    the activation Falcon's loader picks, loader.go:57-58)."""
    h, ff = 4544, 18176
    up = gpu_quant((ff, h), 0.02, 31, t)
    down = gpu_quant((h, ff), 0.02, 32, t)
    x = normal(rng, h, 1.0)
    u = dev.upload_matrix(up, t, ff, h)
    d = dev.upload_matrix(down, t, h, ff)
    got = llg.ffn_dense(dev, u, d, x, act)
    ref = R.ffn_dense(up, down, t, h, ff, x, act)
    assert max_rel_err(got, ref) <= TOL
    u.release()
    d.release()


@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16])
def test_ffn_swiglu_llama7b_shape(dev, rng, t):
    """ffnSwiGLU (forward.go:368-389) at a LLaMA-7B layer's shape (d = 4096,
    F = 11008): the down rows are 11008 long, so the down matvec splits
    columns into chunks and adds their partial sums in chunk order."""
    h, ff = 4096, 11008
    gate = gpu_quant((ff, h), 0.02, 41, t)
    up = gpu_quant((ff, h), 0.02, 42, t)
    down = gpu_quant((h, ff), 0.02, 43, t)
    x = normal(rng, h, 1.0)
    g = dev.upload_matrix(gate, t, ff, h)
    u = dev.upload_matrix(up, t, ff, h)
    d = dev.upload_matrix(down, t, h, ff)
    got = llg.ffn_swiglu(dev, g, u, d, x)
    ref = R.ffn_swiglu(gate, up, down, t, h, ff, x)
    assert max_rel_err(got, ref) <= TOL
    # the device-pointer entry point gives the same bits
    xd = torch.from_numpy(x).cuda()
    od = torch.empty(h, device="cuda")
    torch.cuda.synchronize()
    dev.check(dev.lib.llg_hipd_ffn_swiglu(dev.h, g.id, u.id, d.id, ctypes.c_void_p(xd.data_ptr()),
                                          ctypes.c_void_p(od.data_ptr())), "ffn_swiglu")
    dev.sync()
    assert max_rel_err(od.cpu().numpy(), ref) <= TOL
    for m in (g, u, d):
        m.release()


@pytest.mark.parametrize("rows", [8192, 8224])
def test_ffn_swiglu_tall(dev, rng, rows):
    """gate/up with 8192+ rows take the 16-row workgroup tiles."""
    h, t = 256, gg.Q4_0
    g32, u32 = normal(rng, (rows, h), 0.05), normal(rng, (rows, h), 0.05)
    d32 = normal(rng, (h, rows), 0.05)
    gate, up, down = quant(g32, t), quant(u32, t), quant(d32, t)
    x = normal(rng, h, 1.0)
    g = dev.upload_matrix(gate, t, rows, h)
    u = dev.upload_matrix(up, t, rows, h)
    d = dev.upload_matrix(down, t, h, rows)
    assert max_rel_err(llg.ffn_swiglu(dev, g, u, d, x),
                       R.ffn_swiglu(gate, up, down, t, h, rows, x)) <= TOL
    for m in (g, u, d):
        m.release()


def test_ffn_swiglu_gate_mismatch(dev, rng):
    h, ff = 64, 96
    up = dev.upload_matrix(quant(normal(rng, (ff, h), 0.02), gg.Q4_0), gg.Q4_0, ff, h)
    gate = dev.upload_matrix(quant(normal(rng, (ff, h), 0.02), gg.Q8_0), gg.Q8_0, ff, h)
    down = dev.upload_matrix(quant(normal(rng, (h, ff), 0.02), gg.Q4_0), gg.Q4_0, h, ff)
    with pytest.raises(llg.LlgError) as e:
        llg.ffn_swiglu(dev, gate, up, down, normal(rng, h, 1.0))
    assert e.value.code == llg.LLG_E_ARG
    for m in (gate, up, down):
        m.release()


def test_ffn_dense_shape_mismatch(dev, rng):
    up = quant(normal(rng, (64, 32), 0.02), gg.Q4_0)
    m = dev.upload_matrix(up, gg.Q4_0, 64, 32)
    with pytest.raises(llg.LlgError) as e:
        llg.ffn_dense(dev, m, m, normal(rng, 32, 1.0))
    assert e.value.code == llg.LLG_E_ARG


# ---------------------------------------------------------------- window
@pytest.mark.parametrize("k", [1, 2, 5])
def test_window_tiny_closed_forms(dev, rng, k):
    h, ff = 64, 96
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    b = dev.upload_bundle(up, dn, gg.Q4_0, h, ff)
    nc = llg.NeuronCache(dev, b, k)
    ref = R.NeuronCache(max(256, ff * k // 5), h, k, ff, up, dn, gg.Q4_0)
    sets = window_sets(rng, ff, 16, 24, 0.6)
    sets.insert(5, np.array([], np.int32))  # an empty active set
    for A in sets:
        n_loaded = nc.update(A)
        ref_loaded = ref.update(A)
        assert n_loaded == ref_loaded.size
        assert nc.num_cached() == ref.num_cached()
        assert np.array_equal(nc.resident(), ref.resident())
        x = normal(rng, h, 1.0)
        got = nc.ffn_forward(x, A)
        exp = ref.ffn_forward(x, A)
        assert max_rel_err(got, exp) <= TOL
    b.release()


def test_window_config2(dev, rng):
    """64 tokens, k=5, 909 active per token with 70% carried over."""
    h, ff = 4544, 18176
    up = gpu_quant((ff, h), 0.02, 41, gg.Q4_0)
    dn = gpu_quant((ff, h), 0.02, 42, gg.Q4_0)
    b = dev.upload_bundle(up, dn, gg.Q4_0, h, ff)
    nc = llg.NeuronCache(dev, b, 5)
    ref = R.NeuronCache(ff * 5 // 5, h, 5, ff, up, dn, gg.Q4_0)
    sets = window_sets(rng, ff, 909, 64, 0.7)
    for t, A in enumerate(sets):
        assert nc.update(A) == ref.update(A).size
        assert nc.num_cached() == ref.num_cached()
        if t % 8 == 7:
            x = normal(rng, h, 1.0)
            assert max_rel_err(nc.ffn_forward(x, A), ref.ffn_forward(x, A)) <= TOL
    assert np.array_equal(nc.resident(), ref.resident())
    b.release()


def _window_steps_vs_oracle(dev, rng, t, h, ff, k, n_active, steps, carry, check_every,
                            host_update_at=()):
    """Device steps (llg_hipd_window_step: update, then the list FFN that
    copies the loaded bundles into their resident rows) against the oracle's
    NeuronCache, token by token; host updates (separate gather launch) may be
    interleaved.  Ends by running the FFN over every resident neuron with
    GELU (no zero activations, so every up and down row is read back from its
    resident row) against the oracle on the source rows."""
    up = gpu_quant((ff, h), 0.02, 51, t)
    dn = gpu_quant((ff, h), 0.02, 52, t)
    b = dev.upload_bundle(up, dn, t, h, ff)
    nc = llg.NeuronCache(dev, b, k)
    ref = R.NeuronCache(ff, h, k, ff, up, dn, t)
    sets = window_sets(rng, ff, n_active, steps, carry)
    sets.insert(3, np.array([], np.int32))  # an empty active set
    d_out = torch.empty(h, device="cuda")
    d_n = torch.empty(1, dtype=torch.int32, device="cuda")
    for i, A in enumerate(sets):
        x = normal(rng, h, 1.0)
        if i in host_update_at:
            assert nc.update(A) == ref.update(A).size
            got = nc.ffn_forward(x, A)
        else:
            d_x = torch.from_numpy(x).cuda()
            d_a = torch.from_numpy(np.ascontiguousarray(A, np.int32)).cuda() if A.size else \
                torch.zeros(1, dtype=torch.int32, device="cuda")
            d_n.fill_(A.size)
            torch.cuda.synchronize()
            nc.step_device(d_x.data_ptr(), d_a.data_ptr(), d_n.data_ptr(), d_out.data_ptr())
            dev.sync()
            got = d_out.cpu().numpy()
            ref.update(A)
        exp = ref.ffn_forward(x, A)
        if i % check_every == 0 or i in host_update_at:
            assert max_rel_err(got, exp) <= TOL, f"token {i}"
        if i % check_every == 0:
            assert np.array_equal(nc.resident(), ref.resident()), f"token {i}"
            assert nc.num_cached() == ref.num_cached()
    res = nc.resident()
    assert np.array_equal(res, ref.resident())
    x = normal(rng, h, 1.0)
    got = nc.ffn_forward(x, res, llg.gguf.ACT_GELU)
    exp = R.ffn_sparse_load(up, dn, t, h, ff, x, res, R.ACT_GELU)
    assert max_rel_err(got, exp) <= TOL
    b.release()


@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16, gg.F32])
def test_window_step_device(dev, rng, t):
    _window_steps_vs_oracle(dev, rng, t, 512, 1024, 3, 120, 20, 0.6, 1, host_update_at=(7, 8))


def test_window_step_device_config2(dev, rng):
    """64 device steps at the config-2 shape (k=5, 909 active, 70% carried)."""
    _window_steps_vs_oracle(dev, rng, gg.Q4_0, 4544, 18176, 5, 909, 64, 0.7, 8)


def test_released_bundle_stays_alive_for_its_window(dev, rng):
    """Releasing a bundle that a window reads retires the handle only; the
    window keeps working on it, and destroying the window frees it."""
    h, ff, k = 64, 96, 2
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    b = dev.upload_bundle(up, dn, gg.Q4_0, h, ff)
    nc = llg.NeuronCache(dev, b, k)
    ref = R.NeuronCache(256, h, k, ff, up, dn, gg.Q4_0)
    bid = b.id
    b.release()
    with pytest.raises(llg.LlgError) as e:  # a retired handle is unknown
        dev.check(dev.lib.llg_hip_release(dev.h, bid), "release")
    assert e.value.code == llg.LLG_E_HANDLE
    with pytest.raises(llg.LlgError) as e:
        llg.NeuronCache(dev, llg.Handle(dev, bid, "bundle"), k)
    assert e.value.code == llg.LLG_E_HANDLE
    for A in window_sets(rng, ff, 16, 8, 0.5):
        assert nc.update(A) == ref.update(A).size
        x = normal(rng, h, 1.0)
        assert max_rel_err(nc.ffn_forward(x, A), ref.ffn_forward(x, A)) <= TOL
    nc.win.release()


@pytest.mark.parametrize("act", [-1, 3])
def test_bad_activation_rejected(dev, rng, act):
    h, ff = 64, 64
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    b = dev.upload_bundle(up, dn, gg.Q4_0, h, ff)
    m_up = dev.upload_matrix(up, gg.Q4_0, ff, h)
    m_dn = dev.upload_matrix(quant(normal(rng, (h, ff), 0.02), gg.Q4_0), gg.Q4_0, h, ff)
    x = normal(rng, h, 1.0)
    for call in (lambda: llg.ffn_sparse_load(dev, b, x, np.array([1, 2], np.int32), act),
                 lambda: llg.ffn_sparse_load(dev, b, x, np.array([], np.int32), act),
                 lambda: llg.ffn_dense(dev, m_up, m_dn, x, act)):
        with pytest.raises(llg.LlgError) as e:
            call()
        assert e.value.code == llg.LLG_E_ARG
    nc = llg.NeuronCache(dev, b, 2)
    nc.update(np.array([1, 2], np.int32))
    with pytest.raises(llg.LlgError) as e:
        nc.ffn_forward(x, np.array([1, 2], np.int32), act)
    assert e.value.code == llg.LLG_E_ARG
    for hnd in (nc.win, m_up, m_dn, b):
        hnd.release()


def test_window_step_device_list_out_of_contract(dev, rng):
    """Device lists are not checked on the host; the kernels keep every access
    in bounds whatever such a list holds (indices outside [0, ff), repeats, a
    count above ff or below 0, within a buffer of ff entries).  The window is
    then discarded; a fresh window on the same bundle still matches the oracle."""
    h, ff, k = 128, 256, 2
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    b = dev.upload_bundle(up, dn, gg.Q4_0, h, ff)
    bad = llg.NeuronCache(dev, b, k)
    d_out = torch.empty(h, device="cuda")
    d_n = torch.empty(1, dtype=torch.int32, device="cuda")
    d_x = torch.from_numpy(normal(rng, h, 1.0)).cuda()
    lists = [np.array([-5, ff, ff + 100, 3, 3, 7, 2 ** 31 - 1], np.int32),
             np.repeat(np.arange(0, ff, 2, dtype=np.int32), 2)[:ff]]
    for A, count in [(lists[0], 7), (lists[1], ff + 50), (lists[1], -3), (lists[1], ff)] * 3:
        buf = np.full(ff, 1, np.int32)
        buf[:A.size] = A
        d_a = torch.from_numpy(buf).cuda()
        d_n.fill_(count)
        torch.cuda.synchronize()
        bad.step_device(d_x.data_ptr(), d_a.data_ptr(), d_n.data_ptr(), d_out.data_ptr())
        dev.sync()
        assert np.all(np.isfinite(d_out.cpu().numpy()))
    bad.win.release()
    nc = llg.NeuronCache(dev, b, k)
    ref = R.NeuronCache(ff, h, k, ff, up, dn, gg.Q4_0)
    for A in window_sets(rng, ff, 40, 6, 0.5):
        x = normal(rng, h, 1.0)
        d_a = torch.from_numpy(A).cuda()
        d_xx = torch.from_numpy(x).cuda()
        d_n.fill_(A.size)
        torch.cuda.synchronize()
        nc.step_device(d_xx.data_ptr(), d_a.data_ptr(), d_n.data_ptr(), d_out.data_ptr())
        dev.sync()
        ref.update(A)
        assert max_rel_err(d_out.cpu().numpy(), ref.ffn_forward(x, A)) <= TOL
    nc.win.release()
    b.release()


def test_size_limits(dev, rng):
    """Maximum sizes: a hidden size whose staged x overflows the sparse
    kernels' LDS, and a row too long for one workgroup when the activation
    needs it whole, are argument errors; the same long rows without an
    activation run in column chunks (Q4_0 and the flat Q8_0 layout)."""
    h, ff = 16384, 64  # 512 blocks of x: more than the sparse kernels stage
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    b = dev.upload_bundle(up, dn, gg.Q4_0, h, ff)
    with pytest.raises(llg.LlgError) as e:
        llg.ffn_sparse_load(dev, b, normal(rng, h, 1.0), np.array([1, 5], np.int32))
    assert e.value.code == llg.LLG_E_ARG
    b.release()
    cols, rows = 36864, 32  # 1152 blocks: 166 KB of staged x for a whole row
    for t in (gg.Q4_0, gg.Q8_0):
        w = quant(normal(rng, (rows, cols), 0.02), t)
        wd = quant(normal(rng, (cols, rows), 0.02), t)
        mu = dev.upload_matrix(w, t, rows, cols)
        md = dev.upload_matrix(wd, t, cols, rows)
        x = normal(rng, cols, 1.0)
        with pytest.raises(llg.LlgError) as e:
            llg.ffn_dense(dev, mu, md, x)
        assert e.value.code == llg.LLG_E_ARG
        ref = R.matmulvec(np.stack([R.dequantize(w[r], t) for r in range(rows)]), x)
        assert max_rel_err(dev.matvec_q(mu, x), ref) <= 1e-5
        mu.release()
        md.release()


def test_short_host_buffers_rejected(dev, rng):
    """A host array shorter than the shape it is passed with is an argument
    error before any copy (the C ABI would read past its end)."""
    h, ff = 64, 64
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    calls = [lambda: dev.upload_matrix(up[:-1], gg.Q4_0, ff, h),
             lambda: dev.upload_bundle(up, dn[:-1], gg.Q4_0, h, ff)]
    b = dev.upload_bundle(up, dn, gg.Q4_0, h, ff)
    m = dev.upload_matrix(up, gg.Q4_0, ff, h)
    pred = llg.Predictor(dev, normal(rng, (8, h), 0.05), normal(rng, (ff, 8), 0.05))
    nc = llg.NeuronCache(dev, b, 2)
    short = normal(rng, h - 1, 1.0)
    calls += [lambda: llg.ffn_sparse_load(dev, b, short, np.array([1], np.int32)),
              lambda: llg.ffn_predict_sparse(dev, pred, b, short, normal(rng, h, 1.0)),
              lambda: pred.predict(short),
              lambda: dev.matvec_q(m, short),
              lambda: nc.ffn_forward(short, np.array([1], np.int32))]
    for call in calls:
        with pytest.raises(llg.LlgError) as e:
            call()
        assert e.value.code == llg.LLG_E_ARG
    for hnd in (nc.win, m, b):
        hnd.release()


def test_window_rejects_duplicates(dev, rng):
    up, dn = make_sparse_layer(rng, 32, 32, gg.Q4_0)
    b = dev.upload_bundle(up, dn, gg.Q4_0, 32, 32)
    nc = llg.NeuronCache(dev, b, 2)
    with pytest.raises(llg.LlgError):
        nc.update(np.array([1, 1], np.int32))
    b.release()


# ---------------------------------------------------------------- MoE
def test_moe_route_bit_exact(dev, rng):
    """Router ids and weights equal the oracle's to the bit on identical logits
    (moe_forward.go:43-68, forward.go:463-479), ties and NaN rows included.
    With 8 experts the tie order (index order) is the reference's: Go's
    sort.Slice sorts up to 12 elements by stable insertion sort.  The 64-expert
    case checks the same index-order rule, which is the oracle's; Go's pdqsort
    order among equal scores for more than 12 experts is not restated, so there
    the tie order is parity-unpinned."""
    lg = normal(rng, (200, 8), 1.5)
    lg[0] = 0.0                          # all tied
    lg[1] = [0, 1, 1, 1, 0, 0, 0, 0]     # three-way tie for first
    lg[2, 3] = np.nan                    # every score NaN: index order kept
    lg[3, 5] = np.inf                    # inf - inf: every score NaN
    lg[4] = [-200, 0, -300, 0, -1e30, 5, 5, -5]  # underflow to exact zeros
    ids, w = dev.moe_route(lg, 2)
    for t in range(lg.shape[0]):
        rid, rw = R.moe_route(lg[t], 2)
        assert np.array_equal(ids[t], rid), t
        if t in (2, 3):
            assert np.all(np.isnan(w[t])) and np.all(np.isnan(rw))
        else:
            assert np.array_equal(w[t].view(np.uint32), rw.view(np.uint32)), t
    lg64 = normal(rng, (50, 64), 2.0)
    lg64[:, 10] = lg64[:, 40]            # ties across a wide expert set (oracle's rule)
    ids, w = dev.moe_route(lg64, 8)
    for t in range(lg64.shape[0]):
        rid, rw = R.moe_route(lg64[t], 8)
        assert np.array_equal(ids[t], rid), t
        assert np.array_equal(w[t].view(np.uint32), rw.view(np.uint32)), t


def make_moe(rng, d, eff, E, t, seed=None):
    router = normal(rng, (E, d), 0.02)
    if seed is None:
        gate = quant(normal(rng, (E * eff, d), 0.02), t)
        up = quant(normal(rng, (E * eff, d), 0.02), t)
        down = quant(normal(rng, (E * d, eff), 0.02), t)
    else:
        gate = gpu_quant((E * eff, d), 0.02, seed, t)
        up = gpu_quant((E * eff, d), 0.02, seed + 1, t)
        down = gpu_quant((E * d, eff), 0.02, seed + 2, t)
    return router, gate, up, down


def upload_moe(dev, router, gate, up, down, d, eff, E, t):
    return (dev.upload_f32(router), dev.upload_matrix(gate, t, E * eff, d),
            dev.upload_matrix(up, t, E * eff, d), dev.upload_matrix(down, t, E * d, eff))


@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16])
def test_moe_tiny(dev, rng, t):
    d, eff, E, k = 64, 96, 4, 2
    router, gate, up, down = make_moe(rng, d, eff, E, t)
    router *= 10  # spread the router so softmax is not flat
    hs = upload_moe(dev, router, gate, up, down, d, eff, E, t)
    x = normal(rng, (16, d), 1.0)
    out, ids, w = llg.moe_ffn(dev, *hs, E, k, x)
    for i in range(16):
        ro, rid, rw = R.moe_ffn(router, gate, up, down, t, d, eff, E, k, x[i])
        assert np.array_equal(ids[i], rid)
        assert max_rel_err(out[i], ro) <= TOL
    for hnd in hs:
        hnd.release()


def test_moe_decode_config3(dev, rng):
    """Mixtral-shaped layer: d=4096, 8 experts of 14336, top-2, Q4_0, one token."""
    d, eff, E, k = 4096, 14336, 8, 2
    router, gate, up, down = make_moe(rng, d, eff, E, gg.Q4_0, seed=51)
    hs = upload_moe(dev, router, gate, up, down, d, eff, E, gg.Q4_0)
    x = normal(rng, d, 1.0)
    out, ids, w = llg.moe_ffn(dev, *hs, E, k, x)
    ro, rid, rw = R.moe_ffn(router, gate, up, down, gg.Q4_0, d, eff, E, k, x)
    assert np.array_equal(ids, rid)
    assert max_rel_err(out, ro) <= TOL
    for hnd in hs:
        hnd.release()


@pytest.mark.parametrize("d,eff,E,k,n_tok", [(64, 96, 64, 8, 3),      # the most experts and slots
                                           (64, 96, 5, 1, 4),       # top-1
                                           (256, 128, 16, 4, 40)])  # the GEMM path, k = 4
def test_moe_expert_and_slot_limits(dev, rng, d, eff, E, k, n_tok):
    """Routing and combine at the limits of the expert count (64) and slots
    per token (8), top-1, and a 4-slot batch on the grouped GEMM."""
    router, gate, up, down = make_moe(rng, d, eff, E, gg.Q4_0)
    router *= 10
    hs = upload_moe(dev, router, gate, up, down, d, eff, E, gg.Q4_0)
    x = normal(rng, (n_tok, d), 1.0)
    out, ids, w = llg.moe_ffn(dev, *hs, E, k, x)
    assert ids.shape == (n_tok, k)
    for i in range(n_tok):
        ro, rid, rw = R.moe_ffn(router, gate, up, down, gg.Q4_0, d, eff, E, k, x[i])
        assert np.array_equal(ids[i], rid), i
        assert np.allclose(w[i], rw, rtol=1e-5, atol=1e-7), i
        assert max_rel_err(out[i], ro) <= TOL, i
    for hnd in hs:
        hnd.release()


@pytest.mark.parametrize("n_tok", [16, 77, 200])
def test_moe_prefill_gemm(dev, rng, n_tok):
    """Batches of >= 16 Q4_0 tokens take the grouped MFMA GEMM path (f16
    operands, fp32 accumulation); every token is checked against the oracle.
    The router is biased so one expert gets no token and one gets most of
    them all (empty groups, ragged 64-row tiles, several tiles per expert)."""
    d, eff, E, k = 256, 384, 8, 2
    router, gate, up, down = make_moe(rng, d, eff, E, gg.Q4_0)
    router *= 10
    hs = upload_moe(dev, router, gate, up, down, d, eff, E, gg.Q4_0)
    x = normal(rng, (n_tok, d), 1.0)
    x += 0.5 * router[2] / np.linalg.norm(router[2]) * np.sqrt(d)  # favour expert 2
    x -= 2.0 * router[5] / np.linalg.norm(router[5]) * np.sqrt(d)  # starve expert 5
    out, ids, w = llg.moe_ffn(dev, *hs, E, k, x)
    counts = np.bincount(ids.ravel(), minlength=E)
    assert counts[5] == 0 and counts[2] == n_tok, counts
    for i in range(n_tok):
        ro, rid, rw = R.moe_ffn(router, gate, up, down, gg.Q4_0, d, eff, E, k, x[i])
        assert np.array_equal(ids[i], rid), i
        # logits from x are summed in another order than the oracle's, so the
        # weights agree to rounding (bit-exact routing on equal logits is
        # test_moe_route_bit_exact)
        assert np.allclose(w[i], rw, rtol=1e-5, atol=1e-7), i
        assert max_rel_err(out[i], ro) <= TOL, i
    for hnd in hs:
        hnd.release()


def test_moe_prefill_config3(dev, rng):
    """Mixtral-shaped layer, 512-token prefill on the grouped GEMM path: 12
    sampled tokens against the oracle, and every token against the one-token
    decode path of the same library (same ids and weights bit for bit)."""
    d, eff, E, k, n_tok = 4096, 14336, 8, 2, 512
    router, gate, up, down = make_moe(rng, d, eff, E, gg.Q4_0, seed=61)
    hs = upload_moe(dev, router, gate, up, down, d, eff, E, gg.Q4_0)
    x = normal(rng, (n_tok, d), 1.0)
    out, ids, w = llg.moe_ffn(dev, *hs, E, k, x)
    assert np.all(np.isfinite(out))
    for i in np.linspace(0, n_tok - 1, 12).astype(int):
        ro, rid, rw = R.moe_ffn(router, gate, up, down, gg.Q4_0, d, eff, E, k, x[i])
        assert np.array_equal(ids[i], rid), i
        assert max_rel_err(out[i], ro) <= TOL, i
    for i in range(0, n_tok, 37):
        o1, id1, w1 = llg.moe_ffn(dev, *hs, E, k, x[i])
        assert np.array_equal(ids[i], id1) and np.array_equal(w[i], w1), i
        assert max_rel_err(out[i], o1) <= TOL, i
    for hnd in hs:
        hnd.release()


def test_moe_invalid_hparams(dev, rng):
    d, eff, E = 64, 96, 4
    router, gate, up, down = make_moe(rng, d, eff, E, gg.Q4_0)
    hs = upload_moe(dev, router, gate, up, down, d, eff, E, gg.Q4_0)
    with pytest.raises(llg.LlgError) as e:
        llg.moe_ffn(dev, *hs, E, 0, normal(rng, d, 1.0))
    assert e.value.code == llg.LLG_E_HPARAM


# ---------------------------------------------------------------- Metal parity
def test_metal_parity_matvec_rmsnorm(dev, rng):
    for rows, cols in [(1, 1), (7, 33), (300, 4544)]:
        w, x = normal(rng, (rows, cols), 0.1), normal(rng, cols, 1.0)
        assert max_rel_err(dev.mat_mul_vec(w, rows, cols, x), R.matmulvec(w, x)) <= 1e-5
    x, wt = normal(rng, 4544, 1.0), normal(rng, 4544, 1.0)
    assert max_rel_err(dev.rms_norm(x, wt, 1e-5), R.rmsnorm(x, wt, 1e-5)) <= 1e-5
    with pytest.raises(llg.LlgError):
        dev.mat_mul_vec(w, rows, cols + 1, x)


def test_bad_handles_and_types(dev, rng):
    with pytest.raises(llg.LlgError) as e:
        dev.upload_matrix(np.zeros(36, np.uint8), 12, 1, 64)  # Q4_K is out of scope
    assert e.value.code == llg.LLG_E_TYPE
    with pytest.raises(llg.LlgError) as e:
        dev.upload_matrix(np.zeros(36, np.uint8), gg.Q4_0, 1, 48)
    assert e.value.code == llg.LLG_E_ALIGN
    fake = llg.Handle(dev, 999999, "bundle")
    with pytest.raises(llg.LlgError) as e:
        llg.ffn_sparse_load(dev, fake, np.zeros(64, np.float32), np.array([0], np.int32))
    assert e.value.code == llg.LLG_E_HANDLE


# ---------------------------------------------------------------- Falcon decode
FALCON_GPU = dict(n_layers=2, hidden=256, n_heads=4, n_kv=1, head_dim=64, ff=512, vocab=300,
                  max_seq=32, rank=16, rope_base=10000.0, eps=1e-5)


def _top2_gap(v):
    s = np.sort(v)
    return float(s[-1] - s[-2])


@pytest.mark.parametrize("n_kv,t", [(1, gg.Q4_0), (2, gg.Q4_0), (1, gg.Q8_0)])
def test_falcon_forward(dev, rng, n_kv, t):
    """ForwardFlash token by token against the oracle: logits within the FFN
    bar, per-layer active counts exact (thresholds sit in wide logit gaps),
    greedy token equal wherever the top-2 logit gap is clear.  Q8_0 weights
    take the flat matvec layout under the LayerNorm prologue."""
    d = dict(FALCON_GPU, n_kv=n_kv)
    w = make_falcon(rng, d, t)
    toks = rng.integers(0, d["vocab"], 10)
    _, nact, thr = ref_falcon_f64(w, d, toks, t=t)
    ref = R.Falcon(d, w, thr, t)
    m = llg.FalconModel(dev, d, w, thr, t=t)
    for s, tk in enumerate(toks):
        lg, nxt, na = m.forward(int(tk), s)
        rl, rn = ref.forward(int(tk), s)
        assert np.array_equal(na, rn) and np.array_equal(na, nact[s]), (s, na, rn)
        assert max_rel_err(lg, rl) <= TOL, s
        if _top2_gap(rl) > 1e-3 * np.max(np.abs(rl)):
            assert nxt == R.argmax(rl), s
    with pytest.raises(llg.LlgError) as e:
        m.forward(0, d["max_seq"])
    assert e.value.code == llg.LLG_E_RANGE
    with pytest.raises(llg.LlgError) as e:
        m.forward(d["vocab"], 0)
    assert e.value.code == llg.LLG_E_RANGE
    m.release()


def test_falcon_wide_hidden_layernorm_reduction(dev, rng):
    """hidden 8224 (257 blocks) is above what the QKV LayerNorm merges from the
    residual's block statistics, so the prologue forms the mean and variance
    with workgroup reductions (and the LM head runs in column chunks);
    against the oracle at every position (forward.go:258-301, ops.go:138-165)."""
    d = dict(FALCON_GPU, hidden=8224, n_heads=4, n_kv=1, head_dim=64, ff=512, vocab=256,
             rank=16, n_layers=1, max_seq=16)
    w = make_falcon(rng, d, gg.Q4_0)
    toks = rng.integers(0, d["vocab"], 6)
    _, nact, thr = ref_falcon_f64(w, d, toks)
    ref = R.Falcon(d, w, thr)
    m = llg.FalconModel(dev, d, w, thr)
    for s, tk in enumerate(toks):
        lg, nxt, na = m.forward(int(tk), s)
        rl, rn = ref.forward(int(tk), s)
        assert np.array_equal(na, rn) and np.array_equal(na, nact[s]), (s, na, rn)
        assert max_rel_err(lg, rl) <= TOL, s
        if _top2_gap(rl) > 1e-3 * np.max(np.abs(rl)):
            assert nxt == R.argmax(rl), s
    m.release()


def test_falcon_wide_heads_chunked_wo(dev, rng):
    """48 query heads of 128 over 4 KV heads: Wo's rows are 6144 wide, so its
    matvec runs in column chunks whose partial sums the model adds in order;
    against the oracle at every position."""
    d = dict(FALCON_GPU, hidden=512, n_heads=48, n_kv=4, head_dim=128, ff=1024, max_seq=16)
    w = make_falcon(rng, d, std=0.02)
    toks = rng.integers(0, d["vocab"], 8)
    _, nact, thr = ref_falcon_f64(w, d, toks)
    ref = R.Falcon(d, w, thr)
    m = llg.FalconModel(dev, d, w, thr)
    for s, tk in enumerate(toks):
        lg, _, na = m.forward(int(tk), s)
        rl, rn = ref.forward(int(tk), s)
        assert np.array_equal(na, rn), (s, na, rn)
        assert max_rel_err(lg, rl) <= TOL, s
    m.release()


@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0])
def test_falcon_balanced_matvecs_and_fold(dev, rng, t):
    """Hidden 2048 with 32 heads of 64: QKV (2176 rows) and Wo (2048 rows) take
    the one-workgroup-per-CU matvec, the LayerNorm prologue with two float4
    groups per thread, and Wo the predictor fold (P = WUp . Wo at load, the
    hidden partials computed beside Wo . attn); against the oracle's
    WUp . (Wo . attn) at every position, Q4_0 and Q8_0."""
    d = dict(FALCON_GPU, hidden=2048, n_heads=32, n_kv=2, head_dim=64, ff=4096, rank=32,
             max_seq=16)
    w = make_falcon(rng, d, t, std=0.02)
    toks = rng.integers(0, d["vocab"], 12)
    _, nact, thr = ref_falcon_f64(w, d, toks, t=t)
    ref = R.Falcon(d, w, thr, t)
    m = llg.FalconModel(dev, d, w, thr, t=t)
    for s, tk in enumerate(toks):
        lg, _, na = m.forward(int(tk), s)
        rl, rn = ref.forward(int(tk), s)
        assert np.array_equal(na, rn) and np.array_equal(na, nact[s]), (s, na, rn)
        assert max_rel_err(lg, rl) <= TOL, s
    m.release()


def test_released_weights_stay_alive_for_their_model(dev, rng):
    """Every weight handle released before the model: the model still reads
    them (the handles are retired, the memory is kept until the model goes)."""
    d = dict(FALCON_GPU)
    w = make_falcon(rng, d)
    toks = rng.integers(0, d["vocab"], 4)
    _, _, thr = ref_falcon_f64(w, d, toks)
    ref = R.Falcon(d, w, thr)
    m = llg.FalconModel(dev, d, w, thr)
    for hnd in m._h:
        hnd.release()
    m._h = []
    for s, tk in enumerate(toks):
        lg, _, _ = m.forward(int(tk), s)
        rl, _ = ref.forward(int(tk), s)
        assert max_rel_err(lg, rl) <= TOL, s
    m.release()


def test_falcon_device_greedy_loop(dev, rng):
    """Prompt + greedy decode chained on the device (the next token never goes
    through the host) against the oracle's greedy continuation."""
    d = dict(FALCON_GPU)
    w = make_falcon(rng, d)
    prompt = rng.integers(0, d["vocab"], 6)
    n_gen = 8
    # thresholds from the prompt plus a provisional continuation
    _, _, thr = ref_falcon_f64(w, d, prompt)
    ref = R.Falcon(d, w, thr)
    seq = list(prompt)
    for s in range(len(prompt) + n_gen - 1):
        lg, _ = ref.forward(int(seq[s]), s)
        if s >= len(prompt) - 1:
            seq.append(R.argmax(lg))
    m = llg.FalconModel(dev, d, w, thr)
    toks = torch.tensor(np.array(prompt, np.int32), device="cuda")
    gen = torch.zeros(n_gen + 1, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    for s in range(len(prompt)):
        out = gen.data_ptr() if s == len(prompt) - 1 else gen.data_ptr() + 4 * n_gen
        m.step_device(toks.data_ptr() + 4 * s, s, out)
    for i in range(n_gen - 1):
        m.step_device(gen.data_ptr() + 4 * i, len(prompt) + i, gen.data_ptr() + 4 * (i + 1))
    dev.sync()
    got = gen[:n_gen].cpu().numpy()
    assert np.array_equal(got, np.array(seq[len(prompt):len(prompt) + n_gen])), (got, seq)
    m.release()
