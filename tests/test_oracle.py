"""Pins the CPU oracle (oracle/refcpu.c) without running the reference.

The reference is Go and no Go toolchain exists here, and the reference has no
tests or golden vectors of its own, so each oracle function is pinned by a
check that a plausible restatement mistake would fail:

  function (reference)                     pinned by
  f16_to_f32 (dtype.go:417-443)            all 63 488 non-NaN halves vs numpy's IEEE
                                           conversion; hand-computed specials incl. NaN
                                           canonicalisation to sign|0x7FC00000
  byte_size (types.go:90-102)              closed form + misaligned/unknown errors
  Dequantize Q4_0 (dtype.go:62-82)         hand-built block: byte i = (2i+1)%16<<4|(2i)%16
                                           must decode to the ramp (j % 16) - 8 (catches
                                           ggml's j/j+16 order); scale and sign checks
  Dequantize Q8_0/F16/F32                  hand-built blocks / byte reinterpretation
  MatMulVec (ops.go:39-60)                 small-integer inputs summed exactly (bit-equal
                                           to int64 numpy; a transposed operand fails)
  ReLU/SiLU/GELU (ops.go:168-189)          specials (NaN, -0.0) and float64 formulas
  softmax (forward.go:463-479)             float64 softmax, shift invariance, sum to 1
  select / Predict (predictor.go:51-83)    brute force with strict '>' at ties; float64
                                           logits
  ReadRowsParallel addressing              rows equal slices of the full dequantized tensor
  ReadRowsParallel from a file             a GGUF file written here, read back by 1, 3 and
  (storage.go:246-319)                     32 threads: bit-equal to the in-memory rows;
                                           out-of-range row, missing file and truncated
                                           tensor errors
  ffnSparseLoad (ffn_flash.go:254-299)     float64 brute force; empty list; zero-skip;
                                           all-active sparse vs dense on F32 weights
  NeuronCache (window.go)                  closed forms toLoad_t = A_t minus the previous k
                                           sets, resident_t = union of the last k sets, on
                                           tiny ff and k in {1,2,5}; FFNForward bit-equal
                                           to ffnSparseLoad
  moeFFN router (moe_forward.go:42-68)     brute-force top-k over float64 softmax; ties go
                                           to the lower index; weights sum to 1
  moeFFN experts (moe_forward.go:83-150)   float64 brute force at d=64, eff=96, E=4, k=2
  RMSNorm / LayerNorm (ops.go:114-165)     float64 formulas
  ForwardFlash (ffn_flash.go:115-185)      float64 brute force over 7 tokens (MQA/GQA/MHA),
                                           no-RoPE variant, closed form at position 0
  row threads of the oracle                1, 5 and 16 threads bit-equal (MatMulVec, the
                                           sparse FFN, the attention heads)
  ForwardFlash with rows from a file       bit-equal to the in-memory rows from any
  (ffn_flash.go:262-270)                   position on; unreadable rows are an error

Functions whose last-ulp behaviour only running Go could pin (sequential dot
rounding under Go's FMA rules, math.Exp ulps, sort.Slice tie order for n > 12)
are covered by the tolerances and same-logits protocols noted in the tests.
"""
import math

import numpy as np
import pytest

import llg.gguf as gg
from oracle import refcpu as R
from tests.helpers import (act_f64, deq, make_falcon, make_sparse_layer, max_rel_err, normal,
                           quant, ref_falcon_f64, ref_sparse_f64, window_sets)


# ---------------------------------------------------------------- f16 -> f32
def test_f16_exhaustive_vs_ieee():
    lib = R.lib()
    hs = np.arange(65536, dtype=np.uint32)
    exp = (hs >> 10) & 0x1F
    mant = hs & 0x3FF
    non_nan = ~((exp == 31) & (mant != 0))
    ref = hs[non_nan].astype(np.uint16).view(np.float16).astype(np.float32).view(np.uint32)
    got = np.array([lib.refcpu_f16_to_f32(int(h)) for h in hs[non_nan]], np.float32).view(np.uint32)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("h,bits", [
    (0x0000, 0x00000000), (0x8000, 0x80000000),           # +-0
    (0x0001, 0x33800000),                                   # 2^-24, smallest subnormal
    (0x03FF, 0x387FC000),                                   # largest subnormal
    (0x3C00, 0x3F800000), (0xC000, 0xC0000000),             # 1.0, -2.0
    (0x7BFF, 0x477FE000),                                   # 65504
    (0x7C00, 0x7F800000), (0xFC00, 0xFF800000),             # +-Inf
    (0x7E01, 0x7FC00000), (0x7C01, 0x7FC00000),             # NaN -> canonical
    (0xFE00, 0xFFC00000),                                   # -NaN keeps the sign
])
def test_f16_specials(h, bits):
    assert R.f16_to_f32_bits(h) == bits


# ---------------------------------------------------------------- ByteSize
def test_byte_size():
    assert R.byte_size(R.Q4_0, 4544) == 142 * 18 == 2556
    assert R.byte_size(R.Q8_0, 4544) == 142 * 34 == 4828
    assert R.byte_size(R.F16, 4544) == 9088
    assert R.byte_size(R.F32, 7) == 28
    assert R.byte_size(R.Q4_0, 33) == -1  # not a multiple of the block size
    assert R.byte_size(99, 32) == -1      # unknown type
    for t in (R.F32, R.F16, R.Q4_0, R.Q8_0):
        assert R.byte_size(t, 4096) == gg.byte_size(t, 4096)
    with pytest.raises(ValueError):
        gg.byte_size(gg.Q4_0, 33)


# ---------------------------------------------------------------- dequant KATs
def q4_ramp_block(dbits: int) -> bytes:
    qs = bytes((((2 * i + 1) % 16) << 4) | ((2 * i) % 16) for i in range(16))
    return bytes([dbits & 0xFF, dbits >> 8]) + qs


def test_q4_0_interleaved_ramp():
    out = R.dequantize(np.frombuffer(q4_ramp_block(0x3C00), np.uint8), R.Q4_0)
    assert out.tolist() == [float((j % 16) - 8) for j in range(32)]
    # ggml's own layout would put low nibbles at 0..15 and high nibbles at 16..31
    ggml_order = [float(((2 * j) % 16) - 8) for j in range(16)] + \
                 [float(((2 * j + 1) % 16) - 8) for j in range(16)]
    assert out.tolist() != ggml_order


def test_q4_0_scale_and_sign():
    out = R.dequantize(np.frombuffer(q4_ramp_block(0xB800), np.uint8), R.Q4_0)  # d = -0.5
    assert out.tolist() == [((j % 16) - 8) * -0.5 for j in range(32)]
    sub = R.dequantize(np.frombuffer(q4_ramp_block(0x0001), np.uint8), R.Q4_0)  # d = 2^-24
    assert sub.tolist() == [((j % 16) - 8) * 2.0 ** -24 for j in range(32)]


def test_q8_0_block():
    qs = np.arange(-16, 16, dtype=np.int8)
    blk = np.concatenate([np.array([0x00, 0x40], np.uint8), qs.view(np.uint8)])  # d = 2.0
    out = R.dequantize(blk, R.Q8_0)
    assert out.tolist() == [2.0 * q for q in range(-16, 16)]
    qs2 = np.array([-128, 127] * 16, np.int8)
    blk2 = np.concatenate([np.array([0x00, 0x3C], np.uint8), qs2.view(np.uint8)])
    assert R.dequantize(blk2, R.Q8_0).tolist() == [-128.0, 127.0] * 16


def test_f16_f32_dequant_bytes():
    v = np.array([1.5, -2.25, 65504.0, 6.1e-5], np.float16)
    assert np.array_equal(R.dequantize(v.view(np.uint8), R.F16), v.astype(np.float32))
    w = np.array([1.0, -3.5, 1e-30], np.float32)
    assert np.array_equal(R.dequantize(w.view(np.uint8), R.F32), w)


def test_dequant_bad_length():
    with pytest.raises(ValueError):
        R.dequantize(np.zeros(17, np.uint8), R.Q4_0)


@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16, gg.F32])
def test_quantizer_roundtrip(rng, t):
    """The ggml-method quantizers, decoded by the oracle: error bounded by half
    a quantisation step, and the vectorised torch decoder agrees bit-exactly."""
    x = normal(rng, (8, 256), 0.02)
    raw = quant(x, t)
    assert raw.shape == (8, gg.byte_size(t, 256))
    dq = R.dequantize(raw, t).reshape(8, 256)
    assert np.array_equal(dq.view(np.uint32), deq(raw, t, 256).view(np.uint32))
    err = np.abs(dq - x).reshape(8, -1, 32)
    amax = np.abs(x).reshape(8, -1, 32).max(axis=2, keepdims=True)
    # Q4_0 spans [-8d, 7d] with |d| = amax/8: values near -max lose up to one step.
    # The scale is stored as f16 (relative error 2^-11), which adds |q| * d * 2^-11.
    bound = {gg.Q4_0: amax / 8 * 1.01 + 1e-6, gg.Q8_0: amax / 127 * 0.57 + 1e-6,
             gg.F16: np.abs(x).reshape(8, -1, 32) * 2 ** -11 + 2 ** -25, gg.F32: 0.0}[t]
    assert np.all(err <= bound)


# ---------------------------------------------------------------- MatMulVec
def test_matmulvec_exact_integers(rng):
    w = rng.integers(-4, 5, (37, 53)).astype(np.float32)
    x = rng.integers(-4, 5, 53).astype(np.float32)
    y = R.matmulvec(w, x)
    assert np.array_equal(y, (w.astype(np.int64) @ x.astype(np.int64)).astype(np.float32))
    assert not np.array_equal(y[:37], (w.T[:37, :37].astype(np.int64) @ x[:37]).astype(np.float32))


def test_matmulvec_f64(rng):
    w, x = normal(rng, (64, 300), 1.0), normal(rng, 300, 1.0)
    assert np.max(np.abs(R.matmulvec(w, x) - w.astype(np.float64) @ x)) < 1e-4


# ---------------------------------------------------------------- activations
def test_relu_specials():
    v = np.array([-1.0, -0.0, 0.0, 2.5, np.nan, -np.inf], np.float32)
    out = R.activation(R.ACT_RELU, v)
    assert out[0] == 0.0 and out[3] == 2.5 and np.isnan(out[4]) and out[5] == 0.0
    assert np.signbit(out[1])  # -0.0 is not < 0, so it passes through (ops.go:170)


@pytest.mark.parametrize("act", [R.ACT_SILU, R.ACT_GELU])
def test_silu_gelu_f64(rng, act):
    from tests.helpers import act_f64
    v = normal(rng, 1000, 3.0)
    out = R.activation(act, v)
    ref = act_f64(act, v.astype(np.float64))
    # absolute floor: GELU's float32 `1 + tanh(..)` cancels to 0 for large negative v
    assert np.all(np.abs(out - ref) <= 1e-5 * np.abs(ref) + 1e-6)


# ---------------------------------------------------------------- softmax / norms
def test_softmax(rng):
    v = normal(rng, 8, 2.0)
    p = R.softmax(v)
    e = np.exp(v.astype(np.float64) - v.max())
    assert np.max(np.abs(p - e / e.sum())) < 1e-6
    assert abs(float(p.astype(np.float64).sum()) - 1.0) < 1e-6
    assert np.max(np.abs(R.softmax(v + 10.0) - p)) < 1e-6


def test_norms(rng):
    x, w, b = normal(rng, 300, 1.0), normal(rng, 300, 1.0), normal(rng, 300, 1.0)
    xd = x.astype(np.float64)
    rms = xd / math.sqrt((xd ** 2).mean() + 1e-5) * w
    assert np.max(np.abs(R.rmsnorm(x, w, 1e-5) - rms)) < 1e-5
    ln = (xd - xd.mean()) / math.sqrt(xd.var() + 1e-5) * w + b
    assert np.max(np.abs(R.layernorm(x, w, b, 1e-5) - ln)) < 1e-5


# ---------------------------------------------------------------- predictor
def test_select_strict_and_ascending():
    lg = np.array([0.5, 1.0, 0.5, 2.0, -1.0, 0.5000001], np.float32)
    assert R.select(lg, 0.5).tolist() == [1, 3, 5]  # 0.5 itself is not > 0.5
    assert R.select(lg, 10.0).tolist() == []


def test_predict_f64(rng):
    h, rank, ff = 64, 16, 256
    wup, wout = normal(rng, (rank, h), 0.05), normal(rng, (ff, rank), 0.05)
    bias, a = normal(rng, ff, 0.01), normal(rng, h, 1.0)
    act, lg = R.predict(wup, wout, bias, a, 0.0)
    hid = np.maximum(wup.astype(np.float64) @ a, 0.0)
    ref = wout.astype(np.float64) @ hid + bias
    assert np.max(np.abs(lg - ref)) < 1e-5
    assert act.tolist() == R.select(lg, 0.0).tolist()
    assert act.tolist() == [i for i in range(ff) if lg[i] > 0.0]
    act_nb, lg_nb = R.predict(wup, wout, None, a, 0.0)
    assert np.max(np.abs(lg_nb - (ref - bias))) < 1e-5


# ---------------------------------------------------------------- row gather
def test_read_rows_addressing(rng):
    h, ff = 64, 40
    raw = quant(normal(rng, (ff, h), 0.02), gg.Q4_0)
    full = R.dequantize(raw, R.Q4_0).reshape(ff, h)
    rows = np.array([39, 0, 7, 7, 12], np.int32)
    assert np.array_equal(R.read_rows(raw, R.Q4_0, h, ff, rows), full[rows])
    with pytest.raises(IndexError):
        R.read_rows(raw, R.Q4_0, h, ff, np.array([40], np.int32))


def _layer_file(tmp_path, up, dn, t, h, ff):
    """A GGUF file holding ffn_up and the transposed ffn_down ([h, F] dims,
    F rows of h) after a small leading tensor, so the offsets are not 0."""
    from llg import gguf_file as GF

    path = tmp_path / "layer.gguf"
    pad = np.zeros(7 * 4, np.uint8)
    GF.write_gguf(path, [("general.architecture", GF.T_STRING, "falcon")],
                  [("pad", [7], gg.F32, pad), ("blk.0.ffn_up.weight", [h, ff], t, up),
                   ("blk.0.ffn_down_t.weight", [h, ff], t, dn)])
    f = GF.open_gguf(path)
    return path, f.by_name["blk.0.ffn_up.weight"].offset, f.by_name["blk.0.ffn_down_t.weight"].offset


@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16])
def test_read_rows_file_matches_memory(rng, tmp_path, t):
    h, ff = 96, 70
    up, dn = make_sparse_layer(rng, h, ff, t)
    path, off_up, off_dn = _layer_file(tmp_path, up, dn, t, h, ff)
    rows = np.array([69, 0, 7, 7, 12, 33, 68], np.int32)
    for n in (1, 3, 32):
        assert np.array_equal(R.read_rows_file(path, off_up, t, h, ff, rows, n),
                              R.read_rows(up, t, h, ff, rows))
        assert np.array_equal(R.read_rows_file(path, off_dn, t, h, ff, rows, n),
                              R.read_rows(dn, t, h, ff, rows))
    with pytest.raises(IndexError):
        R.read_rows_file(path, off_up, t, h, ff, np.array([3, 70], np.int32))
    with pytest.raises(OSError, match="open failed"):
        R.read_rows_file(tmp_path / "missing.gguf", off_up, t, h, ff, rows)
    with pytest.raises(OSError, match="short read"):  # the last row runs past the end
        R.read_rows_file(path, off_dn + gg.byte_size(t, h), t, h, ff, np.array([69], np.int32))


def test_ffn_sparse_load_file_matches_memory(rng, tmp_path):
    h, ff = 128, 300
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    path, off_up, off_dn = _layer_file(tmp_path, up, dn, gg.Q4_0, h, ff)
    x = normal(rng, h, 1.0)
    active = np.sort(rng.choice(ff, 45, replace=False)).astype(np.int32)
    ref = R.ffn_sparse_load(up, dn, gg.Q4_0, h, ff, x, active)
    assert np.array_equal(
        R.ffn_sparse_load_file(path, off_up, off_dn, gg.Q4_0, h, ff, x, active), ref)
    assert np.all(R.ffn_sparse_load_file(path, off_up, off_dn, gg.Q4_0, h, ff, x,
                                         np.array([], np.int32)) == 0)
    # rows come from the file: the in-memory arrays are not consulted
    assert not np.array_equal(
        R.ffn_sparse_load_file(path, off_dn, off_up, gg.Q4_0, h, ff, x, active), ref)


# ---------------------------------------------------------------- sparse FFN
@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16])
def test_ffn_sparse_f64(rng, t):
    h, ff = 128, 512
    up, dn = make_sparse_layer(rng, h, ff, t)
    x = normal(rng, h, 1.0)
    active = np.sort(rng.choice(ff, 40, replace=False)).astype(np.int32)
    out = R.ffn_sparse_load(up, dn, t, h, ff, x, active)
    ref = ref_sparse_f64(up, dn, t, h, x, active)
    assert np.max(np.abs(out - ref)) <= 1e-5 * max(1.0, np.abs(ref).max())


def test_ffn_sparse_empty_and_zero_skip(rng):
    h, ff = 64, 64
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    x = normal(rng, h, 1.0)
    assert np.all(R.ffn_sparse_load(up, dn, gg.Q4_0, h, ff, x, np.array([], np.int32)) == 0)
    # a neuron whose activation is exactly zero contributes nothing, even a NaN row
    dn_nan = dn.copy()
    dn_nan[5, 0:2] = [0x00, 0x7E]  # scale of block 0 = NaN
    up_zero = up.copy()
    up_zero[5, :] = 0  # u_5 = 0 -> the row is skipped (ffn_flash.go:290)
    out = R.ffn_sparse_load(up_zero, dn_nan, gg.Q4_0, h, ff, x, np.array([3, 5], np.int32))
    assert np.all(np.isfinite(out))


def test_all_active_sparse_equals_dense_f32(rng):
    h, ff = 64, 96
    up = normal(rng, (ff, h), 0.02)
    down = normal(rng, (h, ff), 0.02)  # standard layout for the dense path
    x = normal(rng, h, 1.0)
    dense = R.ffn_dense(quant(up, gg.F32), quant(down, gg.F32), gg.F32, h, ff, x)
    sparse = R.ffn_sparse_load(quant(up, gg.F32), quant(np.ascontiguousarray(down.T), gg.F32),
                               gg.F32, h, ff, x, np.arange(ff, dtype=np.int32))
    assert np.max(np.abs(dense - sparse)) < 1e-6


@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16])
def test_ffn_swiglu_f64(rng, t):
    """ffnSwiGLU (forward.go:368-389) against float64 over the exactly
    dequantized weights; exchanging gate and up must change the result (so a
    swapped operand cannot pass)."""
    h, ff = 96, 160
    g, u, d = (quant(normal(rng, (ff, h), 0.1), t), quant(normal(rng, (ff, h), 0.1), t),
               quant(normal(rng, (h, ff), 0.1), t))
    x = normal(rng, h, 1.0)
    out = R.ffn_swiglu(g, u, d, t, h, ff, x)
    xd = x.astype(np.float64)
    gv, uv = deq(g, t, h).astype(np.float64) @ xd, deq(u, t, h).astype(np.float64) @ xd
    ref = deq(d, t, ff).astype(np.float64) @ (act_f64(gg.ACT_SILU, gv) * uv)
    assert max_rel_err(out, ref) < 1e-5
    swapped = R.ffn_swiglu(u, g, d, t, h, ff, x)
    assert max_rel_err(swapped, ref) > 1e-2


# ---------------------------------------------------------------- window
@pytest.mark.parametrize("k", [1, 2, 5])
def test_neuron_cache_closed_forms(rng, k):
    h, ff = 32, 64
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    nc = R.NeuronCache(256, h, k, ff, up, dn, gg.Q4_0)
    sets = window_sets(rng, ff, 12, 20, 0.5)
    for t, A in enumerate(sets):
        prev = set().union(*[set(s.tolist()) for s in sets[max(0, t - k):t]])
        loaded = nc.update(A)
        assert loaded.tolist() == [n for n in A.tolist() if n not in prev]
        res = set().union(*[set(s.tolist()) for s in sets[max(0, t - k + 1):t + 1]])
        assert nc.resident().tolist() == sorted(res)
        assert nc.num_cached() == len(res)
        x = normal(rng, h, 1.0)
        got = nc.ffn_forward(x, A)
        ref = R.ffn_sparse_load(up, dn, gg.Q4_0, h, ff, x, A)
        assert np.array_equal(got, ref)


def test_neuron_cache_from_file(rng, tmp_path):
    h, ff, k = 64, 96, 3
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    path, off_up, off_dn = _layer_file(tmp_path, up, dn, gg.Q4_0, h, ff)
    mem = R.NeuronCache(ff, h, k, ff, up, dn, gg.Q4_0)
    fil = R.NeuronCache.from_file(ff, h, k, ff, path, off_up, off_dn, gg.Q4_0)
    for A in window_sets(rng, ff, 10, 24, 0.6):
        assert np.array_equal(fil.update(A), mem.update(A))
        assert fil.num_cached() == mem.num_cached()
        x = normal(rng, h, 1.0)
        assert np.array_equal(fil.ffn_forward(x, A), mem.ffn_forward(x, A))


def test_neuron_cache_grows(rng):
    h, ff = 32, 64
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    nc = R.NeuronCache(4, h, 3, ff, up, dn, gg.Q4_0)  # capacity 4 forces the 10% growth path
    A = np.arange(0, 40, 2, dtype=np.int32)
    nc.update(A)
    x = normal(rng, h, 1.0)
    assert np.array_equal(nc.ffn_forward(x, A), R.ffn_sparse_load(up, dn, gg.Q4_0, h, ff, x, A))


# ---------------------------------------------------------------- MoE
def test_moe_route_brute_force(rng):
    for _ in range(50):
        lg = normal(rng, 8, 1.5)
        ids, w = R.moe_route(lg, 2)
        p = np.exp(lg.astype(np.float64) - lg.max())
        p /= p.sum()
        order = sorted(range(8), key=lambda i: (-p[i], i))
        assert ids.tolist() == order[:2]
        assert abs(float(w.astype(np.float64).sum()) - 1.0) < 1e-6
        assert np.max(np.abs(w - p[order[:2]] / p[order[:2]].sum())) < 1e-6


def test_moe_route_ties_lower_index():
    ids, w = R.moe_route(np.array([0.0, 1.0, 1.0, 1.0, 0.0], np.float32), 2)
    assert ids.tolist() == [1, 2] and w.tolist() == [0.5, 0.5]
    ids, _ = R.moe_route(np.zeros(8, np.float32), 3)
    assert ids.tolist() == [0, 1, 2]


def test_moe_ffn_f64(rng):
    d, eff, E, k = 64, 96, 4, 2
    router = normal(rng, (E, d), 0.2)
    gate = normal(rng, (E * eff, d), 0.05)
    up = normal(rng, (E * eff, d), 0.05)
    down = normal(rng, (E * d, eff), 0.05)
    x = normal(rng, d, 1.0)
    gq, uq, dq = quant(gate, gg.Q4_0), quant(up, gg.Q4_0), quant(down, gg.Q4_0)
    out, ids, w = R.moe_ffn(router, gq, uq, dq, gg.Q4_0, d, eff, E, k, x)
    lg = router.astype(np.float64) @ x
    p = np.exp(lg - lg.max())
    p /= p.sum()
    order = sorted(range(E), key=lambda i: (-p[i], i))[:k]
    assert ids.tolist() == order
    G, U, D = (deq(gq, gg.Q4_0, d).astype(np.float64), deq(uq, gg.Q4_0, d).astype(np.float64),
               deq(dq, gg.Q4_0, eff).astype(np.float64))
    ref = np.zeros(d)
    for e in order:
        g = G[e * eff:(e + 1) * eff] @ x
        u = U[e * eff:(e + 1) * eff] @ x
        hv = g / (1 + np.exp(-g)) * u
        ref += p[e] / p[order].sum() * (D[e * d:(e + 1) * d] @ hv)
    assert np.max(np.abs(out - ref)) <= 1e-5 * np.abs(ref).max()


def test_moe_invalid_hparams(rng):
    with pytest.raises(ValueError):
        R.moe_ffn(np.zeros((4, 32), np.float32), np.zeros(1, np.uint8), np.zeros(1, np.uint8),
                  np.zeros(1, np.uint8), gg.Q4_0, 32, 32, 4, 0, np.zeros(32, np.float32))


# ---------------------------------------------------------------- Falcon decode
FALCON_TINY = dict(n_layers=2, hidden=64, n_heads=4, n_kv=1, head_dim=16, ff=128, vocab=50,
                   max_seq=16, rank=8, rope_base=10000.0, eps=1e-5)


@pytest.mark.parametrize("n_kv", [1, 2, 4])
def test_falcon_forward_f64(rng, n_kv):
    """ForwardFlash restatement against a float64 brute force over 7 tokens:
    LayerNorm, RoPE at each position, MQA/GQA/MHA head mapping, causal softmax
    attention over the KV cache, predictor selection on the attention output,
    the sparse FFN on the normed input, the parallel residual and the LM head.
    The predictor logits it reports (every layer's) match the brute force's."""
    d = dict(FALCON_TINY, n_kv=n_kv)
    w = make_falcon(rng, d)
    toks = rng.integers(0, d["vocab"], 7)
    ref, nact, thr, plg = ref_falcon_f64(w, d, toks, pred_logits=True)
    m = R.Falcon(d, w, thr)
    for s, tk in enumerate(toks):
        lg, na, pl = m.forward(int(tk), s, pred_logits=True)
        assert np.array_equal(na, nact[s]), (s, na, nact[s])
        assert np.max(np.abs(lg - ref[s])) <= 1e-4 * np.max(np.abs(ref[s])), s
        assert np.max(np.abs(pl - plg[s])) <= 1e-5 * np.max(np.abs(plg[s])), s
        assert np.array_equal((pl > thr[:, None]).sum(1), na)
    assert 0 < nact.mean() < d["ff"]


def test_falcon_without_rope_f64(rng):
    """rope.freq_base missing or 0 means no RoPE (forward.go:249-252); the
    float64 brute force without the rotation must match, and differ from the
    rotated model after position 0."""
    d = dict(FALCON_TINY, rope_base=0.0)
    w = make_falcon(rng, d)
    toks = rng.integers(0, d["vocab"], 5)
    ref, nact, thr = ref_falcon_f64(w, d, toks)
    m = R.Falcon(d, w, thr)
    rot = R.Falcon(dict(d, rope_base=10000.0), w, thr)
    for s, tk in enumerate(toks):
        lg, na = m.forward(int(tk), s)
        lr, _ = rot.forward(int(tk), s)
        assert np.array_equal(na, nact[s])
        assert np.max(np.abs(lg - ref[s])) <= 1e-4 * np.max(np.abs(ref[s])), s
        if s > 0:
            assert np.max(np.abs(lr - lg)) > 1e-3 * np.max(np.abs(ref[s]))


def test_falcon_pos0_closed_form(rng):
    """At position 0 softmax over one key is 1, so every head's attention output
    is its KV head's value and RoPE is the identity: the first logits follow from
    the embedding row in closed form (no predictor neuron active)."""
    d = dict(FALCON_TINY, n_layers=1)
    w = make_falcon(rng, d)
    m = R.Falcon(d, w, [1e30])
    lg, na = m.forward(7, 0)
    assert na[0] == 0
    h, hd = d["hidden"], d["head_dim"]
    x = deq(w["embed"], gg.Q4_0, h)[7].astype(np.float64)
    ln = lambda z, g, b: (z - z.mean()) / np.sqrt(z.var() + d["eps"]) * g + b
    n = ln(x, w["norm_w"][0], w["norm_b"][0])
    v = deq(w["wv"][0], gg.Q4_0, h).astype(np.float64) @ n
    att = np.tile(v, d["n_heads"])
    x = x + deq(w["wo"][0], gg.Q4_0, d["n_heads"] * hd).astype(np.float64) @ att
    ref = deq(w["lm_head"], gg.Q4_0, h).astype(np.float64) @ ln(x, w["out_w"], w["out_b"])
    assert np.max(np.abs(lg - ref)) <= 1e-4 * np.max(np.abs(ref))


def test_falcon_kv_and_argmax(rng):
    """Positions beyond the cache are refused; argmax keeps the first maximum."""
    d = dict(FALCON_TINY, max_seq=3)
    w = make_falcon(rng, d)
    m = R.Falcon(d, w, [0.0, 0.0])
    for s in range(3):
        m.forward(1, s)
    with pytest.raises(ValueError):
        m.forward(1, 3)
    assert R.argmax(np.array([1, 3, 3, 2], np.float32)) == 1
    assert R.argmax(np.array([np.nan, 3, 5], np.float32)) == 0
    assert R.argmax(np.array([1, np.nan, 5], np.float32)) == 2


def test_matmulvec_threads_bit_identical():
    """set_threads splits MatMulVec's rows over threads; each row keeps its
    sequential sum (ops.go:51-58), so every thread count gives the same bits."""
    rng = np.random.default_rng(5)
    w = rng.standard_normal((2053, 1031)).astype(np.float32)
    x = rng.standard_normal(1031).astype(np.float32)
    one = R.matmulvec(w, x)
    try:
        for n in (2, 7, 16):
            R.set_threads(n)
            assert np.array_equal(R.matmulvec(w, x), one)
    finally:
        R.set_threads(1)
    ref = (w.astype(np.float64) @ x.astype(np.float64))
    assert np.max(np.abs(one - ref)) <= 1e-4 * np.max(np.abs(ref))


def test_sparse_ffn_and_falcon_threads_bit_identical(rng, tmp_path):
    """set_threads also splits the sparse FFN's up dots over neurons, its down
    sums over output elements and the attention over heads; every output still
    adds its terms in the reference's order, so the bits do not change."""
    h, ff = 512, 1024
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    x = normal(rng, h, 1.0)
    act = np.sort(rng.choice(ff, 300, replace=False)).astype(np.int32)
    d = dict(FALCON_TINY, n_heads=8, hidden=256, ff=512, max_seq=8)
    w = make_falcon(rng, d)
    toks = rng.integers(0, d["vocab"], 6)
    thr = np.zeros(d["n_layers"], np.float32)
    one = R.ffn_sparse_load(up, dn, gg.Q4_0, h, ff, x, act)
    m1 = R.Falcon(d, w, thr)
    ref = [m1.forward(int(t), s) for s, t in enumerate(toks)]
    try:
        R.set_threads(5)
        assert np.array_equal(R.ffn_sparse_load(up, dn, gg.Q4_0, h, ff, x, act), one)
        m5 = R.Falcon(d, w, thr)
        for s, t in enumerate(toks):
            lg, na = m5.forward(int(t), s)
            assert np.array_equal(lg, ref[s][0]) and np.array_equal(na, ref[s][1]), s
    finally:
        R.set_threads(1)
    assert np.max(np.abs(one - ref_sparse_f64(up, dn, gg.Q4_0, h, x, act))) <= 1e-4 * np.max(
        np.abs(one))


def test_falcon_ffn_rows_from_file_bit_identical(rng, tmp_path):
    """ForwardFlash with every layer's FFN rows read from a GGUF file by the
    ReadRowsParallel pool (ffn_flash.go:262-270, storage.go:246-319) gives the
    bits of the in-memory rows, from any position on; a file that cannot give
    the rows is an error of the forward."""
    from llg import gguf_file as GF

    d = dict(FALCON_TINY)
    w = make_falcon(rng, d)
    L, h, ff = d["n_layers"], d["hidden"], d["ff"]
    path = tmp_path / "ffn.gguf"
    tensors = []
    for l in range(L):
        tensors += [(f"blk.{l}.ffn_up.weight", [h, ff], gg.Q4_0, w["up"][l]),
                    (f"blk.{l}.ffn_down_t.weight", [h, ff], gg.Q4_0, w["down_t"][l])]
    GF.write_gguf(str(path), [("general.architecture", GF.T_STRING, "falcon")], tensors)
    gf = GF.open_gguf(str(path))
    up_off = [gf.by_name[f"blk.{l}.ffn_up.weight"].offset for l in range(L)]
    dn_off = [gf.by_name[f"blk.{l}.ffn_down_t.weight"].offset for l in range(L)]
    toks = rng.integers(0, d["vocab"], 8)
    _, _, thr = ref_falcon_f64(w, d, toks)
    mem, fil = R.Falcon(d, w, thr), R.Falcon(d, w, thr)
    for s, t in enumerate(toks):
        if s == 3:
            fil.ffn_file(path, up_off, dn_off, nthreads=4)
        a, b = mem.forward(int(t), s), fil.forward(int(t), s)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1]), s
    assert np.sum([mem.forward(int(toks[0]), 8)[1]]) > 0  # rows were read at all
    fil.forward(int(toks[0]), 8)
    bad = R.Falcon(d, w, thr)
    bad.ffn_file(path, [path.stat().st_size] * L, dn_off, nthreads=2)
    with pytest.raises(OSError):
        bad.forward(int(toks[0]), 0)
