"""On-disk formats (gguf/reader.go, gguf/types.go, flash/bundle.go,
model/loader.go hyperparameters): CPU checks.

The GGUF reader is pinned by a file assembled byte by byte from the format's
definition (independently of this package's writer), the writer by reading
its files back, the bundle file by its byte layout (header fields, neuron
offsets 16 + i * 2 * hidden * 4 for float32 rows as bundle.go:66-111 writes),
and the loader's hyperparameters by the fallbacks of loader.go:102-165.
"""
import struct

import numpy as np
import pytest
import torch

import llg.bundle as B
import llg.gguf as gg
import llg.gguf_file as G
import llg.loader as LD
from oracle import refcpu as R
from tests.helpers import make_falcon, normal, quant


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def handmade_gguf(path, version=3, magic=0x46554747, n_dims=2, meta_type=0,
                  str_len=None, arr_count=None):
    """One Q4_0 tensor [2 rows x 32] and metadata of several types."""
    body = struct.pack("<IIQQ", magic, version, 1, 6)
    body += _s("k.u8") + struct.pack("<I", meta_type) + struct.pack("<B", 0xAB)
    body += _s("k.i32") + struct.pack("<Ii", 5, -7)
    body += _s("k.f32") + struct.pack("<If", 6, 1.5)
    if str_len is None:
        body += _s("k.str") + struct.pack("<I", 8) + _s("falcon")
    else:
        body += _s("k.str") + struct.pack("<IQ", 8, str_len)
    n = 2 if arr_count is None else arr_count
    body += _s("k.arr") + struct.pack("<IIQ", 9, 8, n) + _s("x") + _s("yz")
    body += _s("k.u64") + struct.pack("<IQ", 10, 1 << 40)
    dims = [32, 2, 1, 1, 1][:n_dims]
    body += _s("t.w") + struct.pack("<I", n_dims) + b"".join(struct.pack("<Q", d) for d in dims)
    body += struct.pack("<IQ", gg.Q4_0, 0)
    pos = len(body)
    pad = (pos + 31) // 32 * 32 - pos
    data = bytes(range(36))
    with open(path, "wb") as f:
        f.write(body + b"\0" * pad + data)
    return pos + pad, data


def test_reader_known_file(tmp_path):
    p = tmp_path / "k.gguf"
    data_off, data = handmade_gguf(p)
    f = G.open_gguf(p)
    assert (f.version, f.tensor_count, f.meta_count) == (3, 1, 6)
    assert f.meta["k.u8"].value == 0xAB and f.meta["k.i32"].value == -7
    assert f.meta_float32("k.f32") == 1.5 and f.meta_string("k.str") == "falcon"
    assert f.meta_string_array("k.arr") == ["x", "yz"]
    assert f.meta_uint64("k.u64") == 1 << 40
    ti = f.by_name["t.w"]
    assert ti.dims == [32, 2] and ti.type == gg.Q4_0 and ti.shape() == [2, 32]
    assert f.data_offset == data_off and f.data_offset % 32 == 0 and ti.offset == data_off
    assert bytes(f.tensor_bytes(ti)) == data
    assert f.tensor_rows("t.w").shape == (2, 18)


def test_reader_getter_conversions(tmp_path):
    p = tmp_path / "k.gguf"
    handmade_gguf(p)
    f = G.open_gguf(p)
    assert f.meta_uint32("k.i32") == (-7) & 0xFFFFFFFF      # uint32(int32) (reader.go:146)
    assert f.meta_uint32("k.u64") == 0                        # uint32(1 << 40)
    assert f.meta_int("k.i32") == -7 and f.meta_int("k.u64") == 1 << 40
    with pytest.raises(G.GGUFError):
        f.meta_float32("k.u8")
    with pytest.raises(G.GGUFError):
        f.meta_string("missing")
    with pytest.raises(G.GGUFError):
        f.meta_int("k.f32")


@pytest.mark.parametrize("kw,msg", [
    (dict(magic=0x12345678), "bad magic"), (dict(version=0), "unsupported version"),
    (dict(version=4), "unsupported version"), (dict(n_dims=5), "too many dimensions"),
    (dict(meta_type=13), "unknown MetaValueType"), (dict(str_len=(1 << 24) + 1), "string too long"),
    (dict(arr_count=(1 << 20) + 1), "array too large")])
def test_reader_errors(tmp_path, kw, msg):
    p = tmp_path / "bad.gguf"
    handmade_gguf(p, **kw)
    with pytest.raises(G.GGUFError, match=msg):
        G.open_gguf(p)


def test_reader_truncated(tmp_path):
    p = tmp_path / "k.gguf"
    handmade_gguf(p)
    raw = p.read_bytes()
    (tmp_path / "cut.gguf").write_bytes(raw[:50])
    with pytest.raises(G.GGUFError, match="end of file"):
        G.open_gguf(tmp_path / "cut.gguf")
    (tmp_path / "short.gguf").write_bytes(raw[:-1])  # tensor data one byte short
    f = G.open_gguf(tmp_path / "short.gguf")
    with pytest.raises(G.GGUFError, match="past the end"):
        f.tensor_bytes(f.tensors[0])


def test_writer_round_trip(tmp_path, rng):
    meta = [("a.u8", G.T_U8, 200), ("a.i8", G.T_I8, -3), ("a.u16", G.T_U16, 65000),
            ("a.i16", G.T_I16, -300), ("a.u32", G.T_U32, 4000000000), ("a.i32", G.T_I32, -5),
            ("a.f32", G.T_F32, 0.25), ("a.bool", G.T_BOOL, True), ("a.str", G.T_STRING, "héllo"),
            ("a.u64", G.T_U64, 1 << 50), ("a.i64", G.T_I64, -(1 << 50)), ("a.f64", G.T_F64, 0.1),
            ("a.arr", G.T_ARRAY, (G.T_I32, [1, -2, 3])),
            ("a.nest", G.T_ARRAY, (G.T_ARRAY, [G.ArrayValue(G.T_U8, [1, 2]),
                                               G.ArrayValue(G.T_U8, [])]))]
    w32 = normal(rng, (3, 64), 1.0)
    tensors = [("t.f32", [64, 3], gg.F32, w32),
               ("t.q4", [64, 3], gg.Q4_0, quant(w32, gg.Q4_0)),
               ("t.q8", [64, 3], gg.Q8_0, quant(w32, gg.Q8_0)),
               ("t.f16", [5], gg.F16, np.arange(5, dtype=np.float16)),
               ("t.q4k", [256], 12, np.arange(144, dtype=np.uint8))]
    p = tmp_path / "w.gguf"
    G.write_gguf(p, meta, tensors)
    f = G.open_gguf(p)
    for k, t, v in meta:
        mv = f.meta[k]
        assert mv.type == t
        if t == G.T_ARRAY:
            et, vals = v
            assert mv.value.elem_type == et and len(mv.value.values) == len(vals)
        elif t in (G.T_F32,):
            assert mv.value == np.float32(v)
        else:
            assert mv.value == v
    assert f.meta["a.nest"].value.values[0].values == [1, 2]
    for name, dims, t, data in tensors:
        ti = f.by_name[name]
        assert ti.dims == dims and ti.type == t and (ti.offset - f.data_offset) % 32 == 0
        assert bytes(f.tensor_bytes(ti)) == np.ascontiguousarray(data).view(np.uint8).tobytes()


def test_writer_rejects_wrong_size(tmp_path):
    with pytest.raises(G.GGUFError):
        G.write_gguf(tmp_path / "x.gguf", [], [("t", [64], gg.Q4_0, np.zeros(35, np.uint8))])


def test_type_table():
    """GGMLType.ByteSize over the reference's TypeInfos (types.go:70-102)."""
    assert gg.byte_size(gg.Q4_0, 4544) == 2556 and gg.byte_size(gg.Q8_0, 4544) == 4828
    assert gg.byte_size(gg.F16, 4544) == 9088 and gg.byte_size(12, 512) == 288   # Q4_K
    assert gg.byte_size(14, 256) == 210 and gg.byte_size(28, 3) == 24             # Q6_K, F64
    with pytest.raises(ValueError, match="not divisible"):
        gg.byte_size(gg.Q4_0, 33)
    with pytest.raises(ValueError, match="unknown GGML type"):
        gg.byte_size(4, 32)  # 4 and 5 are not in the table


# ---------------------------------------------------------------- bundle files
def _layer_gguf(tmp_path, rng, t, h=64, n=48):
    up, dn = quant(normal(rng, (n, h), 0.1), t), quant(normal(rng, (n, h), 0.1), t)
    p = tmp_path / "layer.gguf"
    G.write_gguf(p, [], [("blk.0.ffn_up.weight", [h, n], t, up),
                         ("blk.0.ffn_down.weight", [h, n], t, dn)])
    f = G.open_gguf(p)
    return f, f.by_name["blk.0.ffn_up.weight"], f.by_name["blk.0.ffn_down.weight"], up, dn


@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16])
def test_bundle_f32_file_layout(tmp_path, rng, t):
    """The reference's float32 bundle file (bundle.go:66-111) byte for byte."""
    h, n = 64, 48
    f, ui, di, up, dn = _layer_gguf(tmp_path, rng, t, h, n)
    p = tmp_path / "l.bundle"
    B.create_bundle(p, f, ui, di)
    raw = p.read_bytes()
    assert struct.unpack("<IIII", raw[:16]) == (0x424E444C, n, h, 0)
    assert len(raw) == 16 + n * 2 * h * 4
    for i in (0, 17, n - 1):
        off = 16 + i * 2 * h * 4
        row = np.frombuffer(raw[off:off + 2 * h * 4], "<f4")
        assert np.array_equal(row[:h], R.dequantize(up[i], t))
        assert np.array_equal(row[h:], R.dequantize(dn[i], t))


@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16])
def test_bundle_typed_rows(tmp_path, rng, t):
    h, n = 64, 48
    f, ui, di, up, dn = _layer_gguf(tmp_path, rng, t, h, n)
    B.create_bundle(tmp_path / "q.bundle", f, ui, di, row_type=None)
    B.create_bundle(tmp_path / "f.bundle", f, ui, di)
    q, f32 = B.open_bundle(tmp_path / "q.bundle"), B.open_bundle(tmp_path / "f.bundle")
    assert (q.n_neurons, q.hidden, q.row_type) == (n, h, t)
    assert q.bytes_per_row == 2 * gg.byte_size(t, h)
    u, d = q.halves()
    assert np.array_equal(u, up) and np.array_equal(d, dn)
    sel = [5, 0, 47, 5]
    for a, b in zip(q.read_neurons(sel), f32.read_neurons(sel)):
        assert np.array_equal(a, b)


def test_bundle_errors(tmp_path, rng):
    f, ui, di, _, _ = _layer_gguf(tmp_path, rng, gg.Q4_0)
    bad = G.TensorInfo("d", [32, 48], gg.Q4_0, di.offset)
    with pytest.raises(G.GGUFError, match="dimension mismatch"):
        B.create_bundle(tmp_path / "x.bundle", f, ui, bad)
    B.create_bundle(tmp_path / "ok.bundle", f, ui, di)
    with pytest.raises(G.GGUFError, match="outside"):
        B.open_bundle(tmp_path / "ok.bundle").read_neurons([48])
    raw = bytearray((tmp_path / "ok.bundle").read_bytes())
    raw[0] ^= 1
    (tmp_path / "bad.bundle").write_bytes(bytes(raw))
    with pytest.raises(G.GGUFError, match="bad magic"):
        B.open_bundle(tmp_path / "bad.bundle")


# ---------------------------------------------------------------- loader
def test_hparams_fallbacks(tmp_path):
    a = "falcon."
    G.write_gguf(tmp_path / "m.gguf",
                 [("general.architecture", G.T_STRING, "falcon"),
                  (a + "embedding_length", G.T_U32, 64), (a + "feed_forward_length", G.T_U64, 128),
                  (a + "block_count", G.T_I32, 2), (a + "attention.head_count", G.T_U32, 4),
                  (a + "attention.layer_norm_rms_epsilon", G.T_F32, 1e-6)],
                 [("token_embd.weight", [64, 50], gg.Q4_0, np.zeros(50 * 36, np.uint8))])
    hp = LD.load_hparams(G.open_gguf(tmp_path / "m.gguf"), "falcon")
    assert hp["vocab"] == 50                        # from token_embd dims (loader.go:109-115)
    assert hp["n_kv"] == 4 and hp["head_dim"] == 16  # MHA default, HeadDim = hidden / heads
    assert hp["eps"] == np.float32(1e-6)            # rms epsilon fallback
    assert hp["context_len"] == 2048 and hp["rope_base"] == 0.0
    assert LD.activation_for("falcon") == gg.ACT_GELU
    assert LD.activation_for("qwen3moe") == gg.ACT_SILU and LD.activation_for("opt") == gg.ACT_RELU


def test_falcon_gguf_round_trip(tmp_path, rng):
    d = dict(n_layers=2, hidden=64, n_heads=4, n_kv=1, head_dim=16, ff=128, vocab=50,
             max_seq=16, rank=8, rope_base=10000.0, eps=1e-5)
    w = make_falcon(rng, d)
    LD.write_falcon_gguf(tmp_path / "f.gguf", d, w, gg.Q4_0, thresholds=[0.5, -0.25])
    f = G.open_gguf(tmp_path / "f.gguf")
    hp = LD.load_hparams(f, "falcon")
    assert (hp["hidden"], hp["ff"], hp["n_layers"], hp["n_heads"], hp["n_kv"], hp["vocab"]) == \
        (64, 128, 2, 4, 1, 50)
    assert np.array_equal(f.tensor_rows("blk.1.attn_q.weight"), w["wq"][1])
    assert np.array_equal(f.tensor_rows("blk.0.ffn_down.weight"), w["down_t"][0])
    assert f.meta["llg.predictor.thresholds"].value.values == [0.5, -0.25]


def test_load_falcon_rejects_unsupported(tmp_path, rng):
    """RMSNorm layers (no bias), attention biases and other architectures are
    refused before anything reaches the device."""
    d = dict(n_layers=1, hidden=64, n_heads=4, n_kv=1, head_dim=16, ff=128, vocab=50,
             max_seq=16, rank=8, rope_base=10000.0, eps=1e-5)
    w = make_falcon(rng, d)
    p = tmp_path / "f.gguf"
    LD.write_falcon_gguf(p, d, w, gg.Q4_0, thresholds=[0.0])
    f = G.open_gguf(p)
    keep = [(ti.name, ti.dims, ti.type, np.array(f.tensor_bytes(ti))) for ti in f.tensors]
    meta = [(k, v.type, v.value) for k, v in f.meta.items()]

    def variant(name, drop=(), add=(), arch=None):
        m = [(k, t, (arch if k == "general.architecture" and arch else v)) for k, t, v in meta]
        ts = [x for x in keep if x[0] not in drop] + list(add)
        G.write_gguf(tmp_path / name, m, ts)
        return tmp_path / name

    with pytest.raises(G.GGUFError, match="RMSNorm"):
        LD.load_falcon(None, variant("a.gguf", drop=("blk.0.attn_norm.bias",)))
    with pytest.raises(G.GGUFError, match="not supported"):
        LD.load_falcon(None, variant("b.gguf", add=[("blk.0.attn_q.bias", [64], gg.F32,
                                                      np.zeros(64, np.float32))]))
    with pytest.raises(G.GGUFError, match="falcon layout only"):
        LD.load_falcon(None, variant("c.gguf", arch="llama"))
    with pytest.raises(G.GGUFError, match="not found"):
        LD.load_falcon(None, variant("d.gguf", drop=("blk.0.ffn_norm.weight",)))
    with pytest.raises(G.GGUFError, match="dims"):
        bad = [x if x[0] != "blk.0.ffn_down.weight" else (x[0], [128, 64], x[2], x[3])
               for x in keep]
        G.write_gguf(tmp_path / "e.gguf", meta, bad)
        LD.load_falcon(None, tmp_path / "e.gguf")
