"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every stored output bit for bit (the fixtures
freeze the oracle).  GPU: the HIP path matches them (bit-exact for dequant,
index sets and expert ids; 1e-3 of the output max-abs for FFN outputs).
"""
from pathlib import Path

import numpy as np
import pytest

from oracle import refcpu as R

G = Path(__file__).resolve().parent / "golden"
TOL = 1e-3


def load(name):
    return np.load(G / f"{name}.npz", allow_pickle=False)


def rel(got, ref):
    return float(np.max(np.abs(got - ref)) / max(float(np.max(np.abs(ref))), 1e-30))


# ---------------------------------------------------------------- CPU: oracle
def test_oracle_dequant_kat():
    z = load("dequant_kat")
    assert [R.f16_to_f32_bits(int(h)) for h in z["f16_in"]] == z["f16_out_bits"].tolist()
    for b, o in zip(z["q4_in"], z["q4_out"]):
        assert np.array_equal(R.dequantize(b, R.Q4_0), o)
    for b, o in zip(z["q8_in"], z["q8_out"]):
        assert np.array_equal(R.dequantize(b, R.Q8_0), o)


def test_oracle_ffn_swiglu_tiny():
    z = load("ffn_swiglu_tiny")
    h, ff = z["x"].size, z["q4_0_gate"].shape[0]
    for name, t in (("q4_0", R.Q4_0), ("q8_0", R.Q8_0), ("f16", R.F16)):
        out = R.ffn_swiglu(z[f"{name}_gate"], z[f"{name}_up"], z[f"{name}_down"], t, h, ff, z["x"])
        assert np.array_equal(out, z[f"{name}_out"]), name


def test_oracle_pred_tiny():
    z = load("pred_tiny")
    act, lg = R.predict(z["wup"], z["wout"], z["bias"], z["a"], float(z["threshold"]))
    assert np.array_equal(act, z["active"]) and np.array_equal(lg, z["logits"])


def test_oracle_ffn_sparse_tiny():
    z = load("ffn_sparse_tiny")
    h, ff = z["x"].size, z["q4_0_up"].shape[0]
    for name, t in (("q4_0", R.Q4_0), ("q8_0", R.Q8_0), ("f16", R.F16)):
        for act_name, act in (("relu", 0), ("silu", 2), ("gelu", 1)):
            out = R.ffn_sparse_load(z[f"{name}_up"], z[f"{name}_down_t"], t, h, ff, z["x"],
                                    z["active"], act)
            assert np.array_equal(out, z[f"{name}_out_{act_name}"])


def test_oracle_ffn_dense_tiny():
    z = load("ffn_dense_tiny")
    h, ff = z["x"].size, z["up"].shape[0]
    assert np.array_equal(R.ffn_dense(z["up"], z["down"], R.Q4_0, h, ff, z["x"]), z["out"])


def test_oracle_window_tiny():
    z = load("window_tiny")
    ff, h = z["up"].shape[0], z["xs"].shape[1]
    nc = R.NeuronCache(256, h, int(z["k"]), ff, z["up"], z["down_t"], R.Q4_0)
    for t, A in enumerate(z["sets"]):
        assert nc.update(A).size == z["n_loaded"][t]
        assert nc.num_cached() == z["n_cached"][t]
        assert np.array_equal(np.flatnonzero(z["resident"][t]), nc.resident())
        assert np.array_equal(nc.ffn_forward(z["xs"][t], A), z["outs"][t])


def test_oracle_moe_tiny():
    z = load("moe_tiny")
    d, E = z["x"].shape[1], z["router"].shape[0]
    eff = z["gate"].shape[0] // E
    for t in range(z["x"].shape[0]):
        o, i, w = R.moe_ffn(z["router"], z["gate"], z["up"], z["down"], R.Q4_0, d, eff, E,
                            int(z["k"]), z["x"][t])
        assert np.array_equal(o, z["out"][t]) and np.array_equal(i, z["ids"][t])
        assert np.array_equal(w, z["w"][t])
    for t in range(z["route_logits"].shape[0]):
        i, w = R.moe_route(z["route_logits"][t], 2)
        assert np.array_equal(i, z["route_ids"][t]) and np.array_equal(w, z["route_w"][t])


# ---------------------------------------------------------------- GPU: HIP path
@pytest.mark.gpu
def test_gpu_dequant_kat(dev):
    z = load("dequant_kat")
    q4 = dev.upload_matrix(z["q4_in"], R.Q4_0, z["q4_in"].shape[0], 32)
    assert np.array_equal(dev.dequant(q4, 0, z["q4_in"].shape[0]), z["q4_out"])
    q8 = dev.upload_matrix(z["q8_in"], R.Q8_0, z["q8_in"].shape[0], 32)
    assert np.array_equal(dev.dequant(q8, 0, z["q8_in"].shape[0]), z["q8_out"])
    f16 = dev.upload_matrix(z["f16_in"].view(np.uint8), R.F16, 1, z["f16_in"].size)
    assert np.array_equal(dev.dequant(f16, 0, 1).view(np.uint32)[0], z["f16_out_bits"])
    for m in (q4, q8, f16):
        m.release()


@pytest.mark.gpu
def test_gpu_pred_tiny(dev):
    import llg

    z = load("pred_tiny")
    p = llg.Predictor(dev, z["wup"], z["wout"], z["bias"], float(z["threshold"]))
    act, lg = p.predict(z["a"], return_logits=True)
    assert np.array_equal(act, z["active"])
    assert np.max(np.abs(lg - z["logits"])) <= 1e-5 * np.max(np.abs(z["logits"]))


@pytest.mark.gpu
def test_gpu_ffn_sparse_tiny(dev):
    import llg

    z = load("ffn_sparse_tiny")
    h, ff = z["x"].size, z["q4_0_up"].shape[0]
    for name, t in (("q4_0", R.Q4_0), ("q8_0", R.Q8_0), ("f16", R.F16)):
        b = dev.upload_bundle(z[f"{name}_up"], z[f"{name}_down_t"], t, h, ff)
        for act_name, act in (("relu", 0), ("silu", 2), ("gelu", 1)):
            out = llg.ffn_sparse_load(dev, b, z["x"], z["active"], act)
            assert rel(out, z[f"{name}_out_{act_name}"]) <= TOL, (name, act_name)
        b.release()


@pytest.mark.gpu
def test_gpu_ffn_swiglu_tiny(dev):
    import llg

    z = load("ffn_swiglu_tiny")
    h, ff = z["x"].size, z["q4_0_gate"].shape[0]
    for name, t in (("q4_0", R.Q4_0), ("q8_0", R.Q8_0), ("f16", R.F16)):
        g = dev.upload_matrix(z[f"{name}_gate"], t, ff, h)
        u = dev.upload_matrix(z[f"{name}_up"], t, ff, h)
        d = dev.upload_matrix(z[f"{name}_down"], t, h, ff)
        assert rel(llg.ffn_swiglu(dev, g, u, d, z["x"]), z[f"{name}_out"]) <= TOL, name
        for m in (g, u, d):
            m.release()


@pytest.mark.gpu
def test_gpu_ffn_dense_tiny(dev):
    import llg

    z = load("ffn_dense_tiny")
    h, ff = z["x"].size, z["up"].shape[0]
    u = dev.upload_matrix(z["up"], R.Q4_0, ff, h)
    d = dev.upload_matrix(z["down"], R.Q4_0, h, ff)
    assert rel(llg.ffn_dense(dev, u, d, z["x"]), z["out"]) <= TOL
    u.release()
    d.release()


@pytest.mark.gpu
def test_gpu_window_tiny(dev):
    import llg

    z = load("window_tiny")
    ff, h = z["up"].shape[0], z["xs"].shape[1]
    b = dev.upload_bundle(z["up"], z["down_t"], R.Q4_0, h, ff)
    nc = llg.NeuronCache(dev, b, int(z["k"]))
    for t, A in enumerate(z["sets"]):
        assert nc.update(A) == z["n_loaded"][t]
        assert nc.num_cached() == z["n_cached"][t]
        assert np.array_equal(nc.resident(), np.flatnonzero(z["resident"][t]))
        assert rel(nc.ffn_forward(z["xs"][t], A), z["outs"][t]) <= TOL
    b.release()


@pytest.mark.gpu
def test_gpu_moe_tiny(dev):
    import llg

    z = load("moe_tiny")
    d, E = z["x"].shape[1], z["router"].shape[0]
    eff = z["gate"].shape[0] // E
    hs = (dev.upload_f32(z["router"]), dev.upload_matrix(z["gate"], R.Q4_0, E * eff, d),
          dev.upload_matrix(z["up"], R.Q4_0, E * eff, d),
          dev.upload_matrix(z["down"], R.Q4_0, E * d, eff))
    out, ids, w = llg.moe_ffn(dev, *hs, E, int(z["k"]), z["x"])
    assert np.array_equal(ids, z["ids"])
    for t in range(z["x"].shape[0]):
        assert rel(out[t], z["out"][t]) <= TOL
    r_ids, r_w = dev.moe_route(z["route_logits"], 2)
    assert np.array_equal(r_ids, z["route_ids"])
    assert np.array_equal(r_w.view(np.uint32), z["route_w"].view(np.uint32))
    for hnd in hs:
        hnd.release()
