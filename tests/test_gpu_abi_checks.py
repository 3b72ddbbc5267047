"""The C side's own argument checks, called through the raw C ABI (no Python
mirror in between), as a Go binding would call them.

A Go method checks its slice lengths against the shapes llg_hip_object_info
reports (as metal/metal.go:55-60,77-80 checks its own), then relies on the
library to reject what only the library can see: objects whose shapes do not
fit each other, empty or null arguments, indices and row ranges outside the
object (storage.go:292-294), counts above the neuron count.  Each call below
returns its code before any kernel is launched, and the device stays usable."""
import ctypes as C

import numpy as np
import pytest

import llg
import llg.gguf as gg
from tests.helpers import make_sparse_layer, normal

pytestmark = pytest.mark.gpu


def _f(a):
    return a.ctypes.data_as(C.c_void_p)


def _info(dev, hid):
    t, r, c, s = C.c_int(), C.c_int(), C.c_int(), C.c_int64()
    rc = dev.lib.llg_hip_object_info(dev.h, hid, C.byref(t), C.byref(r), C.byref(c), C.byref(s))
    return rc, (t.value, r.value, c.value, s.value)


def test_object_info_shapes_for_the_go_checks(dev, rng):
    """Matrix: (type, rows, cols); bundle and window: (type, neurons, hidden)."""
    h, ff = 64, 96
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    m = dev.upload_matrix(up, gg.Q4_0, ff, h)
    b = dev.upload_bundle(up, dn, gg.Q4_0, h, ff)
    nc = llg.NeuronCache(dev, b, 2)
    for hid in (m.id, b.id, nc.win.id):
        rc, (t, r, c, _) = _info(dev, hid)
        assert rc == 0 and (t, r, c) == (gg.Q4_0, ff, h), (hid, t, r, c)
    nc.win.release()
    m.release()
    b.release()
    rc, _ = _info(dev, m.id)
    assert rc == llg.LLG_E_HANDLE


def test_c_side_rejects_mismatched_and_out_of_range_arguments(dev, rng):
    L, hd = dev.lib, dev.h
    h, ff, rank = 64, 96, 8
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    b = dev.upload_bundle(up, dn, gg.Q4_0, h, ff)
    up2, dn2 = make_sparse_layer(rng, h, 2 * ff, gg.Q4_0)
    b2 = dev.upload_bundle(up2, dn2, gg.Q4_0, h, 2 * ff)
    wup = dev.upload_matrix(normal(rng, (rank, h), 0.05), gg.F32, rank, h)
    wout = dev.upload_matrix(normal(rng, (ff, rank), 0.05), gg.F32, ff, rank)
    wout_bad = dev.upload_matrix(normal(rng, (ff, rank + 4), 0.05), gg.F32, ff, rank + 4)
    m_up = dev.upload_matrix(up, gg.Q4_0, ff, h)
    dq = gg.quantize(__import__("torch").from_numpy(normal(rng, (h, ff), 0.02)), gg.Q4_0).numpy()
    m_dn = dev.upload_matrix(dq, gg.Q4_0, h, ff)
    m_dn_bad = dev.upload_matrix(up2[:, :], gg.Q4_0, 2 * ff, h)
    x = normal(rng, h, 1.0)
    out = np.zeros(h, np.float32)
    act = np.zeros(2 * ff, np.int32)
    n = C.c_int()
    rc = lambda r, code, what: (r == code) or pytest.fail(f"{what}: rc {r} != {code}")

    # RMSNorm / MatMulVec (metal.go:72-113): empty and null arguments
    rc(L.llg_hip_rmsnorm(hd, _f(x), _f(x), _f(out), 0, 1e-5), llg.LLG_E_ARG, "rmsnorm n=0")
    rc(L.llg_hip_rmsnorm(hd, _f(x), None, _f(out), h, 1e-5), llg.LLG_E_ARG, "rmsnorm null w")
    rc(L.llg_hip_matvec(hd, _f(x), 0, h, _f(x), _f(out)), llg.LLG_E_ARG, "matvec rows=0")
    # predictor: W_out cols != W_up rows (predictor.go:57-66)
    rc(L.llg_hip_predict(hd, wup.id, wout_bad.id, 0, _f(x), 0.0, _f(act), C.byref(n), None),
       llg.LLG_E_ARG, "predict rank mismatch")
    # ffnFlash path 2: predictor neurons != bundle neurons
    rc(L.llg_hip_ffn_predict_sparse(hd, wup.id, wout.id, 0, b2.id, _f(x), _f(x), 0.0,
                                    gg.ACT_RELU, _f(out), None, None),
       llg.LLG_E_ARG, "predict_sparse shape mismatch")
    # ffnSparseLoad: an index outside [0, ff) is the storage range error
    bad = np.array([3, ff], np.int32)
    rc(L.llg_hip_ffn_sparse(hd, b.id, _f(x), _f(bad), 2, gg.ACT_RELU, _f(out)),
       llg.LLG_E_RANGE, "ffn_sparse index ff")
    rc(L.llg_hip_ffn_sparse(hd, b.id, _f(x), None, 2, gg.ACT_RELU, _f(out)),
       llg.LLG_E_ARG, "ffn_sparse null list")
    # dense path: up [ff x h] against a down that is not [h x ff]
    rc(L.llg_hip_ffn_dense(hd, m_up.id, m_dn_bad.id, _f(x), gg.ACT_RELU, _f(out)),
       llg.LLG_E_ARG, "ffn_dense mismatch")
    rc(L.llg_hip_ffn_swiglu(hd, m_up.id, m_dn_bad.id, m_dn.id, _f(x), _f(out)),
       llg.LLG_E_ARG, "ffn_swiglu gate != up")
    # window: more entries than neurons, an index out of range
    nc = llg.NeuronCache(dev, b, 2)
    many = np.arange(ff + 1, dtype=np.int32)
    rc(L.llg_hip_window_update(hd, nc.win.id, _f(many), ff + 1, None, None),
       llg.LLG_E_ARG, "window_update count > ff")
    rc(L.llg_hip_window_update(hd, nc.win.id, _f(bad), 2, None, None),
       llg.LLG_E_RANGE, "window_update index ff")
    # MoE: router rows != n_exp
    rc(L.llg_hip_moe_ffn(hd, wup.id, m_up.id, m_up.id, m_dn.id, 4, 2, _f(x), 1, _f(out),
                         None, None),
       llg.LLG_E_ARG, "moe router shape")
    # selection and dequant ranges
    rc(L.llg_hip_select(hd, _f(x), 0, 0.0, _f(act), C.byref(n)), llg.LLG_E_ARG, "select ff=0")
    buf = np.zeros(2 * h * 2, np.float32)
    rc(L.llg_hip_dequant(hd, b.id, ff - 1, 2, _f(buf)), llg.LLG_E_RANGE, "dequant past end")
    # the device is still usable: a valid call succeeds
    good = np.array([1, 5, 7], np.int32)
    assert L.llg_hip_ffn_sparse(hd, b.id, _f(x), _f(good), 3, gg.ACT_RELU, _f(out)) == 0
    assert np.all(np.isfinite(out)) and np.any(out != 0)
    for o in (nc.win, b, b2, wup, wout, wout_bad, m_up, m_dn, m_dn_bad):
        o.release()
