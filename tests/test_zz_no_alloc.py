"""The allocation-free sparse step, llg_hipd_ffn_predict_sparse_noalloc (its
workspace is the GPU's fixed scratch array), through the C ABI against
llg_hipd_ffn_predict_sparse (the handle's growable workspace) on the same
inputs, and both against the oracle (predictor.go:51-83 then
ffn_flash.go:254-299).

Calls follow one another on the handle's stream with the scratch keeping the
previous call's contents: the Falcon-7B layer, then a smaller layer, then the
Falcon-7B layer again; a workload whose workspace exceeds the scratch is
rejected with LLG_E_SCRATCH while the allocating entry point accepts it."""
import ctypes as C

import numpy as np
import pytest
import torch

import llg
import llg.gguf as gg
from oracle import refcpu as R
from tests.helpers import make_sparse_layer, max_rel_err, normal, threshold_for  # noqa: F401

pytestmark = pytest.mark.gpu

TOL = 1e-3  # FFN output tolerance relative to the output's max-abs


def _layer(dev, rng, h, ff, rank, n_active):
    up, dn = make_sparse_layer(rng, h, ff, gg.Q4_0)
    wup = normal(rng, (rank, h), 0.05)
    wout = normal(rng, (ff, rank), 0.05)
    x = normal(rng, h, 1.0)
    _, lg = R.predict(wup, wout, None, x, 0.0)
    thr = threshold_for(lg, n_active)
    ref_act, _ = R.predict(wup, wout, None, x, thr)
    assert ref_act.size == n_active
    ref = R.ffn_sparse_load(up, dn, gg.Q4_0, h, ff, x, ref_act)
    pred = llg.Predictor(dev, wup, wout, None, thr)
    bundle = dev.upload_bundle(up, dn, gg.Q4_0, h, ff)
    return dict(h=h, ff=ff, x=x, thr=thr, pred=pred, bundle=bundle, ref=ref, ref_act=ref_act)


def _call(dev, fn, L):
    """One sparse step through the C ABI on device buffers; returns
    (rc, out, active list)."""
    h, ff, p = L["h"], L["ff"], L["pred"]
    x = torch.from_numpy(L["x"]).cuda()
    out = torch.full((h,), float("nan"), device="cuda")
    act = torch.full((ff,), -7, dtype=torch.int32, device="cuda")
    n = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()  # inputs written on torch's stream before the library's reads
    vp = lambda t: C.c_void_p(t.data_ptr())
    rc = fn(dev.h, p.w_up.id, p.w_out.id, p.bias_id, L["bundle"].id, vp(x), vp(x),
            C.c_float(L["thr"]), gg.ACT_RELU, vp(out), vp(act), vp(n))
    if rc:
        return rc, None, None
    dev.sync()
    k = int(n.cpu()[0])
    return rc, out.cpu().numpy(), act[:k].cpu().numpy()


def _check(dev, L):
    rc0, out0, act0 = _call(dev, dev.lib.llg_hipd_ffn_predict_sparse, L)
    rc1, out1, act1 = _call(dev, dev.lib.llg_hipd_ffn_predict_sparse_noalloc, L)
    dev.check(rc0, "predict_sparse")
    dev.check(rc1, "predict_sparse_noalloc")
    assert np.array_equal(act1, act0) and np.array_equal(act1, L["ref_act"])
    assert max_rel_err(out1, out0.astype(np.float64)) <= TOL
    assert max_rel_err(out1, L["ref"]) <= TOL
    return out1


def test_noalloc_matches_allocating_entry(dev):
    rng = np.random.default_rng(20260)
    big = _layer(dev, rng, 4544, 18176, 128, 909)     # the Falcon-7B layer at 5%
    small = _layer(dev, rng, 1024, 4096, 32, 205)     # a smaller one next
    _check(dev, big)
    _check(dev, small)
    _check(dev, big)
    for L in (big, small):
        L["pred"].w_up.release()
        L["pred"].w_out.release()
        L["bundle"].release()


def test_noalloc_first_on_fresh_handle_allocates_nothing():
    """On a fresh device handle, whose workspace is still empty (uploads take
    none), the allocation-free entry point runs first and leaves the workspace
    at 0 bytes, twice; its results match the oracle.  The allocating entry
    point, called only afterwards, then grows the workspace, which shows that
    the first calls would have had to allocate through it."""
    fresh = llg.Device()
    try:
        rng = np.random.default_rng(20262)
        big = _layer(fresh, rng, 4544, 18176, 128, 909)
        small = _layer(fresh, rng, 1024, 4096, 32, 205)
        assert fresh.workspace_bytes() == 0
        for L in (big, small):
            rc, out, act = _call(fresh, fresh.lib.llg_hipd_ffn_predict_sparse_noalloc, L)
            fresh.check(rc, "predict_sparse_noalloc")
            assert fresh.workspace_bytes() == 0
            assert np.array_equal(act, L["ref_act"])
            assert max_rel_err(out, L["ref"]) <= TOL
        rc, out0, act0 = _call(fresh, fresh.lib.llg_hipd_ffn_predict_sparse, big)
        fresh.check(rc, "predict_sparse")
        assert fresh.workspace_bytes() > 0
        assert np.array_equal(act0, big["ref_act"]) and max_rel_err(out0, big["ref"]) <= TOL
    finally:
        fresh.close()


def test_noalloc_rejects_workload_above_scratch(dev):
    """d_ff 65536 at h 2048 needs 1024 partial rows of 2048 floats (8 MiB) beside
    the predictor's partials, more than the fixed scratch holds: the
    allocation-free entry point refuses the layer, the allocating one runs it."""
    h, ff, rank = 2048, 65536, 16
    g = torch.Generator(device="cuda")
    g.manual_seed(20261)
    up = gg.quantize(torch.randn((ff, h), generator=g, device="cuda") * 0.02, gg.Q4_0)
    dn = gg.quantize(torch.randn((ff, h), generator=g, device="cuda") * 0.02, gg.Q4_0)
    rng = np.random.default_rng(20261)
    wup = normal(rng, (rank, h), 0.05)
    wout = normal(rng, (ff, rank), 0.05)
    x = normal(rng, h, 1.0)
    _, lg = R.predict(wup, wout, None, x, 0.0)
    torch.cuda.synchronize()
    L = dict(h=h, ff=ff, x=x, thr=threshold_for(lg, 3000),
             pred=llg.Predictor(dev, wup, wout, None, 0.0),
             bundle=dev.upload_bundle(up, dn, gg.Q4_0, h, ff))
    rc, _, _ = _call(dev, dev.lib.llg_hipd_ffn_predict_sparse_noalloc, L)
    assert rc == llg.LLG_E_SCRATCH
    assert b"scratch" in dev.lib.llg_hip_last_error(dev.h)
    rc, out, act = _call(dev, dev.lib.llg_hipd_ffn_predict_sparse, L)
    dev.check(rc, "predict_sparse")
    ref_act, _ = R.predict(wup, wout, None, x, L["thr"])
    assert np.array_equal(act, ref_act)
    ref = R.ffn_sparse_load(up.cpu().numpy(), dn.cpu().numpy(), gg.Q4_0, h, ff, x, ref_act)
    assert max_rel_err(out, ref) <= TOL
    L["pred"].w_up.release()
    L["pred"].w_out.release()
    L["bundle"].release()
