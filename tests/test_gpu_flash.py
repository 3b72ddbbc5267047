"""FlashFFN.ffn_flash (ffnFlash, ffn_flash.go:195-251) on the GPU: each path a
layer can take, against the oracle's restatement of the same path.

Bars: FFN outputs max |gpu - oracle| <= 1e-3 * max |oracle|.  The predictor's
threshold is set per token at the fp32 midpoint of the oracle's n-th and
(n+1)-th largest logit, so the GPU and the oracle select the same neurons.
"""
import numpy as np
import pytest

import llg
import llg.gguf as gg
from llg.flash import FlashFFN, FlashFFNConfig, FlashLayer, PredictorSet
from oracle import refcpu as R
from tests.helpers import max_rel_err, normal, quant, threshold_for

pytestmark = pytest.mark.gpu

TOL = 1e-3
H, FF, RANK, N_ACT = 256, 1024, 32, 100
D_MOE, EFF, E, K = 256, 128, 4, 2


def build(dev, rng, t, act_silu=False):
    """Layer 0 MoE; layers 1 and 2 dense-capable with bundles; layer 1 has a
    predictor.  Returns (device layers, host weights, predictor)."""
    host = {}
    router = normal(rng, (E, D_MOE), 0.2)
    gate_e = quant(normal(rng, (E * EFF, D_MOE), 0.02), t)
    up_e = quant(normal(rng, (E * EFF, D_MOE), 0.02), t)
    down_e = quant(normal(rng, (E * D_MOE, EFF), 0.02), t)
    host["moe"] = (router, gate_e, up_e, down_e)
    moe = (dev.upload_f32(router), dev.upload_matrix(gate_e, t, E * EFF, D_MOE),
           dev.upload_matrix(up_e, t, E * EFF, D_MOE), dev.upload_matrix(down_e, t, E * D_MOE, EFF),
           E, K)
    layers = [FlashLayer(moe=moe, ff=EFF)]
    for _ in range(2):
        up = quant(normal(rng, (FF, H), 0.02), t)
        down_t = quant(normal(rng, (FF, H), 0.02), t)        # sparse paths: [F rows x h]
        down = quant(normal(rng, (H, FF), 0.02), t)          # dense path: [h rows x F]
        gate = quant(normal(rng, (FF, H), 0.02), t)
        host.setdefault("dense", []).append((up, down_t, down, gate))
        layers.append(FlashLayer(bundle=dev.upload_bundle(up, down_t, t, H, FF),
                                 up=dev.upload_matrix(up, t, FF, H),
                                 down=dev.upload_matrix(down, t, H, FF),
                                 gate=dev.upload_matrix(gate, t, FF, H), ff=FF))
    wup = normal(rng, (RANK, H), 0.05)
    wout = normal(rng, (FF, RANK), 0.05)
    host["pred"] = (wup, wout)
    pred = llg.Predictor(dev, wup, wout, None, 0.0)
    return layers, host, pred


def set_threshold(pred, host, attn_out):
    wup, wout = host["pred"]
    _, lg = R.predict(wup, wout, None, attn_out, 0.0)
    pred.threshold = threshold_for(lg, N_ACT)
    act, _ = R.predict(wup, wout, None, attn_out, pred.threshold)
    assert act.size == N_ACT
    return act


@pytest.mark.parametrize("t", [gg.Q4_0, gg.Q8_0, gg.F16, gg.F32])
def test_paths_without_window(dev, rng, t):
    layers, host, pred = build(dev, rng, t)
    ffn = FlashFFN(dev, layers, FlashFFNConfig(predictors=PredictorSet([None, pred])))
    # path 0: MoE
    x = normal(rng, D_MOE, 1.0)
    got = ffn.ffn_flash(0, x, x)
    router, g, u, d = host["moe"]
    exp, _, _ = R.moe_ffn(router, g, u, d, t, D_MOE, EFF, E, K, x)
    assert ffn.last_path == 0 and max_rel_err(got, exp) <= TOL
    # path 2: predictor + sparse load over the bundle
    x, a = normal(rng, H, 1.0), normal(rng, H, 1.0)
    active = set_threshold(pred, host, a)
    got = ffn.ffn_flash(1, x, a)
    up, down_t, _, _ = host["dense"][0]
    exp = R.ffn_sparse_load(up, down_t, t, H, FF, x, active)
    assert ffn.last_path == 2 and max_rel_err(got, exp) <= TOL
    # path 3: dense (layer 2 has no predictor)
    got = ffn.ffn_flash(2, x, a)
    up, _, down, _ = host["dense"][1]
    exp = R.ffn_dense(up, down, t, H, FF, x)
    assert ffn.last_path == 3 and max_rel_err(got, exp) <= TOL


def test_dense_swiglu_for_silu_models(dev, rng):
    t = gg.Q4_0
    layers, host, pred = build(dev, rng, t)
    ffn = FlashFFN(dev, layers, FlashFFNConfig(), activation=gg.ACT_SILU)
    x = normal(rng, H, 1.0)
    got = ffn.ffn_flash(2, x, x)
    up, _, down, gate = host["dense"][1]
    assert ffn.last_path == 3
    assert max_rel_err(got, R.ffn_swiglu(gate, up, down, t, H, FF, x)) <= TOL


def test_window_path(dev, rng):
    """Path 1 over 12 tokens: layer 1 with its predictor, layer 2 with every
    neuron active (no predictor), against the oracle's NeuronCache."""
    t, k = gg.Q4_0, 3
    layers, host, pred = build(dev, rng, t)
    ffn = FlashFFN(dev, layers, FlashFFNConfig(window_size=k, predictors=PredictorSet([None, pred])))
    assert ffn.caches[0] is None and ffn.caches[1] is not None and ffn.caches[2] is not None
    refs = [R.NeuronCache(FF, H, k, FF, host["dense"][i][0], host["dense"][i][1], t)
            for i in range(2)]
    for tok in range(12):
        x, a = normal(rng, H, 1.0), normal(rng, H, 1.0)
        active = set_threshold(pred, host, a)
        got = ffn.ffn_flash(1, x, a)
        assert ffn.last_path == 1
        refs[0].update(active)
        assert max_rel_err(got, refs[0].ffn_forward(x, active)) <= TOL, tok
        assert np.array_equal(ffn.caches[1].resident(), refs[0].resident()), tok
        got = ffn.ffn_flash(2, x, a)
        every = np.arange(FF, dtype=np.int32)
        refs[1].update(every)
        assert max_rel_err(got, refs[1].ffn_forward(x, every)) <= TOL, tok
    assert ffn.caches[2].num_cached() == FF
