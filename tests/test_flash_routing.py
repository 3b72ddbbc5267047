"""FlashFFN's routing (ffnFlash, ffn_flash.go:195-251; NewFlashContext's
caches, :58-83; PredictorSet, predictor.go:86-114) on the CPU: the device
calls are replaced by recorders, so these tests check which path a layer
takes and with what arguments, not the arithmetic (the GPU tests do that)."""
import numpy as np
import pytest

import llg
import llg.gguf as gg
from llg.flash import FlashFFN, FlashFFNConfig, FlashLayer, PredictorSet


class FakePredictor:
    def __init__(self, active):
        self.active = np.asarray(active, np.int32)
        self.calls = []

    def predict(self, attn_out):
        self.calls.append(np.asarray(attn_out))
        return self.active


class FakeCache:
    made = []

    def __init__(self, dev, bundle, k):
        self.bundle, self.k, self.updates, self.ffns = bundle, k, [], []
        FakeCache.made.append(self)

    def update(self, active):
        self.updates.append(np.asarray(active))
        return 0

    def ffn_forward(self, x, active, act):
        self.ffns.append((np.asarray(active), act))
        return np.full(4, 1.0, np.float32)


@pytest.fixture
def calls(monkeypatch):
    log = []
    FakeCache.made = []
    monkeypatch.setattr(llg, "NeuronCache", FakeCache)
    monkeypatch.setattr(llg, "moe_ffn", lambda dev, *a: (log.append(("moe", a)) or
                                                         (np.zeros(4, np.float32), None, None)))
    monkeypatch.setattr(llg, "ffn_predict_sparse", lambda dev, pred, b, a, x, act: (
        log.append(("sparse", pred, b, act)) or (np.full(4, 2.0, np.float32), None)))
    monkeypatch.setattr(llg, "ffn_dense", lambda dev, up, down, x, act: (
        log.append(("dense", up, down, act)) or np.full(4, 3.0, np.float32)))
    monkeypatch.setattr(llg, "ffn_swiglu", lambda dev, g, up, down, x: (
        log.append(("swiglu", g, up, down)) or np.full(4, 4.0, np.float32)))
    return log


def layers():
    moe = FlashLayer(moe=("router", "gate", "up", "down", 8, 2), ff=16)
    sparse = FlashLayer(bundle="b1", up="u1", down="d1", gate="g1", ff=16)
    plain = FlashLayer(bundle="b2", up="u2", down="d2", gate="g2", ff=16)
    no_rows = FlashLayer(up="u3", down="d3", ff=16)
    return [moe, sparse, plain, no_rows]


def test_predictor_set_get():
    p = object()
    ps = PredictorSet([None, p])
    assert ps.get(0) is None and ps.get(1) is p
    assert ps.get(2) is None and ps.get(100) is None  # past the end: dense
    assert PredictorSet.dense(3).predictors == [None, None, None]


def test_paths_without_window(calls):
    pred = FakePredictor([1, 5])
    ffn = FlashFFN(None, layers(), FlashFFNConfig(predictors=PredictorSet([pred, pred, None])))
    x, a = np.zeros(4, np.float32), np.ones(4, np.float32)
    assert ffn.caches == [None] * 4  # no window: no caches
    ffn.ffn_flash(0, x, a)
    assert ffn.last_path == 0 and calls[-1][0] == "moe"  # MoE first, predictor or not
    out = ffn.ffn_flash(1, x, a)
    assert ffn.last_path == 2 and calls[-1] == ("sparse", pred, "b1", gg.ACT_RELU)
    assert out[0] == 2.0
    ffn.ffn_flash(2, x, a)  # no predictor for the layer: dense
    assert ffn.last_path == 3 and calls[-1] == ("dense", "u2", "d2", gg.ACT_RELU)
    ffn.ffn_flash(3, x, a)  # past the set's end: dense
    assert ffn.last_path == 3 and calls[-1] == ("dense", "u3", "d3", gg.ACT_RELU)


@pytest.mark.parametrize("act,kind", [(gg.ACT_GELU, "dense"), (gg.ACT_SILU, "swiglu")])
def test_dense_form_by_activation(calls, act, kind):
    ffn = FlashFFN(None, layers(), FlashFFNConfig(), activation=act)
    ffn.ffn_flash(2, np.zeros(4, np.float32), np.zeros(4, np.float32))
    assert calls[-1][0] == kind
    if kind == "dense":
        assert calls[-1][3] == gg.ACT_GELU
    else:
        assert calls[-1][1:] == ("g2", "u2", "d2")


def test_window_path_and_caches(calls):
    pred = FakePredictor([3, 4, 9])
    ps = PredictorSet([None, pred, None, None])
    ffn = FlashFFN(None, layers(), FlashFFNConfig(window_size=5, predictors=ps),
                   activation=gg.ACT_SILU)
    # a cache per layer with rows, none for MoE or row-less layers
    assert [c is not None for c in ffn.caches] == [False, True, True, False]
    assert [c.bundle for c in FakeCache.made] == ["b1", "b2"] and FakeCache.made[0].k == 5
    x, a = np.zeros(4, np.float32), np.arange(4, dtype=np.float32)
    ffn.ffn_flash(0, x, a)
    assert ffn.last_path == 0  # MoE before the window
    ffn.ffn_flash(1, x, a)
    assert ffn.last_path == 1
    c = ffn.caches[1]
    assert c.updates[-1].tolist() == [3, 4, 9] and pred.calls[-1].tolist() == [0, 1, 2, 3]
    assert c.ffns[-1][0].tolist() == [3, 4, 9] and c.ffns[-1][1] == gg.ACT_SILU
    ffn.ffn_flash(2, x, a)  # window without a predictor: every neuron active
    assert ffn.last_path == 1
    assert ffn.caches[2].updates[-1].tolist() == list(range(16))
    ffn.ffn_flash(3, x, a)  # no rows to cache: dense (SwiGLU for SiLU)
    assert ffn.last_path == 3 and calls[-1][0] == "swiglu"


def test_predict_active_all_without_predictor():
    ffn = FlashFFN(None, layers(), FlashFFNConfig(predictors=None))
    assert ffn.predict_active(1, np.zeros(4)).tolist() == list(range(16))
