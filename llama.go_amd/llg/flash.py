"""The FFN routing of inference.FlashContext (ffn_flash.go:14-101, 195-251)
over device objects: PredictorSet, FlashFFNConfig and FlashFFN.ffn_flash,
which takes a layer down the reference's paths in its order (MoE, then the
sliding window, then predictor + sparse load, then dense).

Every path computes on the GPU through the C ABI (llg.moe_ffn,
llg.NeuronCache, llg.ffn_predict_sparse, llg.ffn_dense, llg.ffn_swiglu);
this module only routes, as ffnFlash does.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import gguf as gg


class PredictorSet:
    """inference.PredictorSet (predictor.go:86-114): one Predictor per layer;
    None means dense (all neurons active)."""

    def __init__(self, predictors):
        self.predictors = list(predictors)

    @classmethod
    def dense(cls, n_layers: int) -> "PredictorSet":
        """NewDensePredictorSet (predictor.go:92-97): every layer dense."""
        return cls([None] * n_layers)

    def get(self, layer_idx: int):
        """Get (predictor.go:109-114): None past the end."""
        if layer_idx >= len(self.predictors):
            return None
        return self.predictors[layer_idx]


@dataclass
class FlashFFNConfig:
    """FlashFFNConfig (ffn_flash.go:14-36).  n_threads is the row-read pool of
    the reference's SSD tier; the rows here are resident in HBM, so it is kept
    for the interface only."""
    window_size: int = 0
    predictors: PredictorSet | None = None
    n_threads: int = 32


@dataclass
class FlashLayer:
    """The FFN descriptors of model.Layer (model.go:45-84) as device handles.

    bundle: the bundled up/down rows (sparse and window paths); up/down (and
    gate for SwiGLU): the dense matrices (dense path); moe: (router, gate_exps,
    up_exps, down_exps, n_exp, k) for a MoE layer."""
    bundle: object = None
    up: object = None
    down: object = None
    gate: object = None
    moe: tuple | None = None
    ff: int = 0


@dataclass
class FlashFFN:
    """FlashContext's FFN part (NewFlashContext, ffnFlash, predictActive).

    activation: model.Activation (ACT_RELU, ACT_GELU or ACT_SILU), which picks
    the sparse paths' activation (activationFn, ffn_flash.go:303-312) and the
    dense path's form (Context.ffn, forward.go:318-340)."""
    dev: object
    layers: list
    cfg: FlashFFNConfig
    activation: int = gg.ACT_RELU
    caches: list = field(default_factory=list)
    last_path: int = -1  # the path the last ffn_flash call took (0-3)

    def __post_init__(self):
        from . import NeuronCache

        # ffn_flash.go:58-83: a cache per layer with a bundle when windowing is
        # on; MoE layers and layers without FFN rows get none.  The capacity
        # hint of the reference (F * k / 5, at least 256) is not needed: the
        # device window holds every neuron of the layer.
        self.caches = [None] * len(self.layers)
        if self.cfg.window_size > 0:
            for i, layer in enumerate(self.layers):
                if layer.moe is not None or layer.bundle is None:
                    continue
                self.caches[i] = NeuronCache(self.dev, layer.bundle, self.cfg.window_size)

    def predict_active(self, layer_idx: int, attn_out) -> np.ndarray:
        """predictActive (ffn_flash.go:239-251): all neurons 0..F-1 without a
        predictor, else Predict(attn_out)."""
        ps = self.cfg.predictors
        pred = ps.get(layer_idx) if ps is not None else None
        if pred is None:
            return np.arange(self.layers[layer_idx].ff, dtype=np.int32)
        return pred.predict(attn_out)

    def ffn_flash(self, layer_idx: int, x, attn_out) -> np.ndarray:
        """ffnFlash (ffn_flash.go:195-237) for one token."""
        from . import ffn_dense, ffn_predict_sparse, ffn_swiglu, moe_ffn

        layer = self.layers[layer_idx]
        if layer.moe is not None:  # path 0
            self.last_path = 0
            router, gate, up, down, n_exp, k = layer.moe
            return moe_ffn(self.dev, router, gate, up, down, n_exp, k, x)[0]
        cache = self.caches[layer_idx] if layer_idx < len(self.caches) else None
        if self.cfg.window_size > 0 and cache is not None:  # path 1
            self.last_path = 1
            active = self.predict_active(layer_idx, attn_out)
            cache.update(active)
            return cache.ffn_forward(x, active, self.activation)
        ps = self.cfg.predictors
        if ps is not None and ps.get(layer_idx) is not None:  # path 2
            self.last_path = 2
            out, _ = ffn_predict_sparse(self.dev, ps.get(layer_idx), layer.bundle, attn_out, x,
                                        self.activation)
            return out
        self.last_path = 3  # path 3: Context.ffn (forward.go:318-340)
        if self.activation == gg.ACT_SILU:
            return ffn_swiglu(self.dev, layer.gate, layer.up, layer.down, x)
        return ffn_dense(self.dev, layer.up, layer.down, x, self.activation)
