"""Synthetic data and float64 brute-force references shared by the tests."""
from __future__ import annotations

import numpy as np
import torch

import llg.gguf as gg


def normal(rng: np.random.Generator, shape, std: float) -> np.ndarray:
    return (rng.standard_normal(shape) * std).astype(np.float32)


def quant(w: np.ndarray, t: int) -> np.ndarray:
    """fp32 [rows x cols] -> GGUF bytes uint8 [rows x ByteSize(cols)]."""
    return gg.quantize(torch.from_numpy(np.ascontiguousarray(w)), t).numpy()


def deq(raw: np.ndarray, t: int, cols: int) -> np.ndarray:
    return gg.dequantize_torch(torch.from_numpy(np.ascontiguousarray(raw)), t, cols).numpy()


def make_sparse_layer(rng, h: int, ff: int, t: int, std: float = 0.02):
    """Config-0 style layer: ffn_up [ff x h] and ffn_down stored [ff x h] (W_down^T)."""
    up = normal(rng, (ff, h), std)
    down_t = normal(rng, (ff, h), std)
    return quant(up, t), quant(down_t, t)


def ref_sparse_f64(up_raw, down_t_raw, t, h, x, active, act=gg.ACT_RELU) -> np.ndarray:
    """float64 sparse FFN over the exactly dequantized rows."""
    up = deq(up_raw[active], t, h).astype(np.float64)
    dn = deq(down_t_raw[active], t, h).astype(np.float64)
    u = up @ x.astype(np.float64)
    u = act_f64(act, u)
    return (u[:, None] * dn).sum(axis=0)


def act_f64(act: int, u: np.ndarray) -> np.ndarray:
    if act == gg.ACT_SILU:
        return u / (1.0 + np.exp(-u))
    if act == gg.ACT_GELU:
        c = 0.7978845608028654
        return 0.5 * u * (1.0 + np.tanh(c * (u + 0.044715 * u ** 3)))
    return np.where(u < 0, 0.0, u)


def max_rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| / max |ref| (the 1e-3 output tolerance's measure)."""
    den = float(np.max(np.abs(ref)))
    return float(np.max(np.abs(got.astype(np.float64) - ref))) / (den if den > 0 else 1.0)


def threshold_for(logits: np.ndarray, n_active: int) -> float:
    """fp32 midpoint of the n-th and (n+1)-th largest logit: exactly n_active
    logits lie strictly above it, with a gap far above fp32 reordering error."""
    s = np.sort(logits.astype(np.float32))[::-1]
    return float(np.float32((np.float64(s[n_active - 1]) + np.float64(s[n_active])) / 2))


def window_sets(rng, ff: int, n_active: int, steps: int, carry: float):
    """Active sets for the sliding-window workload: each token keeps
    round(carry * n) of the previous set and draws the rest uniformly from
    its complement; every set is sorted ascending."""
    keep = int(round(carry * n_active))
    sets = [np.sort(rng.choice(ff, n_active, replace=False)).astype(np.int32)]
    for _ in range(steps - 1):
        prev = sets[-1]
        kept = rng.choice(prev, keep, replace=False)
        comp = np.setdiff1d(np.arange(ff), prev)
        new = rng.choice(comp, n_active - keep, replace=False)
        sets.append(np.sort(np.concatenate([kept, new])).astype(np.int32))
    return sets
