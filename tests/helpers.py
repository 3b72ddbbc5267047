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


# ---------------------------------------------------------------- Falcon decode
def make_falcon(rng, d: dict, t: int = gg.Q4_0, std: float = 0.05) -> dict:
    """Random Falcon-layout weights (GGUF bytes for the matrices, f32 for the
    norms and predictors); the norms are random so that weight and bias count.
    `std`: the attention and FFN matrices are N(0, std)."""
    h, nh, nkv, hd, ff = d["hidden"], d["n_heads"], d["n_kv"], d["head_dim"], d["ff"]
    V, r, L = d["vocab"], d["rank"], d["n_layers"]
    w = {"embed": quant(normal(rng, (V, h), 0.5), t), "lm_head": quant(normal(rng, (V, h), 0.05), t),
         "out_w": 1.0 + normal(rng, h, 0.1), "out_b": normal(rng, h, 0.1)}
    for k in ["norm_w", "norm_b", "wq", "wk", "wv", "wo", "pwup", "pwout", "up", "down_t"]:
        w[k] = []
    for _ in range(L):
        w["norm_w"].append(1.0 + normal(rng, h, 0.1))
        w["norm_b"].append(normal(rng, h, 0.1))
        w["wq"].append(quant(normal(rng, (nh * hd, h), std), t))
        w["wk"].append(quant(normal(rng, (nkv * hd, h), std), t))
        w["wv"].append(quant(normal(rng, (nkv * hd, h), std), t))
        w["wo"].append(quant(normal(rng, (h, nh * hd), std), t))
        w["pwup"].append(normal(rng, (r, h), 0.05))
        w["pwout"].append(normal(rng, (ff, r), 0.05))
        w["up"].append(quant(normal(rng, (ff, h), std), t))
        w["down_t"].append(quant(normal(rng, (ff, h), std), t))
    return w


def make_falcon_gpu(seed: int, d: dict, t: int = gg.Q4_0, std: float = 0.02) -> dict:
    """make_falcon's layout at full-model sizes, drawn and quantized on the GPU
    (torch CUDA tensors for the matrices and predictors; host f32 for the
    norms, which are random so that weight and bias count)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    rng = np.random.default_rng(seed)
    h, nh, nkv, hd, ff = d["hidden"], d["n_heads"], d["n_kv"], d["head_dim"], d["ff"]
    V, r, L = d["vocab"], d["rank"], d["n_layers"]

    def rnd(rows, cols, sd):
        return torch.randn((rows, cols), generator=g, device="cuda", dtype=torch.float32) * sd

    def q(rows, cols):
        return gg.quantize(rnd(rows, cols, std), t)

    w = {"embed": q(V, h), "lm_head": q(V, h),
         "out_w": 1.0 + normal(rng, h, 0.1), "out_b": normal(rng, h, 0.1)}
    for k in ["norm_w", "norm_b", "wq", "wk", "wv", "wo", "pwup", "pwout", "up", "down_t"]:
        w[k] = []
    for _ in range(L):
        w["norm_w"].append(1.0 + normal(rng, h, 0.1))
        w["norm_b"].append(normal(rng, h, 0.1))
        w["wq"].append(q(nh * hd, h))
        w["wk"].append(q(nkv * hd, h))
        w["wv"].append(q(nkv * hd, h))
        w["wo"].append(q(h, nh * hd))
        w["pwup"].append(rnd(r, h, 0.05).contiguous())
        w["pwout"].append(rnd(ff, r, 0.05).contiguous())
        w["up"].append(q(ff, h))
        w["down_t"].append(q(ff, h))
    return w


def to_host(w: dict) -> dict:
    """The same weights as host numpy arrays (for the oracle)."""
    def h(a):
        return a.cpu().numpy() if hasattr(a, "is_cuda") else np.asarray(a)
    return {k: ([h(x) for x in v] if isinstance(v, list) else h(v)) for k, v in w.items()}


def _gap_threshold(lg: np.ndarray, frac: float) -> float:
    """A float32 threshold near the (1-frac) quantile of lg, at the midpoint of
    the widest gap between neighbouring values there (so selection does not
    depend on fp32 rounding)."""
    s = np.sort(lg.ravel())
    n = s.size
    c = int((1.0 - frac) * n)
    lo, hi = max(1, c - n // 20), min(n - 1, c + n // 20)
    gaps = s[lo:hi + 1] - s[lo - 1:hi]
    i = lo + int(np.argmax(gaps))
    return float(np.float32((s[i - 1] + s[i]) / 2))


def ref_falcon_f64(w: dict, d: dict, tokens, frac: float = 0.1, t: int = gg.Q4_0,
                   pred_logits: bool = False):
    """float64 ForwardFlash over a token sequence (positions 0..T-1), layer by
    layer over all tokens; each layer's threshold is picked at a wide gap of its
    predictor logits.  Returns (logits [T x V], n_active [T x L], thresholds),
    and with pred_logits also the predictor logits [T x L x ff]."""
    h, nh, nkv, hd, ff = d["hidden"], d["n_heads"], d["n_kv"], d["head_dim"], d["ff"]
    L, eps, base = d["n_layers"], d["eps"], d["rope_base"]
    dq = lambda raw, cols: deq(raw, t, cols).astype(np.float64)
    tokens = np.asarray(tokens)
    T = tokens.size
    X = dq(w["embed"], h)[tokens]

    def ln(Z, g, b):
        mu = Z.mean(1, keepdims=True)
        var = ((Z - mu) ** 2).mean(1, keepdims=True)
        return (Z - mu) / np.sqrt(var + eps) * g.astype(np.float64) + b.astype(np.float64)

    def rope(M, nheads):
        if not base > 0:  # forward.go:249: no RoPE
            return M.reshape(T, nheads, hd).copy()
        M = M.reshape(T, nheads, hd).copy()
        half = hd // 2
        i = np.arange(half)
        for s in range(T):
            fr = s / np.power(float(base), 2.0 * i / hd)
            c, sn = np.cos(fr), np.sin(fr)
            x0, x1 = M[s, :, :half].copy(), M[s, :, half:].copy()
            M[s, :, :half] = x0 * c - x1 * sn
            M[s, :, half:] = x0 * sn + x1 * c
        return M

    thr, nact, plg = [], np.zeros((T, L), np.int64), []
    for l in range(L):
        N = ln(X, w["norm_w"][l], w["norm_b"][l])
        Q = rope(N @ dq(w["wq"][l], h).T, nh)
        K = rope(N @ dq(w["wk"][l], h).T, nkv)
        Vv = (N @ dq(w["wv"][l], h).T).reshape(T, nkv, hd)
        att = np.zeros((T, nh, hd))
        for s in range(T):
            for head in range(nh):
                kvh = head * nkv // nh
                sc = K[:s + 1, kvh] @ Q[s, head] / np.sqrt(hd)
                p = np.exp(sc - sc.max())
                p /= p.sum()
                att[s, head] = p @ Vv[:s + 1, kvh]
        A = att.reshape(T, nh * hd) @ dq(w["wo"][l], nh * hd).T
        lg = np.maximum(A @ w["pwup"][l].T.astype(np.float64), 0.0) @ w["pwout"][l].T.astype(np.float64)
        plg.append(lg)
        th = _gap_threshold(lg, frac)
        thr.append(th)
        on = lg > th
        nact[:, l] = on.sum(1)
        U = np.maximum(N @ dq(w["up"][l], h).T, 0.0) * on
        X = X + A + U @ dq(w["down_t"][l], h)
    out = ln(X, w["out_w"], w["out_b"]) @ dq(w["lm_head"], h).T
    if pred_logits:
        return out, nact, np.array(thr, np.float32), np.stack(plg, 1)
    return out, nact, np.array(thr, np.float32)
