"""model.Load (model/loader.go) for GGUF files, with the weights put in HBM.

load_hparams   loadHParams (loader.go:102-165): the same keys under the
               architecture prefix, the same fallbacks (vocab from the
               token_embd dims, head_count_kv = head_count, layer_norm_epsilon
               then layer_norm_rms_epsilon then 1e-5, context_length 2048,
               rope.freq_base 0 = no RoPE).
activation_for loader.go:54-61: falcon -> GELU; llama, mistral, qwen2, qwen3,
               qwen3moe -> SiLU; anything else -> ReLU.
load_falcon    build() + loadLayer() (loader.go:33-239) for the falcon
               architecture, straight into a FalconModel: the tensor names,
               must/try semantics and weight tying of output.weight to
               token_embd.weight are the reference's; Wq, Wk and Wv are
               joined row-wise into one device matrix.
write_falcon_gguf  the inverse, for synthetic models.

What the device model runs is ForwardFlash's falcon branch with the sparse
FFN on every layer (ffn_flash.go:115-185, path 2), so the loader also needs
what FlashContext gets from its caller: one predictor per layer (WUp
[rank x hidden], WOut [ff x rank], threshold).  The reference keeps these
outside the GGUF file (inference/predictor.go builds them in code); here they
are passed in, or read from optional extra tensors blk.N.ffn_pred_up.weight /
blk.N.ffn_pred_out.weight (F32) and the F32 array llg.predictor.thresholds,
which the reference's loader ignores.  The sparse FFN reads ffn_down by
neuron, so ffn_down must be stored transposed (dims [hidden, ff]), as the
reference's sparse path and CreateBundle require (flash/storage.go:277-281,
flash/bundle.go:40-48).  Layers with RMSNorm (no norm bias), attention
biases, q/k norms or MoE routers are rejected with an error.
"""
from __future__ import annotations

import numpy as np
import torch

from . import gguf as gg
from .gguf_file import (T_ARRAY, T_F32, T_STRING, T_U32, GGUFError, GGUFFile, open_gguf,
                        write_gguf)

ACT_RELU, ACT_GELU, ACT_SILU = gg.ACT_RELU, gg.ACT_GELU, gg.ACT_SILU


def activation_for(arch: str) -> int:
    if arch == "falcon":
        return ACT_GELU
    if arch in ("llama", "mistral", "qwen2", "qwen3", "qwen3moe"):
        return ACT_SILU
    return ACT_RELU


def load_hparams(gf: GGUFFile, arch: str) -> dict:
    """loadHParams (loader.go:102-165) as a dict."""
    p = arch + "."

    def opt_int(key, default):
        try:
            return gf.meta_int(p + key)
        except GGUFError:
            return default

    def opt_f32(key):
        try:
            return gf.meta_float32(p + key)
        except GGUFError:
            return None

    hp = {}
    try:
        hp["vocab"] = gf.meta_int(p + "vocab_size")
    except GGUFError:
        ti = gf.by_name.get("token_embd.weight")
        if ti is None:
            raise GGUFError("cannot determine vocab_size")
        hp["vocab"] = int(ti.dims[1])
    hp["hidden"] = gf.meta_int(p + "embedding_length")
    hp["ff"] = gf.meta_int(p + "feed_forward_length")
    hp["n_layers"] = gf.meta_int(p + "block_count")
    hp["n_heads"] = gf.meta_int(p + "attention.head_count")
    hp["n_kv"] = opt_int("attention.head_count_kv", hp["n_heads"])
    eps = opt_f32("attention.layer_norm_epsilon")
    if eps is None:
        eps = opt_f32("attention.layer_norm_rms_epsilon")
    hp["eps"] = 1e-5 if eps is None else eps
    rb = opt_f32("rope.freq_base")
    hp["rope_base"] = 0.0 if rb is None else rb
    hp["context_len"] = opt_int("context_length", 2048)
    hp["head_dim_k"] = opt_int("attention.key_length", 0)
    hp["head_dim_v"] = opt_int("attention.value_length", 0)
    hp["n_experts"] = opt_int("expert_count", 0)
    hp["n_experts_per_tok"] = opt_int("expert_used_count", 0)
    hp["expert_ff"] = opt_int("expert_feed_forward_length", 0)
    # HParams.HeadDim (model/model.go:32-37)
    hp["head_dim"] = hp["head_dim_k"] if hp["head_dim_k"] > 0 else hp["hidden"] // hp["n_heads"]
    return hp


def _f32_vec(gf: GGUFFile, name: str, n: int) -> np.ndarray:
    ti = gf.by_name[name]
    if ti.n_elements() != n:
        raise GGUFError(f"tensor {name!r}: {ti.n_elements()} elements, want {n}")
    raw = np.array(gf.tensor_bytes(ti))
    if ti.type == gg.F32:
        return raw.view("<f4").astype(np.float32)
    if ti.type == gg.F16:
        return raw.view("<f2").astype(np.float32)
    raise GGUFError(f"tensor {name!r}: norm vectors must be F32 or F16")


def _must(gf: GGUFFile, name: str):
    if name not in gf.by_name:
        raise GGUFError(f"tensor {name!r} not found in GGUF")
    return gf.by_name[name]


def _matrix(gf: GGUFFile, name: str, rows: int, cols: int):
    ti = _must(gf, name)
    if len(ti.dims) != 2 or int(ti.dims[0]) != cols or int(ti.dims[1]) != rows:
        raise GGUFError(f"tensor {name!r}: dims {ti.dims}, want [{cols}, {rows}]")
    if ti.type not in gg.DEVICE_TYPES:
        raise GGUFError(f"tensor {name!r}: type {ti.type} has no device path")
    return gf.tensor_rows(name), ti.type


def load_falcon(dev, path, predictors=None, thresholds=None, act: int | None = None,
                max_seq: int | None = None):
    """model.Load + the device FalconModel (see the module docstring).

    predictors: per layer (WUp [rank x hidden], WOut [ff x rank]) float32, or
    None to read them from the file; thresholds: per layer, or None to read
    llg.predictor.thresholds.  act: the FFN activation (default: the
    architecture's, GELU for falcon as loader.go:56 sets it).  max_seq: the KV
    cache length (default: the context length).  Returns (model, hparams).
    """
    from . import FalconModel

    gf = open_gguf(path)
    arch = gf.meta_string("general.architecture")
    if arch != "falcon":
        raise GGUFError(f"architecture {arch!r}: the device model runs the falcon layout only")
    hp = load_hparams(gf, arch)
    if hp["n_experts"] > 0:
        raise GGUFError("MoE falcon layers are not supported by the device model")
    h, nh, nkv, hd = hp["hidden"], hp["n_heads"], hp["n_kv"], hp["head_dim"]
    ff, V, L = hp["ff"], hp["vocab"], hp["n_layers"]
    embed, t_embed = _matrix(gf, "token_embd.weight", V, h)
    _must(gf, "output_norm.weight")
    if "output_norm.bias" not in gf.by_name:
        raise GGUFError("output_norm.bias missing: RMSNorm models are not supported")
    if "output.weight" in gf.by_name:
        lm_head, t_lm = _matrix(gf, "output.weight", V, h)
    else:
        lm_head, t_lm = embed, t_embed  # weight tying (loader.go:75-78)
    w = {"embed": embed, "lm_head": lm_head,
         "out_w": _f32_vec(gf, "output_norm.weight", h),
         "out_b": _f32_vec(gf, "output_norm.bias", h)}
    for k in ["norm_w", "norm_b", "wq", "wk", "wv", "wo", "pwup", "pwout", "up", "down_t"]:
        w[k] = []
    types = {"embed": t_embed, "lm_head": t_lm}
    for i in range(L):
        p = f"blk.{i}."
        _must(gf, p + "attn_norm.weight")
        if p + "attn_norm.bias" not in gf.by_name:
            raise GGUFError(f"{p}attn_norm.bias missing: RMSNorm models are not supported")
        for opt in ("attn_q.bias", "attn_k.bias", "attn_v.bias", "attn_output.bias",
                    "attn_q_norm.weight", "attn_k_norm.weight", "ffn_gate_inp.weight"):
            if p + opt in gf.by_name:
                raise GGUFError(f"tensor {p + opt!r} is not supported by the device model")
        _must(gf, p + "ffn_norm.weight")  # loaded by the reference, unused by falcon
        w["norm_w"].append(_f32_vec(gf, p + "attn_norm.weight", h))
        w["norm_b"].append(_f32_vec(gf, p + "attn_norm.bias", h))
        q, tq = _matrix(gf, p + "attn_q.weight", nh * hd, h)
        k, tk = _matrix(gf, p + "attn_k.weight", nkv * hd, h)
        v, tv = _matrix(gf, p + "attn_v.weight", nkv * hd, h)
        o, to = _matrix(gf, p + "attn_output.weight", h, nh * hd)
        up, tu = _matrix(gf, p + "ffn_up.weight", ff, h)
        dn, td = _matrix(gf, p + "ffn_down.weight", ff, h)  # transposed: rows = neurons
        if not tq == tk == tv:
            raise GGUFError(f"{p}attn_q/k/v: one type needed to join them")
        if tu != td:
            raise GGUFError(f"{p}ffn_up / ffn_down: one type needed for the bundle")
        for key, ty in (("wqkv", tq), ("wo", to), ("bundle", tu)):
            if types.setdefault(key, ty) != ty:
                raise GGUFError(f"{p}: the {key} type differs from layer 0's")
        w["wq"].append(q)
        w["wk"].append(k)
        w["wv"].append(v)
        w["wo"].append(o)
        w["up"].append(up)
        w["down_t"].append(dn)
        if predictors is None:
            pu = _must(gf, p + "ffn_pred_up.weight")
            rank = int(pu.dims[1])
            w["pwup"].append(np.array(gf.tensor_bytes(pu)).view("<f4").reshape(rank, h))
            po = _must(gf, p + "ffn_pred_out.weight")
            w["pwout"].append(np.array(gf.tensor_bytes(po)).view("<f4").reshape(ff, rank))
        else:
            w["pwup"].append(np.asarray(predictors[i][0], np.float32))
            w["pwout"].append(np.asarray(predictors[i][1], np.float32))
    if thresholds is None:
        mv = gf.meta.get("llg.predictor.thresholds")
        if mv is None:
            raise GGUFError("no predictor thresholds given or stored")
        thresholds = mv.value.values
    thresholds = np.asarray(thresholds, np.float32)
    if thresholds.size != L:
        raise GGUFError(f"{thresholds.size} thresholds for {L} layers")
    dims = dict(n_layers=L, hidden=h, n_heads=nh, n_kv=nkv, head_dim=hd, ff=ff, vocab=V,
                max_seq=max_seq or hp["context_len"], rope_base=hp["rope_base"], eps=hp["eps"])
    model = FalconModel(dev, dims, w, thresholds, t=types,
                        act=activation_for(arch) if act is None else act)
    return model, hp


def write_falcon_gguf(path, dims: dict, w: dict, t: int, thresholds=None,
                      context_len: int | None = None, with_predictors: bool = True,
                      tie_output: bool = False) -> None:
    """A falcon-architecture GGUF of the FalconModel weight dict `w` (GGUF row
    bytes of type t for the matrices, float32 norms and predictors)."""
    h, nh, nkv, hd = dims["hidden"], dims["n_heads"], dims["n_kv"], dims["head_dim"]
    ff, V, L = dims["ff"], dims["vocab"], dims["n_layers"]
    a = "falcon."
    meta = [("general.architecture", T_STRING, "falcon"),
            ("general.name", T_STRING, "synthetic-falcon"),
            (a + "embedding_length", T_U32, h), (a + "feed_forward_length", T_U32, ff),
            (a + "block_count", T_U32, L), (a + "attention.head_count", T_U32, nh),
            (a + "attention.head_count_kv", T_U32, nkv),
            (a + "attention.layer_norm_epsilon", T_F32, float(dims["eps"])),
            (a + "rope.freq_base", T_F32, float(dims["rope_base"])),
            (a + "context_length", T_U32, int(context_len or dims["max_seq"]))]
    if hd != h // nh:
        meta.append((a + "attention.key_length", T_U32, hd))
    if thresholds is not None:
        meta.append(("llg.predictor.thresholds", T_ARRAY,
                     (T_F32, [float(x) for x in np.asarray(thresholds, np.float32)])))
    f32 = lambda v: np.asarray(v, np.float32)
    ts = [("token_embd.weight", [h, V], t, w["embed"]),
          ("output_norm.weight", [h], gg.F32, f32(w["out_w"])),
          ("output_norm.bias", [h], gg.F32, f32(w["out_b"]))]
    if not tie_output:
        ts.append(("output.weight", [h, V], t, w["lm_head"]))
    for i in range(L):
        p = f"blk.{i}."
        ts += [(p + "attn_norm.weight", [h], gg.F32, f32(w["norm_w"][i])),
               (p + "attn_norm.bias", [h], gg.F32, f32(w["norm_b"][i])),
               (p + "attn_q.weight", [h, nh * hd], t, w["wq"][i]),
               (p + "attn_k.weight", [h, nkv * hd], t, w["wk"][i]),
               (p + "attn_v.weight", [h, nkv * hd], t, w["wv"][i]),
               (p + "attn_output.weight", [nh * hd, h], t, w["wo"][i]),
               (p + "ffn_norm.weight", [h], gg.F32, f32(w["norm_w"][i])),
               (p + "ffn_up.weight", [h, ff], t, w["up"][i]),
               (p + "ffn_down.weight", [h, ff], t, w["down_t"][i])]
        if with_predictors:
            r = np.asarray(w["pwup"][i]).shape[0]
            ts += [(p + "ffn_pred_up.weight", [h, r], gg.F32, f32(w["pwup"][i])),
                   (p + "ffn_pred_out.weight", [r, ff], gg.F32, f32(w["pwout"][i]))]
    write_gguf(path, meta, [(n, d, ty, _bytes(x)) for n, d, ty, x in ts])


def _bytes(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        x = x.contiguous().cpu().numpy()
    return np.ascontiguousarray(x).view(np.uint8).ravel()
