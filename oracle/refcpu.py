"""ctypes wrapper of the CPU oracle oracle/librefcpu.so (oracle/refcpu.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.  Each function
names the reference file:line restated by the C function it calls.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

import os

HERE = Path(__file__).resolve().parent
# REFCPU_LIB selects another build of the same source (the sanitizer builds of
# oracle/Makefile, loaded by oracle/sanitize.sh)
LIB_PATH = Path(os.environ.get("REFCPU_LIB", HERE / "librefcpu.so"))

F32, F16, Q4_0, Q8_0 = 0, 1, 2, 8
ACT_RELU, ACT_GELU, ACT_SILU = 0, 1, 2

_vp = C.c_void_p
_SIGS = {
    "refcpu_byte_size": (C.c_int64, [C.c_int, C.c_int64]),
    "refcpu_f16_to_f32": (C.c_float, [C.c_uint16]),
    "refcpu_dequantize": (C.c_int64, [_vp, C.c_int64, C.c_int, _vp]),
    "refcpu_matmulvec": (None, [_vp, C.c_int, C.c_int, _vp, _vp]),
    "refcpu_set_threads": (None, [C.c_int]),
    "refcpu_activation": (None, [C.c_int, _vp, C.c_int]),
    "refcpu_rmsnorm": (None, [_vp, _vp, _vp, C.c_int, C.c_float]),
    "refcpu_layernorm": (None, [_vp, _vp, _vp, _vp, C.c_int, C.c_float]),
    "refcpu_softmax_inplace": (None, [_vp, C.c_int]),
    "refcpu_select": (C.c_int, [_vp, C.c_int, C.c_float, _vp]),
    "refcpu_predict": (C.c_int, [_vp, _vp, _vp, C.c_int, C.c_int, C.c_int, _vp, C.c_float, _vp,
                                 _vp]),
    "refcpu_read_rows": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, _vp, C.c_int, _vp]),
    "refcpu_ffn_sparse_load": (C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp, _vp, C.c_int,
                                         C.c_int, _vp]),
    "refcpu_read_rows_file": (C.c_int, [C.c_char_p, C.c_int64, C.c_int, C.c_int, C.c_int, _vp,
                                        C.c_int, C.c_int, _vp]),
    "refcpu_ffn_sparse_load_file": (C.c_int, [C.c_char_p, C.c_int64, C.c_int64, C.c_int, C.c_int,
                                              C.c_int, _vp, _vp, C.c_int, C.c_int, C.c_int,
                                              _vp]),
    "refcpu_nc_new_file": (_vp, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_char_p, C.c_int64,
                                 C.c_int64, C.c_int, C.c_int]),
    "refcpu_ffn_dense": (C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp, C.c_int, _vp]),
    "refcpu_ffn_swiglu": (C.c_int, [_vp, _vp, _vp, C.c_int, C.c_int, C.c_int, _vp, _vp]),
    "refcpu_nc_new": (_vp, [C.c_int, C.c_int, C.c_int, C.c_int, _vp, _vp, C.c_int]),
    "refcpu_nc_free": (None, [_vp]),
    "refcpu_nc_update": (C.c_int, [_vp, _vp, C.c_int, _vp, _vp]),
    "refcpu_nc_ffn_forward": (C.c_int, [_vp, _vp, _vp, C.c_int, C.c_int, _vp]),
    "refcpu_nc_num_cached": (C.c_int, [_vp]),
    "refcpu_nc_is_cached": (C.c_int, [_vp, C.c_int]),
    "refcpu_moe_ffn": (C.c_int, [_vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                 _vp, _vp, _vp, _vp]),
    "refcpu_moe_route": (C.c_int, [_vp, C.c_int, C.c_int, _vp, _vp]),
}

_lib = None


def build() -> Path:
    """Compile the oracle with its Makefile (gcc -O2 -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(_vp) if a is not None else None


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    if hasattr(a, "numpy"):
        a = a.contiguous().cpu().numpy()
    return np.ascontiguousarray(a).view(np.uint8).ravel()


def set_threads(n: int) -> None:
    """Row threads of the oracle's MatMulVec (1 = the reference's single
    goroutine, the default and what the CPU baseline uses).  Every row keeps
    its sequential sum, so any n gives bit-identical results."""
    lib().refcpu_set_threads(int(n))


def byte_size(t: int, n: int) -> int:
    """gguf/types.go:90-102 (-1 on error)."""
    return int(lib().refcpu_byte_size(t, n))


def f16_to_f32(h: int) -> float:
    """tensor/dtype.go:417-443."""
    return float(lib().refcpu_f16_to_f32(h))


def f16_to_f32_bits(h: int) -> int:
    v = np.array([lib().refcpu_f16_to_f32(h)], np.float32)
    return int(v.view(np.uint32)[0])


def dequantize(raw, t: int) -> np.ndarray:
    """tensor/dtype.go:249-268 (Dequantize)."""
    r = _u8(raw)
    bs = {F32: 4, F16: 2, Q4_0: 18, Q8_0: 34}[t]
    per = {F32: 1, F16: 1, Q4_0: 32, Q8_0: 32}[t]
    out = np.empty(max(r.size // bs * per, 1), np.float32)
    n = lib().refcpu_dequantize(_p(r), r.size, t, _p(out))
    if n < 0:
        raise ValueError("dequantize: bad length or type")
    return out[:n]


def matmulvec(w, x) -> np.ndarray:
    """tensor/ops.go:39-60."""
    w, x = _f32(w), _f32(x).ravel()
    y = np.empty(w.shape[0], np.float32)
    lib().refcpu_matmulvec(_p(w), w.shape[0], w.shape[1], _p(x), _p(y))
    return y


def activation(act: int, x) -> np.ndarray:
    """ffn_flash.go:303-312 -> ops.go:168-189."""
    x = _f32(x).copy().ravel()
    lib().refcpu_activation(act, _p(x), x.size)
    return x


def rmsnorm(x, w, eps: float) -> np.ndarray:
    """tensor/ops.go:114-135."""
    x, w = _f32(x).ravel(), _f32(w).ravel()
    out = np.empty_like(x)
    lib().refcpu_rmsnorm(_p(x), _p(w), _p(out), x.size, eps)
    return out


def layernorm(x, w, b, eps: float) -> np.ndarray:
    """tensor/ops.go:138-165."""
    x, w, b = _f32(x).ravel(), _f32(w).ravel(), _f32(b).ravel()
    out = np.empty_like(x)
    lib().refcpu_layernorm(_p(x), _p(w), _p(b), _p(out), x.size, eps)
    return out


def softmax(v) -> np.ndarray:
    """inference/forward.go:463-479."""
    v = _f32(v).copy().ravel()
    lib().refcpu_softmax_inplace(_p(v), v.size)
    return v


def select(logits, thr: float) -> np.ndarray:
    """inference/predictor.go:76-82."""
    lg = _f32(logits).ravel()
    act = np.empty(max(lg.size, 1), np.int32)
    n = lib().refcpu_select(_p(lg), lg.size, thr, _p(act))
    return act[:n].copy()


def predict(w_up, w_out, bias, a, thr: float):
    """inference/predictor.go:51-83 -> (active, logits)."""
    w_up, w_out, a = _f32(w_up), _f32(w_out), _f32(a).ravel()
    b = _f32(bias).ravel() if bias is not None else None
    rank, h = w_up.shape
    ff = w_out.shape[0]
    act = np.empty(ff, np.int32)
    logits = np.empty(ff, np.float32)
    n = lib().refcpu_predict(_p(w_up), _p(w_out), _p(b), h, rank, ff, _p(a), thr, _p(act),
                             _p(logits))
    if n < 0:
        raise ValueError("predictor: weights not loaded")
    return act[:n].copy(), logits


def read_rows(raw, t: int, in_dim: int, out_dim: int, rows) -> np.ndarray:
    """flash/storage.go:246-319 (row addressing + per-row dequant)."""
    r = _u8(raw)
    rows = np.ascontiguousarray(rows, np.int32)
    out = np.empty((rows.size, in_dim), np.float32)
    rc = lib().refcpu_read_rows(_p(r), t, in_dim, out_dim, _p(rows), rows.size, _p(out))
    if rc == -2:
        raise IndexError("row out of range")
    if rc:
        raise ValueError("read_rows: bad type/length")
    return out


def ffn_sparse_load(up_raw, down_t_raw, t: int, h: int, ff: int, x, active,
                    act: int = ACT_RELU) -> np.ndarray:
    """inference/ffn_flash.go:254-299."""
    u, dn = _u8(up_raw), _u8(down_t_raw)
    x = _f32(x).ravel()
    a = np.ascontiguousarray(active, np.int32)
    out = np.empty(h, np.float32)
    rc = lib().refcpu_ffn_sparse_load(_p(u), _p(dn), t, h, ff, _p(x), _p(a), a.size, act,
                                      _p(out))
    if rc:
        raise ValueError(f"ffn_sparse_load rc={rc}")
    return out


_FILE_ERRORS = {-1: "bad type/length", -2: "row out of range", -3: "open failed",
                -4: "short read"}


def read_rows_file(path, tensor_offset: int, t: int, in_dim: int, out_dim: int, rows,
                   nthreads: int = 32) -> np.ndarray:
    """flash/storage.go:246-319 ReadRowsParallel: rows of the tensor at byte
    offset tensor_offset of the file, read by nthreads threads with pread."""
    r = np.ascontiguousarray(rows, np.int32)
    out = np.empty((r.size, in_dim), np.float32)
    rc = lib().refcpu_read_rows_file(str(path).encode(), tensor_offset, t, in_dim, out_dim,
                                     _p(r), r.size, nthreads, _p(out))
    if rc == -2:
        raise IndexError("row out of range")
    if rc:
        raise OSError(f"read_rows_file: {_FILE_ERRORS.get(rc, rc)}")
    return out


def ffn_sparse_load_file(path, up_offset: int, down_t_offset: int, t: int, h: int, ff: int, x,
                         active, act: int = ACT_RELU, nthreads: int = 32) -> np.ndarray:
    """inference/ffn_flash.go:254-299 with the up and down rows read from the
    file as the reference does (two ReadRowsParallel calls, :262-270)."""
    x = _f32(x).ravel()
    a = np.ascontiguousarray(active, np.int32)
    out = np.empty(h, np.float32)
    rc = lib().refcpu_ffn_sparse_load_file(str(path).encode(), up_offset, down_t_offset, t, h,
                                           ff, _p(x), _p(a), a.size, act, nthreads, _p(out))
    if rc:
        raise OSError(f"ffn_sparse_load_file: {_FILE_ERRORS.get(rc, rc)}")
    return out


def ffn_dense(up_raw, down_raw, t: int, h: int, ff: int, x, act: int = ACT_RELU) -> np.ndarray:
    """inference/forward.go:318-367 dense ReLU/GELU path."""
    u, dn = _u8(up_raw), _u8(down_raw)
    x = _f32(x).ravel()
    out = np.empty(h, np.float32)
    rc = lib().refcpu_ffn_dense(_p(u), _p(dn), t, h, ff, _p(x), act, _p(out))
    if rc:
        raise ValueError(f"ffn_dense rc={rc}")
    return out


def ffn_swiglu(gate_raw, up_raw, down_raw, t: int, h: int, ff: int, x) -> np.ndarray:
    """inference/forward.go:368-389 ffnSwiGLU: down @ (silu(gate @ x) * (up @ x))."""
    g, u, dn = _u8(gate_raw), _u8(up_raw), _u8(down_raw)
    x = _f32(x).ravel()
    out = np.empty(h, np.float32)
    rc = lib().refcpu_ffn_swiglu(_p(g), _p(u), _p(dn), t, h, ff, _p(x), _p(out))
    if rc:
        raise ValueError(f"ffn_swiglu rc={rc}")
    return out


class NeuronCache:
    """inference/window.go:21-245."""

    def __init__(self, max_neurons: int, hidden: int, window: int, ff: int, up_raw, down_t_raw,
                 t: int):
        self._u, self._d = _u8(up_raw), _u8(down_t_raw)  # keep alive
        self.ff = ff
        self.c = lib().refcpu_nc_new(max_neurons, hidden, window, ff, _p(self._u), _p(self._d), t)

    @classmethod
    def from_file(cls, max_neurons: int, hidden: int, window: int, ff: int, path,
                  up_offset: int, down_t_offset: int, t: int, nthreads: int = 32):
        """A cache whose loadRows reads the file (window.go:208-216)."""
        self = cls.__new__(cls)
        self.ff = ff
        self.c = lib().refcpu_nc_new_file(max_neurons, hidden, window, ff, str(path).encode(),
                                          up_offset, down_t_offset, t, nthreads)
        return self

    def update(self, active):
        a = np.ascontiguousarray(active, np.int32)
        nl = C.c_int()
        ll = np.empty(max(a.size, 1), np.int32)
        rc = lib().refcpu_nc_update(self.c, _p(a), a.size, C.byref(nl), _p(ll))
        if rc:
            raise ValueError(f"update rc={rc}")
        return ll[: nl.value].copy()

    def ffn_forward(self, x, active, act: int = ACT_RELU) -> np.ndarray:
        x = _f32(x).ravel()
        a = np.ascontiguousarray(active, np.int32)
        out = np.empty_like(x)
        lib().refcpu_nc_ffn_forward(self.c, _p(x), _p(a), a.size, act, _p(out))
        return out

    def num_cached(self) -> int:
        return int(lib().refcpu_nc_num_cached(self.c))

    def resident(self) -> np.ndarray:
        return np.array([n for n in range(self.ff) if lib().refcpu_nc_is_cached(self.c, n)],
                        np.int32)

    def __del__(self):
        if getattr(self, "c", None) and _lib is not None:  # the module may be gone at exit
            _lib.refcpu_nc_free(self.c)
            self.c = None


def moe_route(logits, k: int):
    """moe_forward.go:42-68 on given logits -> (ids, weights)."""
    lg = _f32(logits).ravel()
    ids = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    if lib().refcpu_moe_route(_p(lg), lg.size, k, _p(ids), _p(w)):
        raise ValueError("moe_route: invalid hparams")
    return ids, w


def moe_ffn(router, gate_raw, up_raw, down_raw, t: int, hidden: int, eff: int, n_exp: int, k: int,
            x):
    """inference/moe_forward.go:32-150 for one token -> (out, ids, weights)."""
    router = _f32(router)
    g, u, dn = _u8(gate_raw), _u8(up_raw), _u8(down_raw)
    x = _f32(x).ravel()
    out = np.empty(hidden, np.float32)
    ids = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    rc = lib().refcpu_moe_ffn(_p(router), _p(g), _p(u), _p(dn), t, hidden, eff, n_exp, k, _p(x),
                              _p(out), _p(ids), _p(w))
    if rc:
        raise ValueError(f"moeFFN: invalid hparams (rc={rc})")
    return out, ids, w


class _FalconParams(C.Structure):
    _fields_ = [(n, C.c_int) for n in ["n_layers", "hidden", "n_heads", "n_kv", "head_dim", "ff",
                                       "vocab", "max_seq", "rank", "act", "t"]] + \
               [("rope_base", C.c_float), ("eps", C.c_float)] + \
               [(n, C.c_void_p) for n in ["embed", "norm_w", "norm_b", "wq", "wk", "wv", "wo",
                                          "pwup", "pwout", "thr", "up", "down_t", "out_w",
                                          "out_b", "lm_head"]]


_SIGS.update({
    "refcpu_falcon_new": (_vp, [C.POINTER(_FalconParams)]),
    "refcpu_falcon_free": (None, [_vp]),
    "refcpu_falcon_forward": (C.c_int, [_vp, C.c_int32, C.c_int, _vp, _vp]),
    "refcpu_falcon_forward_ex": (C.c_int, [_vp, C.c_int32, C.c_int, _vp, _vp, _vp]),
    "refcpu_falcon_commit": (None, [_vp]),
    "refcpu_falcon_ffn_file": (C.c_int, [_vp, C.c_char_p, _vp, _vp, C.c_int]),
    "refcpu_argmax": (C.c_int, [_vp, C.c_int]),
})


class Falcon:
    """inference/ffn_flash.go:115-185 (ForwardFlash on the Falcon layout, path 2)
    with kvcache/kvcache.go.  `w` holds the weights: embed, lm_head (vocab GGUF
    rows), and per-layer lists norm_w, norm_b (f32 [hidden]), wq, wk, wv, wo (GGUF
    rows), pwup, pwout (f32), up, down_t (GGUF rows of the bundle halves); out_w,
    out_b (f32).  Per-layer arrays are concatenated here."""

    def __init__(self, dims: dict, w: dict, thr, t: int = Q4_0, act: int = ACT_RELU):
        cat = lambda k, conv: np.ascontiguousarray(np.concatenate([conv(a).ravel() for a in w[k]]))
        self._keep = {
            "embed": _u8(w["embed"]), "lm_head": _u8(w["lm_head"]),
            "out_w": _f32(w["out_w"]), "out_b": _f32(w["out_b"]),
            "thr": _f32(np.asarray(thr, np.float32)),
        }
        for k in ["norm_w", "norm_b", "pwup", "pwout"]:
            self._keep[k] = cat(k, _f32)
        for k in ["wq", "wk", "wv", "wo", "up", "down_t"]:
            self._keep[k] = cat(k, _u8)
        p = _FalconParams()
        for k in ["n_layers", "hidden", "n_heads", "n_kv", "head_dim", "ff", "vocab", "max_seq",
                  "rank"]:
            setattr(p, k, int(dims[k]))
        p.act, p.t = act, t
        p.rope_base, p.eps = float(dims["rope_base"]), float(dims["eps"])
        for k, a in self._keep.items():
            setattr(p, k, a.ctypes.data)
        self.vocab, self.n_layers, self.ff = int(dims["vocab"]), int(dims["n_layers"]), int(dims["ff"])
        self.m = lib().refcpu_falcon_new(C.byref(p))
        if not self.m:
            raise MemoryError("refcpu_falcon_new failed")

    def forward(self, token: int, pos: int, pred_logits: bool = False):
        """ForwardFlash(token, pos) -> (logits, n_active per layer[, predictor
        logits [n_layers x ff]]); then commit."""
        lg = np.empty(self.vocab, np.float32)
        na = np.empty(self.n_layers, np.int32)
        pl = np.empty((self.n_layers, self.ff), np.float32) if pred_logits else None
        rc = lib().refcpu_falcon_forward_ex(self.m, token, pos, _p(lg), _p(na), _p(pl))
        if rc == -2:
            raise OSError("falcon forward: FFN rows could not be read from the file")
        if rc:
            raise ValueError("falcon forward: token or position out of range")
        lib().refcpu_falcon_commit(self.m)
        return (lg, na, pl) if pred_logits else (lg, na)

    def ffn_file(self, path, up_offsets, down_offsets, nthreads: int = 32) -> None:
        """From the next token on, read each layer's FFN rows from the GGUF file
        at `path` (tensor byte offsets per layer) with the ReadRowsParallel
        pool of nthreads (ffn_flash.go:262-270, storage.go:246-319) instead of
        from memory; the results are the same.  path None: rows from memory."""
        if path is None:
            lib().refcpu_falcon_ffn_file(self.m, None, None, None, 0)
            return
        self._offs = (np.ascontiguousarray(up_offsets, np.int64),
                      np.ascontiguousarray(down_offsets, np.int64))
        assert all(o.size == self.n_layers for o in self._offs)
        if lib().refcpu_falcon_ffn_file(self.m, str(path).encode(), _p(self._offs[0]),
                                        _p(self._offs[1]), int(nthreads)):
            raise MemoryError("refcpu_falcon_ffn_file failed")

    def __del__(self):
        if getattr(self, "m", None) and _lib is not None:  # the module may be gone at exit
            _lib.refcpu_falcon_free(self.m)
            self.m = None


def argmax(v) -> int:
    """cmd/generate.go:197-205"""
    v = _f32(v)
    return int(lib().refcpu_argmax(_p(v), v.size))
