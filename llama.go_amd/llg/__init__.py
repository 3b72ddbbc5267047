"""Host-side binding of libllg_hip.so, the gfx950 sparse-FFN library.

This module mirrors the reference's Go API for the hot path so that callers
and tests read like the reference's own code:

  reference (AndersHsueh/llama.go)              here
  metal.Available / NewDevice / Device.Close    available(), Device(), Device.close()
    (metal/metal.go:46-70)
  Device.MatMulVec / Device.RMSNorm             Device.mat_mul_vec / Device.rms_norm
    (metal/metal.go:72-113)
  Predictor{WUp,WOut,Bias,Threshold}.Predict    Predictor(...).predict(attn_out)
    (inference/predictor.go:21-83)
  FlashContext.ffnSparseLoad                    ffn_sparse_load(dev, bundle, x, active, act)
    (inference/ffn_flash.go:254-299)
  Context.ffn dense ReLU/GELU                   ffn_dense(dev, up, down, x, act)
  Context.ffn dense SiLU (ffnSwiGLU)            ffn_swiglu(dev, gate, up, down, x)
    (inference/forward.go:318-389)
  NeuronCache.Update / FFNForward / NumCached   NeuronCache(dev, bundle, k).update / ...
    (inference/window.go:48-183)
  moeFFN                                        moe_ffn(dev, router, gate, up, down, ...)
    (inference/moe_forward.go:32-79)

Go's `error` returns become LlgError exceptions carrying the library's return
code and message.  Every compute call runs on the GPU through the C ABI in
include/llg_hip.h; there is no CPU fallback: without the built library or a
GPU these calls raise.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

from . import gguf  # noqa: F401  (re-exported helpers)
from .gguf import ACT_GELU, ACT_RELU, ACT_SILU, F16, F32, Q4_0, Q8_0  # noqa: F401

LIB_PATH = Path(__file__).resolve().parent / "libllg_hip.so"

# Return codes (include/llg_hip.h)
LLG_OK = 0
LLG_E_ARG = -1
LLG_E_TYPE = -2
LLG_E_ALIGN = -3
LLG_E_RANGE = -4
LLG_E_HANDLE = -5
LLG_E_NOMEM = -6
LLG_E_HPARAM = -7
LLG_E_NODEV = -8
LLG_E_SCRATCH = -9

_i32p = C.POINTER(C.c_int32)
_f32p = C.POINTER(C.c_float)
_i64p = C.POINTER(C.c_int64)
_ip = C.POINTER(C.c_int)
_vp = C.c_void_p
_i64 = C.c_int64

# name -> (restype, argtypes); the full C ABI of include/llg_hip.h
_SIGS = {
    "llg_hip_available": (C.c_int, []),
    "llg_hip_init": (_vp, []),
    "llg_hip_free": (None, [_vp]),
    "llg_hip_last_error": (C.c_char_p, [_vp]),
    "llg_hip_stream": (_vp, [_vp]),
    "llg_hip_sync": (C.c_int, [_vp]),
    "llg_hip_workspace_bytes": (C.c_int, [_vp, C.POINTER(C.c_size_t)]),
    "llg_hip_matvec": (C.c_int, [_vp, _vp, C.c_int, C.c_int, _vp, _vp]),
    "llg_hip_rmsnorm": (C.c_int, [_vp, _vp, _vp, _vp, C.c_int, C.c_float]),
    "llg_hip_upload_matrix": (C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_int, _i64p]),
    "llg_hipd_upload_matrix": (C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_int, _i64p]),
    "llg_hip_upload_bundle": (C.c_int, [_vp, _vp, _vp, C.c_int, C.c_int, C.c_int, _i64p]),
    "llg_hipd_upload_bundle": (C.c_int, [_vp, _vp, _vp, C.c_int, C.c_int, C.c_int, _i64p]),
    "llg_hip_release": (C.c_int, [_vp, _i64]),
    "llg_hip_object_info": (C.c_int, [_vp, _i64, _ip, _ip, _ip, _i64p]),
    "llg_hip_dequant": (C.c_int, [_vp, _i64, C.c_int, C.c_int, _vp]),
    "llg_hip_predict": (C.c_int, [_vp, _i64, _i64, _i64, _vp, C.c_float, _vp, _ip, _vp]),
    "llg_hip_select": (C.c_int, [_vp, _vp, C.c_int, C.c_float, _vp, _ip]),
    "llg_hip_ffn_sparse": (C.c_int, [_vp, _i64, _vp, _vp, C.c_int, C.c_int, _vp]),
    "llg_hip_ffn_predict_sparse": (
        C.c_int, [_vp, _i64, _i64, _i64, _i64, _vp, _vp, C.c_float, C.c_int, _vp, _vp, _ip]),
    "llg_hip_matvec_q": (C.c_int, [_vp, _i64, _vp, _vp]),
    "llg_hip_ffn_dense": (C.c_int, [_vp, _i64, _i64, _vp, C.c_int, _vp]),
    "llg_hip_ffn_swiglu": (C.c_int, [_vp, _i64, _i64, _i64, _vp, _vp]),
    "llg_hip_window_create": (C.c_int, [_vp, _i64, C.c_int, _i64p]),
    "llg_hip_window_update": (C.c_int, [_vp, _i64, _vp, C.c_int, _ip, _ip]),
    "llg_hip_window_ffn": (C.c_int, [_vp, _i64, _vp, _vp, C.c_int, C.c_int, _vp]),
    "llg_hip_window_resident": (C.c_int, [_vp, _i64, _vp, _ip]),
    "llg_hip_moe_ffn": (
        C.c_int, [_vp, _i64, _i64, _i64, _i64, C.c_int, C.c_int, _vp, C.c_int, _vp, _vp, _vp]),
    "llg_hip_moe_route": (C.c_int, [_vp, _vp, C.c_int, C.c_int, C.c_int, _vp, _vp]),
    "llg_hipd_predict": (C.c_int, [_vp, _i64, _i64, _i64, _vp, C.c_float, _vp, _vp, _vp]),
    "llg_hipd_ffn_sparse": (C.c_int, [_vp, _i64, _vp, _vp, _vp, C.c_int, _vp]),
    "llg_hipd_ffn_predict_sparse": (
        C.c_int, [_vp, _i64, _i64, _i64, _i64, _vp, _vp, C.c_float, C.c_int, _vp, _vp, _vp]),
    "llg_hipd_ffn_predict_sparse_noalloc": (
        C.c_int, [_vp, _i64, _i64, _i64, _i64, _vp, _vp, C.c_float, C.c_int, _vp, _vp, _vp]),
    "llg_hipd_matvec_q": (C.c_int, [_vp, _i64, _vp, _vp]),
    "llg_hipd_ffn_dense": (C.c_int, [_vp, _i64, _i64, _vp, C.c_int, _vp]),
    "llg_hipd_ffn_swiglu": (C.c_int, [_vp, _i64, _i64, _i64, _vp, _vp]),
    "llg_hipd_window_step": (C.c_int, [_vp, _i64, _vp, _vp, _vp, C.c_int, _vp]),
    "llg_hipd_moe_ffn": (
        C.c_int, [_vp, _i64, _i64, _i64, _i64, C.c_int, C.c_int, _vp, C.c_int, _vp, _vp, _vp]),
    "llg_hip_falcon_create": (C.c_int, [_vp, _vp, C.c_float, C.c_float, C.c_int, _i64, _vp, _vp,
                                        _i64, _i64, _i64, _i64p]),
    "llg_hip_falcon_set_thresholds": (C.c_int, [_vp, _i64, _vp]),
    "llg_hip_falcon_forward": (C.c_int, [_vp, _i64, C.c_int32, C.c_int, _vp, _vp, _vp, _vp]),
    "llg_hipd_falcon_step": (C.c_int, [_vp, _i64, _vp, C.c_int, _vp, _vp]),
}

_lib = None


class LlgError(RuntimeError):
    """A nonzero return code from the library (the Go side's `error`)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"{msg} (rc={code})")
        self.code = code


def load_library(path: str | Path | None = None) -> C.CDLL:
    """Load libllg_hip.so and bind every entry point; raises if it is not built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(
            f"{p} is not built; run __graft_entry__.build() (hipcc --offload-arch=gfx950)")
    lib = C.CDLL(str(p))
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def available() -> bool:
    """metal.Available (metal/metal.go:46-49)."""
    return bool(load_library().llg_hip_available())


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


class Device:
    """metal.Device (metal/metal.go:40-113) for gfx950: an opaque context with
    its own HIP stream.  All llg_hip_* calls are synchronous."""

    def __init__(self):
        self.lib = load_library()
        h = self.lib.llg_hip_init()
        if not h:
            raise LlgError(LLG_E_NODEV, "llg: no usable HIP device")
        self.h = C.c_void_p(h)

    # -- lifecycle --------------------------------------------------------
    def close(self):
        if getattr(self, "h", None):
            self.lib.llg_hip_free(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def check(self, rc: int, what: str = ""):
        if rc != 0:
            msg = self.lib.llg_hip_last_error(self.h)
            raise LlgError(rc, f"{what}: {msg.decode() if msg else ''}")

    @property
    def stream(self) -> int:
        return int(self.lib.llg_hip_stream(self.h) or 0)

    def sync(self):
        self.check(self.lib.llg_hip_sync(self.h), "sync")

    def workspace_bytes(self) -> int:
        """Bytes of the handle's growable device workspace (0 until first needed)."""
        n = C.c_size_t(0)
        self.check(self.lib.llg_hip_workspace_bytes(self.h, C.byref(n)), "workspace_bytes")
        return int(n.value)

    # -- Metal-parity calls -------------------------------------------------
    def mat_mul_vec(self, w, rows: int, cols: int, x) -> np.ndarray:
        """Device.MatMulVec (metal/metal.go:72-92)."""
        w, x = _f32(w).ravel(), _f32(x).ravel()
        if w.size != rows * cols:
            raise LlgError(LLG_E_ARG, f"MatMulVec: w length {w.size} != rows*cols {rows * cols}")
        if x.size != cols:
            raise LlgError(LLG_E_ARG, f"MatMulVec: x length {x.size} != cols {cols}")
        y = np.empty(rows, np.float32)
        self.check(self.lib.llg_hip_matvec(self.h, _ptr(w), rows, cols, _ptr(x), _ptr(y)),
                   "MatMulVec")
        return y

    def rms_norm(self, x, weight, eps: float) -> np.ndarray:
        """Device.RMSNorm (metal/metal.go:94-113)."""
        x, weight = _f32(x).ravel(), _f32(weight).ravel()
        if weight.size != x.size:
            raise LlgError(LLG_E_ARG, "RMSNorm: weight length != x length")
        out = np.empty_like(x)
        self.check(self.lib.llg_hip_rmsnorm(self.h, _ptr(x), _ptr(weight), _ptr(out), x.size,
                                            eps), "RMSNorm")
        return out

    # -- residency ---------------------------------------------------------------
    def upload_matrix(self, raw, ggml_type: int, rows: int, cols: int) -> "Handle":
        """GGUF bytes of a [rows x cols] tensor (host numpy/torch-CPU or a CUDA tensor)."""
        out = C.c_int64()
        rb = _row_bytes(ggml_type, cols)
        if rb and rows > 0:
            _need(_nbytes(raw), rows * rb, "upload_matrix bytes")
        if _is_device_tensor(raw):
            rc = self.lib.llg_hipd_upload_matrix(self.h, C.c_void_p(raw.data_ptr()), ggml_type,
                                                 rows, cols, C.byref(out))
        else:
            a = _host_bytes(raw)
            rc = self.lib.llg_hip_upload_matrix(self.h, _ptr(a), ggml_type, rows, cols,
                                                C.byref(out))
        self.check(rc, "upload_matrix")
        return Handle(self, out.value, "matrix")

    def upload_f32(self, m) -> "Handle":
        m = _f32(m)
        if m.ndim == 1:
            m = m.reshape(1, -1)
        return self.upload_matrix(m, F32, m.shape[0], m.shape[1])

    def upload_bundle(self, up_raw, down_t_raw, ggml_type: int, h: int, ff: int) -> "Handle":
        """flash.CreateBundle (flash/bundle.go:37-111) into HBM, bytes kept quantized."""
        out = C.c_int64()
        rb = _row_bytes(ggml_type, h)
        if rb and ff > 0:
            _need(_nbytes(up_raw), ff * rb, "upload_bundle up bytes")
            _need(_nbytes(down_t_raw), ff * rb, "upload_bundle down bytes")
        if _is_device_tensor(up_raw):
            rc = self.lib.llg_hipd_upload_bundle(self.h, C.c_void_p(up_raw.data_ptr()),
                                                 C.c_void_p(down_t_raw.data_ptr()), ggml_type, h,
                                                 ff, C.byref(out))
        else:
            a, b = _host_bytes(up_raw), _host_bytes(down_t_raw)
            rc = self.lib.llg_hip_upload_bundle(self.h, _ptr(a), _ptr(b), ggml_type, h, ff,
                                                C.byref(out))
        self.check(rc, "upload_bundle")
        return Handle(self, out.value, "bundle")

    def dequant(self, handle: "Handle", row0: int, nrows: int) -> np.ndarray:
        info = handle.info()
        per = info["cols"] * (2 if handle.is_bundle else 1)
        out = np.empty(nrows * per, np.float32)
        self.check(self.lib.llg_hip_dequant(self.h, handle.id, row0, nrows, _ptr(out)), "dequant")
        return out.reshape(nrows, per)

    def select(self, logits, threshold: float) -> np.ndarray:
        """predictor.go:76-82 on given logits (the bit-exact selection hook)."""
        lg = _f32(logits).ravel()
        act = np.empty(max(lg.size, 1), np.int32)
        n = C.c_int()
        self.check(self.lib.llg_hip_select(self.h, _ptr(lg), lg.size, threshold, _ptr(act),
                                           C.byref(n)), "select")
        return act[: n.value].copy()

    def matvec_q(self, mat: "Handle", x) -> np.ndarray:
        info = mat.info()
        x = _f32(x).ravel()
        _need(x.size, info["cols"], "matvec_q x")
        y = np.empty(info["rows"], np.float32)
        self.check(self.lib.llg_hip_matvec_q(self.h, mat.id, _ptr(x), _ptr(y)), "matvec_q")
        return y

    def moe_route(self, logits, k: int):
        lg = _f32(logits)
        if lg.ndim == 1:
            lg = lg.reshape(1, -1)
        if lg.ndim != 2:
            raise LlgError(LLG_E_ARG, "moe_route: logits must be [n_tok x n_exp]")
        n_tok, n_exp = lg.shape
        ids = np.empty((n_tok, k), np.int32)
        w = np.empty((n_tok, k), np.float32)
        self.check(self.lib.llg_hip_moe_route(self.h, _ptr(lg), n_tok, n_exp, k, _ptr(ids),
                                              _ptr(w)), "moe_route")
        return ids, w


def _is_device_tensor(a) -> bool:
    return hasattr(a, "is_cuda") and bool(getattr(a, "is_cuda"))


def _nbytes(a) -> int:
    if hasattr(a, "element_size"):
        return a.numel() * a.element_size()
    return np.asarray(a).nbytes


def _row_bytes(ggml_type: int, cols: int) -> int:
    """ByteSize of a row, or 0 when the C ABI will reject the type or length
    itself (with its own error code)."""
    try:
        return gguf.byte_size(ggml_type, cols) if ggml_type in gguf.DEVICE_TYPES and cols > 0 else 0
    except ValueError:
        return 0


def _need(n_have: int, n_want: int, what: str):
    """The C ABI reads exactly n_want elements (or bytes): a shorter buffer
    is an argument error here, before any copy."""
    if n_have != n_want:
        raise LlgError(LLG_E_ARG, f"{what}: {n_have} given, {n_want} expected")


def _host_bytes(a) -> np.ndarray:
    if hasattr(a, "numpy"):
        a = a.contiguous().numpy()
    return np.ascontiguousarray(a).view(np.uint8).ravel()


class Handle:
    """A library-owned device object (matrix, bundle or window)."""

    def __init__(self, dev: Device, hid: int, kind: str):
        self.dev = dev
        self.id = hid
        self.kind = kind

    def info(self) -> dict:
        """type, rows, cols, stride of the object (queried once; objects never change shape)."""
        if getattr(self, "_info", None) is None:
            t, r, c, s = C.c_int(), C.c_int(), C.c_int(), C.c_int64()
            self.dev.check(self.dev.lib.llg_hip_object_info(self.dev.h, self.id, C.byref(t),
                                                            C.byref(r), C.byref(c), C.byref(s)),
                           "object_info")
            self._info = {"type": t.value, "rows": r.value, "cols": c.value, "stride": s.value}
        return self._info

    @property
    def is_bundle(self) -> bool:
        return self.kind == "bundle"

    def release(self):
        if self.id:
            self.dev.check(self.dev.lib.llg_hip_release(self.dev.h, self.id), "release")
            self.id = 0


class Predictor:
    """inference.Predictor (predictor.go:21-34): WUp [rank x h], WOut [ff x rank],
    optional Bias [ff], Threshold."""

    def __init__(self, dev: Device, w_up, w_out, bias=None, threshold: float = 0.0):
        w_up, w_out = _f32(w_up), _f32(w_out)
        self.dev = dev
        self.h, self.rank, self.ff = w_up.shape[1], w_up.shape[0], w_out.shape[0]
        self.w_up = dev.upload_f32(w_up)
        self.w_out = dev.upload_f32(w_out)
        self.bias = dev.upload_f32(_f32(bias).reshape(1, -1)) if bias is not None else None
        self.threshold = float(threshold)

    @property
    def bias_id(self) -> int:
        return self.bias.id if self.bias is not None else 0

    def predict(self, attn_out, return_logits: bool = False):
        """Predict (predictor.go:51-83): ascending indices with logit > Threshold."""
        a = _f32(attn_out).ravel()
        _need(a.size, self.h, "Predict attn_out")
        act = np.empty(self.ff, np.int32)
        n = C.c_int()
        logits = np.empty(self.ff, np.float32) if return_logits else None
        self.dev.check(self.dev.lib.llg_hip_predict(
            self.dev.h, self.w_up.id, self.w_out.id, self.bias_id, _ptr(a), self.threshold,
            _ptr(act), C.byref(n), _ptr(logits) if logits is not None else None), "Predict")
        idx = act[: n.value].copy()
        return (idx, logits) if return_logits else idx


def ffn_sparse_load(dev: Device, bundle: Handle, x, active, act: int = ACT_RELU) -> np.ndarray:
    """ffnSparseLoad (ffn_flash.go:254-299) over an HBM bundle."""
    x = _f32(x).ravel()
    _need(x.size, bundle.info()["cols"], "ffnSparseLoad x")
    a = _i32(active).ravel()
    out = np.empty_like(x)
    dev.check(dev.lib.llg_hip_ffn_sparse(dev.h, bundle.id, _ptr(x), _ptr(a) if a.size else None,
                                         a.size, act, _ptr(out)), "ffnSparseLoad")
    return out


def ffn_predict_sparse(dev: Device, pred: Predictor, bundle: Handle, attn_out, x,
                       act: int = ACT_RELU):
    """ffnFlash path 2 (ffn_flash.go:225-231): Predict then ffnSparseLoad, on the device."""
    a, x = _f32(attn_out).ravel(), _f32(x).ravel()
    _need(a.size, pred.h, "ffnFlash attn_out")
    _need(x.size, bundle.info()["cols"], "ffnFlash x")
    out = np.empty_like(x)
    idx = np.empty(pred.ff, np.int32)
    n = C.c_int()
    dev.check(dev.lib.llg_hip_ffn_predict_sparse(
        dev.h, pred.w_up.id, pred.w_out.id, pred.bias_id, bundle.id, _ptr(a), _ptr(x),
        pred.threshold, act, _ptr(out), _ptr(idx), C.byref(n)), "ffnFlash")
    return out, idx[: n.value].copy()


def ffn_dense(dev: Device, up: Handle, down: Handle, x, act: int = ACT_RELU) -> np.ndarray:
    """Context.ffn ReLU/GELU path (forward.go:342-367): down @ act(up @ x)."""
    x = _f32(x).ravel()
    _need(x.size, up.info()["cols"], "ffn x")
    out = np.empty(down.info()["rows"], np.float32)
    dev.check(dev.lib.llg_hip_ffn_dense(dev.h, up.id, down.id, _ptr(x), act, _ptr(out)), "ffn")
    return out


def ffn_swiglu(dev: Device, gate: Handle, up: Handle, down: Handle, x) -> np.ndarray:
    """Context.ffn SiLU path, ffnSwiGLU (forward.go:368-389):
    down @ (silu(gate @ x) * (up @ x))."""
    x = _f32(x).ravel()
    _need(x.size, gate.info()["cols"], "ffn_swiglu x")
    out = np.empty(down.info()["rows"], np.float32)
    dev.check(dev.lib.llg_hip_ffn_swiglu(dev.h, gate.id, up.id, down.id, _ptr(x), _ptr(out)),
              "ffn_swiglu")
    return out


class NeuronCache:
    """inference.NeuronCache (window.go:21-245) with its rows resident in HBM."""

    def __init__(self, dev: Device, bundle: Handle, window_size: int):
        self.dev = dev
        self.bundle = bundle
        self.window_size = window_size
        info = bundle.info()  # kept: the window outlives a released bundle handle
        self.hidden, self.ff = info["cols"], info["rows"]
        out = C.c_int64()
        dev.check(dev.lib.llg_hip_window_create(dev.h, bundle.id, window_size, C.byref(out)),
                  "NewNeuronCache")
        self.win = Handle(dev, out.value, "window")
        self.last_loaded = 0
        self._num = 0

    def update(self, active_neurons) -> int:
        """Update (window.go:71-117); returns the number of rows loaded."""
        a = _i32(active_neurons).ravel()
        nl, nr = C.c_int(), C.c_int()
        self.dev.check(self.dev.lib.llg_hip_window_update(
            self.dev.h, self.win.id, _ptr(a) if a.size else None, a.size, C.byref(nl),
            C.byref(nr)), "NeuronCache.Update")
        self.last_loaded, self._num = nl.value, nr.value
        return nl.value

    def ffn_forward(self, x, active_neurons, act: int = ACT_RELU) -> np.ndarray:
        """FFNForward (window.go:143-180)."""
        x = _f32(x).ravel()
        _need(x.size, self.hidden, "FFNForward x")
        a = _i32(active_neurons).ravel()
        out = np.empty_like(x)
        self.dev.check(self.dev.lib.llg_hip_window_ffn(
            self.dev.h, self.win.id, _ptr(x), _ptr(a) if a.size else None, a.size, act,
            _ptr(out)), "NeuronCache.FFNForward")
        return out

    def step_device(self, d_x: int, d_active: int, d_n_active: int, d_out: int,
                    act: int = ACT_RELU) -> None:
        """Update + FFNForward of one token on device buffers (x f32[h], the
        active list int32[n] and its count int32[1], out f32[h]), enqueued on
        the device's stream without waiting: the bundles that the update
        loads are copied into their resident rows by the FFN's first read.
        num_cached() is refreshed by resident()."""
        self.dev.check(self.dev.lib.llg_hipd_window_step(self.dev.h, self.win.id, d_x, d_active,
                                                         d_n_active, act, d_out),
                       "NeuronCache.step")

    def num_cached(self) -> int:
        """NumCached (window.go:183)."""
        return self._num

    def resident(self) -> np.ndarray:
        flags = np.empty(self.ff, np.uint8)
        n = C.c_int()
        self.dev.check(self.dev.lib.llg_hip_window_resident(self.dev.h, self.win.id,
                                                            _ptr(flags), C.byref(n)), "resident")
        self._num = n.value
        return np.flatnonzero(flags).astype(np.int32)


def moe_ffn(dev: Device, router: Handle, gate: Handle, up: Handle, down: Handle, n_exp: int,
            k: int, x):
    """moeFFN (moe_forward.go:32-79) for one or more tokens x [n_tok x hidden].

    Returns (out [n_tok x hidden], expert ids [n_tok x k], weights [n_tok x k])."""
    x = _f32(x)
    squeeze = x.ndim == 1
    if squeeze:
        x = x.reshape(1, -1)
    n_tok = x.shape[0]
    if x.ndim != 2:
        raise LlgError(LLG_E_ARG, "moeFFN: x must be [hidden] or [n_tok x hidden]")
    _need(x.shape[1], gate.info()["cols"], "moeFFN x width")
    out = np.empty_like(x)
    ids = np.empty((n_tok, k), np.int32)
    w = np.empty((n_tok, k), np.float32)
    dev.check(dev.lib.llg_hip_moe_ffn(dev.h, router.id, gate.id, up.id, down.id, n_exp, k,
                                      _ptr(x), n_tok, _ptr(out), _ptr(ids), _ptr(w)), "moeFFN")
    if squeeze:
        return out[0], ids[0], w[0]
    return out, ids, w


class FalconModel:
    """The Falcon decode of inference.FlashContext.ForwardFlash
    (ffn_flash.go:115-185) with its weights in HBM.  `dims`: n_layers, hidden,
    n_heads, n_kv, head_dim, ff, vocab, max_seq, rope_base, eps.  `w`: embed,
    lm_head (GGUF rows), out_w, out_b (f32 [hidden]), and per-layer lists
    norm_w, norm_b (f32), wq, wk, wv, wo (GGUF rows), pwup, pwout (f32
    predictor), up, down_t (GGUF rows of the bundle halves).  Arrays may be
    host numpy arrays or CUDA tensors.  `t` is the GGUF type of every matrix,
    or a dict of types by key (embed, lm_head, wqkv, wo, bundle)."""

    def __init__(self, dev: Device, dims: dict, w: dict, thresholds, t=2,
                 act: int = ACT_RELU):
        self.dev, self.dims = dev, dict(dims)
        h, nh, nkv, hd = dims["hidden"], dims["n_heads"], dims["n_kv"], dims["head_dim"]
        ff, V, L = dims["ff"], dims["vocab"], dims["n_layers"]
        thr = _f32(thresholds).ravel()
        _need(thr.size, L, "falcon thresholds")  # the C ABI reads one per layer
        self._h = []
        up = self._keep

        def vec(a):
            return up(dev.upload_f32(_as_host_f32(a).reshape(1, -1)))

        def cat_rows(parts):
            if all(hasattr(p, "is_cuda") for p in parts):
                import torch
                return torch.cat([p.reshape(p.shape[0], -1) for p in parts])
            return np.concatenate([np.asarray(p) for p in parts])

        ty = t if isinstance(t, dict) else dict.fromkeys(
            ("embed", "lm_head", "wqkv", "wo", "bundle"), t)
        self.embed = up(dev.upload_matrix(w["embed"], ty["embed"], V, h))
        self.lm_head = up(dev.upload_matrix(w["lm_head"], ty["lm_head"], V, h))
        self.out_w, self.out_b = vec(w["out_w"]), vec(w["out_b"])
        lh = []
        for l in range(L):
            wqkv = cat_rows([w["wq"][l], w["wk"][l], w["wv"][l]])
            hs = [vec(w["norm_w"][l]), vec(w["norm_b"][l]),
                  up(dev.upload_matrix(wqkv, ty["wqkv"], (nh + 2 * nkv) * hd, h)),
                  up(dev.upload_matrix(w["wo"][l], ty["wo"], h, nh * hd)),
                  up(dev.upload_matrix(w["pwup"][l], F32, w["pwup"][l].shape[0], h)),
                  up(dev.upload_matrix(w["pwout"][l], F32, ff, w["pwout"][l].shape[1])),
                  up(dev.upload_bundle(w["up"][l], w["down_t"][l], ty["bundle"], h, ff))]
            lh += [x.id for x in hs]
        d32 = np.array([L, h, nh, nkv, hd, ff, V, dims["max_seq"]], np.int32)
        lh = np.array(lh, np.int64)
        out = C.c_int64()
        dev.check(dev.lib.llg_hip_falcon_create(
            dev.h, _ptr(d32), float(dims["rope_base"]), float(dims["eps"]), act, self.embed.id,
            _ptr(lh), _ptr(thr), self.out_w.id, self.out_b.id, self.lm_head.id, C.byref(out)),
            "falcon_create")
        self.model = Handle(dev, out.value, "model")

    def _keep(self, hnd: "Handle") -> "Handle":
        self._h.append(hnd)
        return hnd

    def set_thresholds(self, thresholds):
        thr = _f32(thresholds).ravel()
        _need(thr.size, self.dims["n_layers"], "falcon thresholds")
        self.dev.check(self.dev.lib.llg_hip_falcon_set_thresholds(self.dev.h, self.model.id,
                                                                  _ptr(thr)), "thresholds")

    def forward(self, token: int, pos: int, pred_logits: bool = False):
        """ForwardFlash(token, pos) -> (logits, greedy next token, n_active per
        layer[, predictor logits [n_layers x ff]])."""
        lg = np.empty(self.dims["vocab"], np.float32)
        nt = np.zeros(1, np.int32)
        na = np.empty(self.dims["n_layers"], np.int32)
        pl = np.empty((self.dims["n_layers"], self.dims["ff"]), np.float32) if pred_logits else None
        self.dev.check(self.dev.lib.llg_hip_falcon_forward(
            self.dev.h, self.model.id, int(token), int(pos), _ptr(lg), _ptr(nt), _ptr(na),
            _ptr(pl) if pl is not None else None), "ForwardFlash")
        if pred_logits:
            return lg, int(nt[0]), na, pl
        return lg, int(nt[0]), na

    def step_device(self, d_token: int, pos: int, d_next: int, d_logits: int = 0):
        """Enqueue one token on the library stream (device pointers as ints)."""
        self.dev.check(self.dev.lib.llg_hipd_falcon_step(
            self.dev.h, self.model.id, C.c_void_p(d_token), int(pos), C.c_void_p(d_next),
            C.c_void_p(d_logits) if d_logits else None), "falcon_step")

    def release(self):
        self.model.release()
        for x in self._h:
            x.release()
        self._h = []


def _as_host_f32(a) -> np.ndarray:
    if hasattr(a, "is_cuda"):
        a = a.detach().float().cpu().numpy()
    return _f32(a)


from .flash import FlashFFN, FlashFFNConfig, FlashLayer, PredictorSet  # noqa: E402,F401
