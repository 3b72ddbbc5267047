"""GGUF element types, row sizes and block quantizers for synthetic weights.

Type codes and block sizes follow gguf/types.go:40-102.  The reference ships
no quantizer; the ones here follow ggml's published reference method
(quantize_row_q4_0_ref / quantize_row_q8_0_ref) and pack Q4_0 nibbles in the
order the reference decodes them (tensor/dtype.go:73-79: element 2i is the
low nibble of byte i, element 2i+1 the high nibble), so that
Dequantize(quantize(x)) returns elements in their original order.

The quantizers run on torch tensors on any device, so multi-hundred-MB
weights are made on the GPU and small fixtures on the CPU.
"""
from __future__ import annotations

import torch

F32, F16, Q4_0, Q8_0 = 0, 1, 2, 8
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q8_0: "Q8_0"}
# (block size, bytes per block) of every type the reference knows
# (gguf/types.go:70-89); the device path computes on F32, F16, Q4_0 and Q8_0.
TYPE_INFO = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24),
             Q8_0: (32, 34), 9: (32, 36), 10: (256, 84), 11: (256, 110), 12: (256, 144),
             13: (256, 176), 14: (256, 210), 15: (256, 292), 24: (1, 1), 25: (1, 2),
             26: (1, 4), 27: (1, 8), 28: (1, 8)}
DEVICE_TYPES = (F32, F16, Q4_0, Q8_0)

ACT_RELU, ACT_GELU, ACT_SILU = 0, 1, 2  # model/model.go:97-103


def byte_size(ggml_type: int, n: int) -> int:
    """GGMLType.ByteSize (gguf/types.go:90-102); raises ValueError like its error returns."""
    if ggml_type not in TYPE_INFO:
        raise ValueError(f"unknown GGML type: {ggml_type}")
    bs, ts = TYPE_INFO[ggml_type]
    if n % bs:
        raise ValueError(f"element count {n} not divisible by block size {bs}")
    return n // bs * ts


def _u8(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous().view(torch.uint8)


def quantize_q4_0(x: torch.Tensor) -> torch.Tensor:
    """fp32 [..., n] -> uint8 [..., n/32*18] (GGUF Q4_0 bytes, reference nibble order)."""
    assert x.dtype == torch.float32 and x.shape[-1] % 32 == 0
    lead = x.shape[:-1]
    xb = x.reshape(-1, 32)
    idx = xb.abs().argmax(dim=1, keepdim=True)  # first index of max |v|
    mx = xb.gather(1, idx)
    d = mx / -8.0
    inv = torch.where(d != 0, 1.0 / d, torch.zeros_like(d))
    q = torch.clamp(torch.trunc(xb * inv + 8.5), max=15.0).to(torch.uint8)
    packed = q[:, 0::2] | (q[:, 1::2] << 4)  # byte i = elem 2i | elem 2i+1 << 4
    dh = _u8(d.to(torch.float16)).reshape(-1, 2)
    out = torch.cat([dh, packed], dim=1)
    return out.reshape(*lead, -1)


def quantize_q8_0(x: torch.Tensor) -> torch.Tensor:
    """fp32 [..., n] -> uint8 [..., n/32*34] (GGUF Q8_0 bytes)."""
    assert x.dtype == torch.float32 and x.shape[-1] % 32 == 0
    lead = x.shape[:-1]
    xb = x.reshape(-1, 32)
    amax = xb.abs().amax(dim=1, keepdim=True)
    d = amax / 127.0
    inv = torch.where(d != 0, 1.0 / d, torch.zeros_like(d))
    v = xb * inv
    q = (torch.sign(v) * torch.floor(v.abs() + 0.5)).to(torch.int8)  # roundf: half away from 0
    dh = _u8(d.to(torch.float16)).reshape(-1, 2)
    out = torch.cat([dh, q.view(torch.uint8)], dim=1)
    return out.reshape(*lead, -1)


def quantize(x: torch.Tensor, ggml_type: int) -> torch.Tensor:
    """fp32 [..., n] -> GGUF bytes uint8 [..., ByteSize(n)]."""
    if ggml_type == Q4_0:
        return quantize_q4_0(x)
    if ggml_type == Q8_0:
        return quantize_q8_0(x)
    if ggml_type == F16:
        h = x.to(torch.float16).contiguous()
        return h.view(torch.uint8).reshape(*x.shape[:-1], -1)
    if ggml_type == F32:
        return x.contiguous().view(torch.uint8).reshape(*x.shape[:-1], -1)
    raise ValueError(f"unsupported type {ggml_type}")


def dequantize_torch(raw: torch.Tensor, ggml_type: int, n: int) -> torch.Tensor:
    """Vectorised GGUF -> fp32 (same values as tensor/dtype.go for non-NaN scales).

    Used to build float64 brute-force references in tests; the oracle's C
    dequant is the checked restatement of the reference.
    """
    lead = raw.shape[:-1]
    r = raw.reshape(-1, raw.shape[-1])
    if ggml_type == Q4_0:
        blk = r.reshape(r.shape[0], -1, 18)
        d = blk[:, :, :2].contiguous().view(torch.float16).to(torch.float32)
        qs = blk[:, :, 2:].to(torch.int32)
        lo = (qs & 15) - 8
        hi = (qs >> 4) - 8
        q = torch.stack([lo, hi], dim=-1).reshape(r.shape[0], -1, 32).to(torch.float32)
        out = (q * d).reshape(r.shape[0], -1)
    elif ggml_type == Q8_0:
        blk = r.reshape(r.shape[0], -1, 34)
        d = blk[:, :, :2].contiguous().view(torch.float16).to(torch.float32)
        q = blk[:, :, 2:].contiguous().view(torch.int8).to(torch.float32)
        out = (q * d).reshape(r.shape[0], -1)
    elif ggml_type == F16:
        out = r.contiguous().view(torch.float16).to(torch.float32)
    elif ggml_type == F32:
        out = r.contiguous().view(torch.float32)
    else:
        raise ValueError(f"unsupported type {ggml_type}")
    assert out.shape[-1] == n
    return out.reshape(*lead, n)
