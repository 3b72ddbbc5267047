"""Row-column bundle files (flash/bundle.go) and their upload into HBM.

File layout (bundle.go:20-73): a 16-byte little-endian header {u32 magic
"BNDL" = 0x424E444C, u32 n_neurons, u32 hidden, u32 reserved}, then neuron i
at 16 + i * bytes_per_row holding [up_i | down_i], the i-th row of ffn_up and
the i-th row of the transposed ffn_down (dims [hidden, n_neurons] for both,
bundle.go:40-48).  The reference writes both rows dequantized to float32 and
leaves reserved = 0; that file is produced here byte for byte with
row_type=F32.  With row_type=None the rows keep their GGUF block bytes (the
layout the device gathers from, 5 112 B per Q4_0 neuron of 4544 instead of
36 352 B) and reserved holds the GGML type code; the reference's OpenBundle
does not read reserved, so only this module reads such files.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np
import torch

from . import gguf as gg
from .gguf_file import GGUFError, GGUFFile, TensorInfo

BUNDLE_MAGIC = 0x424E444C  # "BNDL" (bundle.go:20)
HEADER_BYTES = 16


def _dequant_rows(raw: np.ndarray, t: int, n: int) -> np.ndarray:
    return gg.dequantize_torch(torch.from_numpy(np.array(raw)), t, n).numpy()


def create_bundle(out_path, gf: GGUFFile, up: TensorInfo, down: TensorInfo,
                  row_type: int | None = gg.F32, chunk: int = 4096) -> None:
    """CreateBundle (bundle.go:37-117).  row_type F32: the reference's file
    (dequantized rows, reserved 0); None: GGUF row bytes, reserved = type."""
    if len(up.dims) != 2 or len(down.dims) != 2:
        raise GGUFError("bundle: up and down must be 2D tensors")
    hidden, n = int(up.dims[0]), int(up.dims[1])
    if int(down.dims[0]) != hidden or int(down.dims[1]) != n:
        raise GGUFError("bundle: up/down dimension mismatch")
    if row_type is None and up.type != down.type:
        raise GGUFError("bundle: typed rows need up and down of one type")
    if row_type not in (None, gg.F32):
        raise GGUFError(f"bundle: row type {row_type} (F32 or the tensors' own)")
    up_rows = gf.tensor_bytes(up).reshape(n, up.row_bytes())
    dn_rows = gf.tensor_bytes(down).reshape(n, down.row_bytes())
    reserved = 0 if row_type == gg.F32 else up.type
    with open(out_path, "wb") as f:
        f.write(struct.pack("<IIII", BUNDLE_MAGIC, n, hidden, reserved))
        for i0 in range(0, n, chunk):
            i1 = min(n, i0 + chunk)
            if row_type == gg.F32:
                u = _dequant_rows(up_rows[i0:i1], up.type, hidden)
                d = _dequant_rows(dn_rows[i0:i1], down.type, hidden)
                f.write(np.concatenate([u, d], axis=1).astype("<f4").tobytes())
            else:
                f.write(np.concatenate([up_rows[i0:i1], dn_rows[i0:i1]], axis=1).tobytes())


@dataclass
class BundleFile:
    """BundleFile (bundle.go:24-31) over a memory map of the file."""
    path: str
    n_neurons: int
    hidden: int
    row_type: int
    bytes_per_row: int   # both halves
    _rows: np.ndarray    # [n_neurons, bytes_per_row] uint8

    def halves(self):
        """(up rows, down rows) as [n_neurons, row_bytes] uint8 views."""
        hb = self.bytes_per_row // 2
        return self._rows[:, :hb], self._rows[:, hb:]

    def read_neurons(self, neurons):
        """ReadNeurons (bundle.go:150-216): float32 (up, down) rows of the
        listed neurons, each [len(neurons), hidden]."""
        idx = np.asarray(neurons, dtype=np.int64).ravel()
        if idx.size and (idx.min() < 0 or idx.max() >= self.n_neurons):
            bad = int(idx[(idx < 0) | (idx >= self.n_neurons)][0])
            raise GGUFError(f"bundle read neuron {bad}: outside [0, {self.n_neurons})")
        u, d = self.halves()
        return (_dequant_rows(u[idx], self.row_type, self.hidden),
                _dequant_rows(d[idx], self.row_type, self.hidden))

    def upload(self, dev):
        """The device bundle (llg_hip_upload_bundle) of all neurons."""
        if self.row_type not in gg.DEVICE_TYPES:
            raise GGUFError(f"bundle: rows of type {self.row_type} have no device path")
        u, d = self.halves()
        return dev.upload_bundle(np.ascontiguousarray(u), np.ascontiguousarray(d), self.row_type,
                                 self.hidden, self.n_neurons)


def open_bundle(path) -> BundleFile:
    """OpenBundle (bundle.go:124-145), plus the row type in `reserved`."""
    path = str(path)
    with open(path, "rb") as f:
        hdr = f.read(HEADER_BYTES)
    if len(hdr) != HEADER_BYTES:
        raise GGUFError("bundle: short header")
    magic, n, hidden, reserved = struct.unpack("<IIII", hdr)
    if magic != BUNDLE_MAGIC:
        raise GGUFError(f"bundle: bad magic 0x{magic:08x}")
    row_type = reserved
    bpr = 2 * gg.byte_size(row_type, hidden)
    rows = np.memmap(path, dtype=np.uint8, mode="r", offset=HEADER_BYTES, shape=(n, bpr))
    return BundleFile(path, n, hidden, row_type, bpr, rows)
