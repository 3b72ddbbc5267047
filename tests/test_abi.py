"""CPU-side checks of the C ABI: the library loads, exports every entry point
declared in include/llg_hip.h, and the Python binding fails loudly when the
library is absent.  No compute call is made here (there is no GPU)."""
import ctypes
import re
from pathlib import Path

import pytest

import llg

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "llg_hip.h"


def declared_symbols() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"\b(llg_hipd?_[a-z_0-9]+)\s*\(", text))


def test_header_declares_hot_path():
    syms = declared_symbols()
    for s in ["llg_hip_init", "llg_hip_free", "llg_hip_available", "llg_hip_matvec",
              "llg_hip_rmsnorm", "llg_hip_predict", "llg_hip_select", "llg_hip_ffn_sparse",
              "llg_hip_window_update", "llg_hip_window_ffn", "llg_hip_moe_ffn",
              "llg_hip_dequant", "llg_hip_matvec_q", "llg_hip_ffn_dense"]:
        assert s in syms


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(llg.LIB_PATH))
    missing = [s for s in sorted(declared_symbols()) if not hasattr(lib, s)]
    assert not missing, missing


def test_binding_covers_header():
    assert declared_symbols() == set(llg._SIGS)


def test_missing_library_raises(tmp_path):
    with pytest.raises(FileNotFoundError):
        llg.load_library(tmp_path / "nope.so")


def test_error_codes_match_header():
    text = HEADER.read_text()
    for name in ["LLG_E_ARG", "LLG_E_TYPE", "LLG_E_ALIGN", "LLG_E_RANGE", "LLG_E_HANDLE",
                 "LLG_E_NOMEM", "LLG_E_HPARAM", "LLG_E_NODEV", "LLG_E_SCRATCH"]:
        m = re.search(rf"{name}\s*=\s*(-?\d+)", text)
        assert m and int(m.group(1)) == getattr(llg, name)
