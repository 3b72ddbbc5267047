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


def test_falcon_thresholds_length_checked():
    """The C ABI reads one threshold per layer: a shorter or longer list (or a
    scalar for a multi-layer model) is rejected before any device call."""
    dims = dict(n_layers=2, hidden=64, n_heads=1, n_kv=1, head_dim=64, ff=128, vocab=8,
                max_seq=4, rope_base=10000.0, eps=1e-5)
    for bad in ([0.5], [0.1, 0.2, 0.3], 0.5):
        with pytest.raises(llg.LlgError) as e:
            llg.FalconModel(None, dims, {}, bad)
        assert e.value.code == llg.LLG_E_ARG
    m = llg.FalconModel.__new__(llg.FalconModel)
    m.dev, m.dims = None, dims
    with pytest.raises(llg.LlgError) as e:
        m.set_thresholds([0.5])
    assert e.value.code == llg.LLG_E_ARG
