"""The C-ABI library loads and exports every entry point include/superl8_kv.h
declares (no compute calls: this runs without a GPU)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "superl8_kv.h"
LIB = ROOT / "superl8_serve_amd" / "libsuperl8_kv.so"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(s8kv_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for name in ("s8kv_append_int8", "s8kv_append_k8v3", "s8kv_decode_int8", "s8kv_decode_k8v3",
                 "s8kv_decode_workspace_size", "s8kv_copy_blocks", "s8kv_last_error", "s8kv_version"):
        assert name in syms


@pytest.mark.skipif(not LIB.exists(), reason="libsuperl8_kv.so not built (run __graft_entry__.build())")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(LIB))
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, f"not exported: {missing}"


@pytest.mark.skipif(not LIB.exists(), reason="libsuperl8_kv.so not built (run __graft_entry__.build())")
def test_python_binding_matches_header():
    from superl8_serve_amd import _lib

    assert set(_lib.SIGNATURES) == set(declared_symbols())
    lib = _lib.load()
    assert lib.s8kv_version() >= 100


@pytest.mark.skipif(not LIB.exists(), reason="libsuperl8_kv.so not built (run __graft_entry__.build())")
def test_host_validation_without_gpu():
    """Argument checks run on the host and report through s8kv_last_error."""
    from superl8_serve_amd import _lib

    lib = _lib.load()
    rc = lib.s8kv_append_int8(None, None, 1, 8, 96, 0, 0, 0, 0, None, None, None, None, None, 10, 16, None)
    assert rc == -2 and b"head_dim" in lib.s8kv_last_error()
    rc = lib.s8kv_append_int8(None, None, 1, 8, 128, 0, 0, 0, 0, None, None, None, None, None, 10, 12, None)
    assert rc == -2 and b"block_size" in lib.s8kv_last_error()
    rc = lib.s8kv_decode_int8(None, 2, 12, 8, 128, 0, 0, None, None, None, None, 4, 16, None, 0, None, 16, 0.1,
                              None, None, 0, None)
    assert rc == -1 and b"multiple" in lib.s8kv_last_error()
    assert lib.s8kv_decode_workspace_size(64, 32, 8, 128, 8192) > 0
    assert lib.s8kv_decode_workspace_size(0, 32, 8, 128, 8192) == 0
    with pytest.raises(ValueError):
        _lib.check(-1, "probe")
