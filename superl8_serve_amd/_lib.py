"""ctypes binding of ``libsuperl8_kv.so`` (declared in ``include/superl8_kv.h``).

The library is loaded from this package directory only; there is no other
implementation to fall back to.  ``load()`` raises ``RuntimeError`` when the
library has not been built.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libsuperl8_kv.so"

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

# name -> (restype, argtypes); mirrors include/superl8_kv.h
SIGNATURES: dict[str, tuple] = {
    "s8kv_version": (_i32, []),
    "s8kv_last_error": (ctypes.c_char_p, []),
    "s8kv_append_int8": (_i32, [
        _c_void_p, _c_void_p, _i64, _i32, _i32,
        _i64, _i64, _i64, _i64,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
        _i64, _i32, _c_void_p,
    ]),
    "s8kv_append_k8v3": (_i32, [
        _c_void_p, _c_void_p, _i64, _i32, _i32,
        _i64, _i64, _i64, _i64,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32,
        _i64, _i32, _c_void_p,
    ]),
    "s8kv_decode_workspace_size": (_i64, [_i32, _i32, _i32, _i32, _i32]),
    "s8kv_decode_int8": (_i32, [
        _c_void_p, _i32, _i32, _i32, _i32,
        _i64, _i64,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32,
        _c_void_p, _i64, _c_void_p,
        _i32, _f32, _c_void_p, _c_void_p, _i64, _c_void_p,
    ]),
    "s8kv_decode_append_int8": (_i32, [
        _c_void_p, _i32, _i32, _i32, _i32,
        _i64, _i64,
        _c_void_p, _i64, _i64, _c_void_p, _i64, _i64,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32,
        _c_void_p, _i64, _c_void_p,
        _i32, _f32, _c_void_p, _c_void_p, _i64, _c_void_p,
    ]),
    "s8kv_decode_append_int8_noalloc": (_i32, [
        _c_void_p, _i32, _i32, _i32, _i32,
        _i64, _i64,
        _c_void_p, _i64, _i64, _c_void_p, _i64, _i64,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32,
        _c_void_p, _i64, _c_void_p,
        _i32, _f32, _c_void_p, _c_void_p,
    ]),
    "s8kv_decode_append_k8v3": (_i32, [
        _c_void_p, _i32, _i32, _i32, _i32,
        _i64, _i64,
        _c_void_p, _i64, _i64, _c_void_p, _i64, _i64,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i32,
        _c_void_p, _i64, _c_void_p,
        _i32, _f32, _c_void_p, _c_void_p, _i64, _c_void_p,
    ]),
    "s8kv_decode_append_int8_planned": (_i32, [
        _c_void_p, _i32, _i32, _i32, _i32,
        _i64, _i64,
        _c_void_p, _i64, _i64, _c_void_p, _i64, _i64,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32,
        _c_void_p, _i64, _c_void_p,
        _i32, _f32, _c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p, _i64,
    ]),
    "s8kv_decode_append_k8v3_planned": (_i32, [
        _c_void_p, _i32, _i32, _i32, _i32,
        _i64, _i64,
        _c_void_p, _i64, _i64, _c_void_p, _i64, _i64,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i32,
        _c_void_p, _i64, _c_void_p,
        _i32, _f32, _c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p, _i64,
    ]),
    "s8kv_decode_plan_size": (_i64, [_i32]),
    "s8kv_decode_plan": (_i32, [
        _i32, _i32, _i32, _i32, _i32, _i32,
        _i64, _i32, _c_void_p, _i64, _c_void_p, _i32,
        _c_void_p, _i64, _c_void_p,
    ]),
    "s8kv_decode_plan_adaptive": (_i32, [
        _i32, _i32, _i32, _i32, _i32, _i32,
        _i64, _i32, _c_void_p, _i64, _c_void_p, _i32,
        _c_void_p, _i64, _c_void_p,
    ]),
    "s8kv_decode_k8v3": (_i32, [
        _c_void_p, _i32, _i32, _i32, _i32,
        _i64, _i64,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i32,
        _c_void_p, _i64, _c_void_p,
        _i32, _f32, _c_void_p, _c_void_p, _i64, _c_void_p,
    ]),
    "s8kv_decode_window_int8": (_i32, [
        _c_void_p, _i32, _i32, _i32, _i32,
        _i64, _i64,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32,
        _c_void_p, _i64, _c_void_p,
        _i32, _i32, _f32, _c_void_p, _c_void_p, _i64, _c_void_p,
    ]),
    "s8kv_decode_window_k8v3": (_i32, [
        _c_void_p, _i32, _i32, _i32, _i32,
        _i64, _i64,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i32,
        _c_void_p, _i64, _c_void_p,
        _i32, _i32, _f32, _c_void_p, _c_void_p, _i64, _c_void_p,
    ]),
    "s8kv_verify_workspace_size": (_i64, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "s8kv_verify_set_splits": (_i32, [_i32]),
    "s8kv_verify_int8": (_i32, [
        _c_void_p, _i32, _i32, _i32, _i32, _i32,
        _i64, _i64, _i64,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32,
        _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p,
        _i32, _f32, _c_void_p, _c_void_p, _i64, _c_void_p,
    ]),
    "s8kv_verify_k8v3": (_i32, [
        _c_void_p, _i32, _i32, _i32, _i32, _i32,
        _i64, _i64, _i64,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i32,
        _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p,
        _i32, _f32, _c_void_p, _c_void_p, _i64, _c_void_p,
    ]),
    "s8kv_verify_window_int8": (_i32, [
        _c_void_p, _i32, _i32, _i32, _i32, _i32,
        _i64, _i64, _i64,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32,
        _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p,
        _i32, _i32, _c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _i64, _i64, _f32, _c_void_p,
        _c_void_p, _i64, _c_void_p,
    ]),
    "s8kv_verify_window_k8v3": (_i32, [
        _c_void_p, _i32, _i32, _i32, _i32, _i32,
        _i64, _i64, _i64,
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i64, _i32,
        _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p,
        _i32, _i32, _c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _i64, _i64, _f32, _c_void_p,
        _c_void_p, _i64, _c_void_p,
    ]),
    "s8kv_attn_varlen_f16": (_i32, [
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i32, _i32, _i32, _i32, _i32, _i32,
        _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _f32, _c_void_p, _i64, _i64, _c_void_p,
    ]),
    "s8kv_rotate_rows": (_i32, [_c_void_p, _i64, _i32, _i64, _i32, _c_void_p, _i64, _c_void_p]),
    "s8kv_quantize_rows_int8": (_i32, [_c_void_p, _i64, _i32, _i64, _i32, _c_void_p, _c_void_p, _c_void_p]),
    "s8kv_quantize_rows_lloydmax3": (_i32, [_c_void_p, _i64, _i32, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p]),
    "s8kv_pack_codes3": (_i32, [_c_void_p, _i64, _i32, _c_void_p, _c_void_p]),
    "s8kv_unpack_codes3": (_i32, [_c_void_p, _i64, _i32, _c_void_p, _c_void_p]),
    "s8kv_snapkv_workspace_size": (_i64, [_i32, _i32]),
    "s8kv_snapkv_scores_paged": (_i32, [
        _c_void_p, _i32, _i64, _i32, _i32, _i32, _c_void_p, _c_void_p, _i64, _i32, _c_void_p, _i32, _f32,
        _c_void_p, _c_void_p, _i64, _c_void_p,
    ]),
    "s8kv_snapkv_scores_dense": (_i32, [
        _c_void_p, _i32, _i64, _i32, _i32, _i32, _c_void_p, _i32, _i64, _i64, _i32, _f32,
        _c_void_p, _c_void_p, _i64, _c_void_p,
    ]),
    "s8kv_gather_slots": (_i32, [
        _i32, ctypes.POINTER(_c_void_p), ctypes.POINTER(_i64), ctypes.POINTER(_i64), _i32, _i32, _i64, _i32,
        _c_void_p, _c_void_p, _i32, _c_void_p,
    ]),
    "s8kv_timing_begin": (_i32, []),
    "s8kv_timing_end": (_i32, [ctypes.POINTER(_i32), ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
    "s8kv_probe_read_tiles": (_i32, [
        _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i32, _c_void_p, _i32, _i32, _c_void_p, _c_void_p,
    ]),
    "s8kv_probe_read_linear": (_i32, [_c_void_p, _i64, _i32, _c_void_p, _c_void_p]),
    "s8kv_copy_blocks": (_i32, [
        _i32, ctypes.POINTER(_c_void_p), ctypes.POINTER(_i64), ctypes.POINTER(_i64), _i32, _i64,
        _c_void_p, _c_void_p, _i32, _c_void_p,
    ]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load the HIP library once and attach the prototypes."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH.name} is not built; run `python -m superl8_serve_amd.build_ext` "
                    "(the quantized paged-KV ops have no other implementation)"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    """Turn a non-zero status into a Python exception (the reference's ops
    raise RuntimeError/ValueError, which PagedKVCache catches,
    kv_cache.py:1183-1189)."""
    if rc == 0:
        return
    msg = (load().s8kv_last_error() or b"").decode(errors="replace")
    if rc == -1:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what} failed ({rc}): {msg}")
