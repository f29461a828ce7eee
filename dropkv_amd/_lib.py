"""ctypes binding of ``libdropkv_amd.so`` (the C ABI in ``include/dropkv_amd.h``).

The library is loaded from this package directory.  There is no fallback:
if it is missing, every op raises ``RuntimeError`` telling how to build it.
"""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdropkv_amd.so")

DROPKV_BF16 = 1
DROPKV_FP16 = 2
DROPKV_FP32 = 3

_c_i64 = ctypes.c_int64
_c_vp = ctypes.c_void_p
_c_int = ctypes.c_int
_c_size = ctypes.c_size_t
_c_float = ctypes.c_float

# name -> (restype, argtypes); mirrors include/dropkv_amd.h
_SIGNATURES = {
    "dropkv_version": (_c_int, []),
    "dropkv_last_error": (ctypes.c_char_p, []),
    "dropkv_supported_head_dims": (_c_int, [ctypes.POINTER(_c_i64), _c_int]),
    "dropkv_scores_workspace_bytes": (_c_size, [_c_i64] * 7),
    "dropkv_scores": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_int,
                               _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                               _c_float, _c_int, _c_int, _c_i64, _c_vp, _c_vp, _c_size, _c_vp]),
    "dropkv_scores_debug_state": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                           _c_vp, _c_vp, _c_vp]),
    "dropkv_select_workspace_bytes": (_c_size, [_c_i64, _c_i64]),
    "dropkv_select": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_vp, _c_size,
                               _c_vp]),
    "dropkv_compact": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                _c_vp, _c_i64, _c_vp, _c_vp, _c_vp]),
    "dropkv_compact2": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64,
                                 _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64,
                                 _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp, _c_vp]),
    "dropkv_evict_workspace_bytes": (_c_size, [_c_i64] * 7),
    "dropkv_evict": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_int,
                              _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                              _c_float, _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_i64,
                              _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_size, _c_vp]),
    "dropkv_evict_noalloc": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_int,
                                      _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                      _c_float, _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_i64,
                                      _c_vp, _c_vp, _c_vp, _c_vp, _c_vp]),
    "dropkv_evict_ld": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_int,
                                 _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                 _c_float, _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_i64,
                                 _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_vp, _c_size, _c_vp]),
    "dropkv_append": (_c_int, [_c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                               _c_vp, _c_vp, _c_i64, _c_i64, _c_vp]),
    "dropkv_set_tail_select": (_c_int, [_c_int, _c_i64, _c_i64]),
    "dropkv_timing_enable": (_c_int, [_c_int]),
    "dropkv_timing_read": (_c_int, [ctypes.POINTER(ctypes.c_double), _c_int]),
    "dropkv_selftest_mfma": (_c_int, [_c_vp, _c_vp]),
    "dropkv_decode_workspace_bytes": (_c_size, [_c_i64] * 5),
    "dropkv_decode_attention": (_c_int, [_c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,
                                         _c_vp, _c_vp, _c_vp, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                         _c_float, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_size, _c_vp]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

# Size of the static per-GPU scratch of dropkv_evict_noalloc
# (DROPKV_NOALLOC_SCRATCH_BYTES in include/dropkv_amd.h).
NOALLOC_SCRATCH_BYTES = 32 << 20

# Leading bytes of a dropkv_evict workspace that must be zero when the
# workspace is first used (DROPKV_SYNC_BYTES in include/dropkv_amd.h).
SYNC_BYTES = 4096

# Largest head dimension the scoring kernels take (the generic kernels'
# limit; include/dropkv_amd.h, dropkv_scores).
MAX_HEAD_DIM = 4096

_lib = None
_lock = threading.Lock()


def load():
    """Load and return the ctypes handle (raises RuntimeError if absent)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"DropKV HIP library not found at {LIB_PATH}; build it with "
                    "`python -m dropkv_amd._build` (hipcc, gfx950)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().dropkv_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


_head_dims = None


def supported_head_dims() -> tuple[int, ...]:
    """Head dimensions of the matrix-core scoring kernels (asked once; the
    library does not change while loaded).  Other head dimensions up to
    ``MAX_HEAD_DIM`` and fp32 inputs are scored by the library's generic
    kernels."""
    global _head_dims
    if _head_dims is None:
        buf = (_c_i64 * 16)()
        n = load().dropkv_supported_head_dims(buf, 16)
        _head_dims = tuple(int(buf[i]) for i in range(min(n, 16)))
    return _head_dims
