"""ctypes binding of libflash_evict_hip.so (the C ABI declared in include/flash_evict.h).

No torch C++ ABI is involved: tensors cross the boundary as data pointers, element
strides and the current HIP stream handle. The library is loaded once, from this
package directory; a missing library is an error (there is no fallback path).
"""
import ctypes
import os
import threading

LIB_NAME = "libflash_evict_hip.so"
# FLASH_EVICT_LIB may name another build of the same library (e.g. a tuning variant).
LIB_PATH = os.environ.get("FLASH_EVICT_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

FE_DTYPE_F16 = 0
FE_DTYPE_BF16 = 1
FE_STATIC_BIAS_ROWS = 4194304   # include/flash_evict.h: rows of fe_prefill_static's device buffer

_lock = threading.Lock()
_lib = None

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_I64P = ctypes.POINTER(ctypes.c_int64)

_SIGNATURES = {
    "fe_prefill": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _I64P, _I64P, _I64P,
                                  ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_float, _i64, _vp]),
    "fe_prefill_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i64, ctypes.c_int]),
    "fe_prefill_workspace_bytes_kv": (ctypes.c_size_t, [_i64, _i64, _i64, _i64, _i64, ctypes.c_int, _vp, _I64P,
                                                        _vp, _I64P]),
    "fe_replay_rows": (_i64, [_i64, _i64, ctypes.c_float]),
    "fe_prefill_ws": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _I64P, _I64P, _I64P,
                                     ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_float, _i64, _vp, ctypes.c_size_t, _vp]),
    "fe_prefill_static": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _I64P, _I64P,
                                         _I64P, ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_float, _i64, _vp]),
    "fe_zero_f32": (ctypes.c_int, [_vp, _i64, _vp]),
    "fe_select_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i64, _i64, ctypes.c_int]),
    "fe_select": (ctypes.c_int, [_vp, _i64, _i64, _i64, _i64, _i64, ctypes.c_int, _vp, _vp, ctypes.c_int,
                                 _vp, ctypes.c_size_t, _vp]),
    "fe_select_host": (ctypes.c_int, [_vp, _i64, _i64, _i64, _i64, _i64, ctypes.c_int, _vp, _vp,
                                      ctypes.c_int]),
    "fe_gather_rows": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _I64P, _I64P, ctypes.c_int,
                                      _vp]),
    "fe_snap_scores_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i64, _i64, _i64]),
    "fe_snap_scores": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _I64P, _I64P, ctypes.c_int,
                                      _i64, _vp, ctypes.c_size_t, _vp]),
    "fe_fused_timing_enable": (ctypes.c_int, [ctypes.c_int]),
    "fe_fused_timing_read": (ctypes.c_int, [_I64P, ctypes.POINTER(ctypes.c_double)]),
    "fe_kernel_resources": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_size_t]),
    "fe_last_plan": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_size_t]),
    "fe_last_error": (ctypes.c_char_p, []),
    "fe_abi_version": (ctypes.c_int, []),
}

ABI_VERSION = 1


def lib():
    """Return the loaded library, loading it on first use."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    "flash_evict native library not found at %s; build it with "
                    "`python flash-evict-prefill_amd/build.py` (or __graft_entry__.build())" % LIB_PATH)
            handle = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            if handle.fe_abi_version() != ABI_VERSION:
                raise RuntimeError("flash_evict native library ABI mismatch")
            _lib = handle
    return _lib


def check(rc, what):
    """Raise RuntimeError with the library's message when rc is nonzero."""
    if rc != 0:
        msg = lib().fe_last_error().decode(errors="replace")
        raise RuntimeError("%s failed (%d): %s" % (what, rc, msg))


def strides(t):
    """Element strides of a tensor as a ctypes int64[len] array."""
    st = t.stride()
    return (ctypes.c_int64 * len(st))(*st)
