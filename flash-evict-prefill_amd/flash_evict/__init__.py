"""MI355X-native flash_evict prefill hot path.

`prefill`, `select_tokens` and `evict` keep the signatures and contracts of the
reference package (anishesg/flash-evict-prefill, flash_evict/__init__.py:1-3); the work
runs in gfx950 HIP kernels behind the C ABI of libflash_evict_hip.so.
"""
import json

from .prefill import prefill, evict, select_tokens
from .cache import gather_tokens


def kernel_resources():
    """Registers, LDS and scratch of every device kernel in the library (needs a GPU).

    Stands in for the reference benchmark's `_prefill.device_caches` resource dump
    (scripts/benchmark.py:104-111).
    """
    import ctypes
    from . import _lib
    buf = ctypes.create_string_buffer(1 << 16)
    _lib.check(_lib.lib().fe_kernel_resources(buf, len(buf)), "fe_kernel_resources")
    return json.loads(buf.value.decode())


__all__ = ["prefill", "evict", "select_tokens", "gather_tokens", "kernel_resources"]
