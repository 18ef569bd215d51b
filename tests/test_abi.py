"""The C ABI library loads, exports every declared entry point, and rejects bad arguments
before touching a GPU (CPU-only checks: no device compute is launched here)."""
import ctypes
import os
import re

import pytest

from flash_evict import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flash_evict.h")

FE_ERR_INVALID = -1
FE_ERR_WORKSPACE = -3


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(fe_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_version():
    L = _lib.lib()
    assert L.fe_abi_version() == _lib.ABI_VERSION
    assert os.path.exists(_lib.LIB_PATH)


def test_every_declared_symbol_is_exported():
    syms = declared_symbols()
    assert len(syms) >= 10
    handle = ctypes.CDLL(_lib.LIB_PATH)
    missing = [s for s in syms if not hasattr(handle, s)]
    assert not missing, missing
    # ...and the Python binding declares a signature for each of them
    assert set(syms) <= set(_lib._SIGNATURES), set(syms) - set(_lib._SIGNATURES)


def _err():
    return _lib.lib().fe_last_error().decode()


def test_prefill_rejects_bad_arguments_before_launch():
    L = _lib.lib()
    st = (ctypes.c_int64 * 4)(1, 1, 1, 1)
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    cases = [
        dict(B=0, Hq=1, Hkv=1, N=4, D=8, dtype=1, window=4),      # empty batch
        dict(B=1, Hq=3, Hkv=2, N=4, D=8, dtype=1, window=4),      # Hq % Hkv
        dict(B=1, Hq=2, Hkv=1, N=4, D=257, dtype=1, window=4),    # D > 256
        dict(B=1, Hq=2, Hkv=1, N=4, D=8, dtype=7, window=4),      # dtype
        dict(B=1, Hq=2, Hkv=1, N=4, D=8, dtype=1, window=0),      # window
        dict(B=1, Hq=2, Hkv=1, N=4, D=8, dtype=1, window=5),      # window > N
    ]
    for c in cases:
        rc = L.fe_prefill(p, p, p, p, p, c["B"], c["Hq"], c["Hkv"], c["N"], c["D"], st, st, st, c["dtype"],
                          0.125, 1, 1, 1, 0.0, c["window"], None)
        assert rc == FE_ERR_INVALID, c
        assert _err().startswith("fe_prefill"), _err()
    rc = L.fe_prefill(p, p, p, p, None, 1, 2, 1, 4, 8, st, st, st, 1, 0.125, 1, 1, 1, 0.0, 4, None)
    assert rc == FE_ERR_INVALID and "null" in _err()      # score without an importance buffer
    rc = L.fe_prefill(p, p, p, p, p, 1, 2, 1, 4, 8, st, st, st, 1, float("nan"), 1, 1, 1, 0.0, 4, None)
    assert rc == FE_ERR_INVALID
    rc = L.fe_prefill(p, p, p, p, p, 1, 2, 1, 4, 8, st, st, st, 1, 0.125, 1, 1, 1, -1.0, 4, None)
    assert rc == FE_ERR_INVALID


def test_select_rejects_bad_arguments_before_launch():
    L = _lib.lib()
    p = ctypes.c_void_p(16)
    bad = [(1, 10, 10, 0, 0, 1), (1, 10, 10, 11, 0, 1), (1, 10, 10, 4, 5, 1), (1, 10, 10, 4, 0, 2),
           (1, 10, 10, 4, 0, 0), (2, 10, 9, 4, 0, 1), (-1, 10, 10, 4, 0, 1)]
    for rows, n, stride, budget, recent, pk in bad:
        assert L.fe_select(p, rows, n, stride, budget, recent, pk, p, p, 0, None, 0, None) == FE_ERR_INVALID
        assert L.fe_select_host(p, rows, n, stride, budget, recent, pk, p, p, 0) == FE_ERR_INVALID
    # pooling needs a workspace of the advertised size
    need = L.fe_select_workspace_bytes(3, 100, 10, 2, 5)
    assert need == 3 * 98 * 4
    assert L.fe_select_workspace_bytes(3, 100, 10, 10, 5) == 0      # budget == recent: no pooling
    assert L.fe_select_workspace_bytes(3, 100, 10, 2, 1) == 0
    assert L.fe_select(p, 3, 100, 100, 10, 2, 5, p, p, 0, None, 0, None) == FE_ERR_WORKSPACE
    assert L.fe_select(p, 3, 100, 100, 10, 2, 5, p, p, 0, p, need - 1, None) == FE_ERR_WORKSPACE


def test_zero_and_timing_entry_points():
    L = _lib.lib()
    assert L.fe_zero_f32(None, 5, None) == FE_ERR_INVALID
    assert L.fe_zero_f32(None, 0, None) == 0           # nothing to do, nothing launched
    assert L.fe_fused_timing_enable(0) == 0
    n = ctypes.c_int64(-1)
    ms = ctypes.c_double(-1)
    assert L.fe_fused_timing_read(ctypes.byref(n), ctypes.byref(ms)) == 0
    assert n.value == 0 and ms.value == 0.0


def test_last_error_is_per_call():
    L = _lib.lib()
    L.fe_zero_f32(None, 5, None)
    assert _err()
    assert L.fe_abi_version() == _lib.ABI_VERSION
    assert L.fe_zero_f32(None, 0, None) == 0
    assert _err() == ""


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    import importlib
    monkeypatch.setenv("FLASH_EVICT_LIB", str(tmp_path / "absent.so"))
    mod = importlib.reload(_lib)
    try:
        with pytest.raises(RuntimeError, match="not found"):
            mod.lib()
    finally:
        monkeypatch.delenv("FLASH_EVICT_LIB")
        importlib.reload(_lib)


def test_workspace_sizer_adds_repack_room_only_for_layouts_the_fast_kernels_cannot_read():
    """fe_prefill_workspace_bytes_kv inspects the K/V pointers' alignment and strides (it never
    dereferences them): aligned unit-stride rows of a head dim that is a multiple of 8 need only the
    base workspace; misaligned or channel-strided rows, broadcasts and other head dims add room for
    K and V repacked to D rounded up to 8 channels (256-byte aligned areas)."""
    L = _lib.lib()
    B, Hq, Hkv, N = 1, 8, 2, 1000

    def size(d, kptr, kst, vptr=4096, vst=None, score=1):
        vst = vst or (Hkv * N * d, N * d, d, 1)
        return L.fe_prefill_workspace_bytes_kv(B, Hq, Hkv, N, d, score, ctypes.c_void_p(kptr),
                                               (ctypes.c_int64 * 4)(*kst), ctypes.c_void_p(vptr),
                                               (ctypes.c_int64 * 4)(*vst))

    def repack(d):
        dp = (d + 7) // 8 * 8
        return 2 * ((B * Hkv * N * dp * 2 + 255) // 256 * 256)

    for score in (0, 1):
        base = L.fe_prefill_workspace_bytes(B, Hq, N, score)
        assert size(128, 4096, (Hkv * N * 128, N * 128, 128, 1), score=score) == base
        assert size(128, 4098, (Hkv * N * 128, N * 128, 128, 1), score=score) == base + repack(128)
        assert size(128, 4096, (2 * Hkv * N * 128, 2 * N * 128, 256, 2), score=score) == base + repack(128)
        assert size(128, 4096, (Hkv * 128, 128, 0, 1), score=score) == base + repack(128)      # broadcast over N
        assert size(100, 4096, (Hkv * N * 100, N * 100, 100, 1), vst=(Hkv * N * 100, N * 100, 100, 1),
                    score=score) == base + repack(100)
        assert size(128, 4096, (Hkv * N * 128, N * 128, 128, 1), vptr=4100, score=score) == base + repack(128)
