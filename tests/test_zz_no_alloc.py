"""fe_prefill_static, the allocation-free entry point, against fe_prefill_ws (the entry
point it is a variant of) through the C ABI.

fe_prefill_static runs the same split attention + replay kernels with the replay-bias
buffer in a static device array of the library instead of a caller workspace. Bar: the
attention output is bitwise equal to fe_prefill_ws's; the importance equals it up to the
order of FP32 atomic additions (element-wise rtol 2e-6 + 1e-6 of the row maximum, the bar of
tests/test_schedules_gpu.py). Two calls in a row, the second smaller, so a result left in
the shared buffer by the first call cannot leak into the second. The size limit is checked
on the host before anything is launched (CPU test).
"""
import ctypes

import pytest
import torch

from flash_evict import _lib
from flash_evict.prefill import _DTYPES

from _helpers import seeded_randn, transposed_qkv

FE_ERR_WORKSPACE = -3


def _args(q, k, v, out, imp, causal, weighted, decay, window):
    b, h, n, d = q.shape
    hk = k.shape[1]
    return (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), imp.data_ptr(), b, h, hk, n, d,
            _lib.strides(q), _lib.strides(k), _lib.strides(v), _DTYPES[q.dtype], d ** -0.5, int(causal),
            int(weighted), 1, decay, min(n, window or n))


def _run(q, k, v, causal, weighted, decay, window, static):
    b, h, n, d = q.shape
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    imp = torch.empty((b, k.shape[1], n), dtype=torch.float32, device=q.device)
    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    args = _args(q, k, v, out, imp, causal, weighted, decay, window)
    if static:
        rc = L.fe_prefill_static(*args, stream)
    else:
        nbytes = L.fe_prefill_workspace_bytes(b, h, n, 1)
        ws = torch.empty(nbytes // 4, dtype=torch.float32, device=q.device)
        rc = L.fe_prefill_ws(*args, ws.data_ptr(), nbytes, stream)
    _lib.check(rc, "fe_prefill_static" if static else "fe_prefill_ws")
    torch.cuda.synchronize()
    return out, imp


@pytest.mark.gpu
def test_static_entry_matches_workspace_entry_on_two_calls():
    cases = [
        # larger call first, then smaller ones (fewer rows, another dtype and head dim; D = 120 runs
        # the two-row-tile attention kernel below its tile dim)
        ((1, 32, 8, 4096, 128, torch.bfloat16, 20261201), dict(causal=True, weighted=True, decay=0.0, window=0)),
        ((2, 8, 2, 1000, 64, torch.float16, 20261202), dict(causal=True, weighted=True, decay=0.05, window=0)),
        ((1, 8, 2, 777, 120, torch.bfloat16, 20261203), dict(causal=True, weighted=True, decay=0.0, window=300)),
    ]
    for (b, hq, hk, n, d, dt, seed), kw in cases:
        print("fe_prefill_static vs fe_prefill_ws: B=%d Hq=%d Hkv=%d N=%d D=%d %s %s" % (b, hq, hk, n, d, dt, kw),
              flush=True)
        q, k, v = transposed_qkv(b, n, hq, hk, d, dt, seed)
        out_s, imp_s = _run(q, k, v, static=True, **kw)
        out_w, imp_w = _run(q, k, v, static=False, **kw)
        assert torch.equal(out_s, out_w)
        tol = 2e-6 * imp_w.abs() + 1e-6 * imp_w.abs().amax(-1, keepdim=True)
        assert bool(((imp_s - imp_w).abs() <= tol).all())
        assert torch.isfinite(out_s).all() and float(imp_s.sum()) > 0


@pytest.mark.gpu
def test_static_entry_without_score_and_at_head_dim_96():
    """score=0 needs no buffer; D=96 runs the split schedule's two-row-tile kernel at tile dim 96."""
    q = seeded_randn((1, 4, 300, 96), torch.bfloat16, 11)
    k = seeded_randn((1, 2, 300, 96), torch.bfloat16, 12)
    v = seeded_randn((1, 2, 300, 96), torch.bfloat16, 13)
    out_s, imp_s = _run(q, k, v, True, True, 0.0, 0, static=True)
    out_w, imp_w = _run(q, k, v, True, True, 0.0, 0, static=False)
    assert torch.equal(out_s, out_w)
    torch.testing.assert_close(imp_s, imp_w, rtol=2e-6, atol=1e-6 * float(imp_w.abs().max()))
    L = _lib.lib()
    out = torch.empty_like(q)
    args = list(_args(q, k, v, out, out, True, True, 0.0, 0))
    args[4] = None
    args[17] = 0                                   # score = 0: importance may be NULL
    _lib.check(L.fe_prefill_static(*args, torch.cuda.current_stream().cuda_stream), "fe_prefill_static")
    torch.cuda.synchronize()
    assert torch.equal(out, out_w)


@pytest.mark.gpu
def test_static_entry_under_graph_capture_allocates_nothing():
    """fe_prefill_static for a caller that cannot allocate: one eager call (it looks up the
    static buffer and the kernels' occupancy on this device), more eager calls that leave the
    device's free memory unchanged, then the call captured in a HIP graph (torch.cuda.CUDAGraph)
    and replayed three times with eager work and synchronisations between the replays. The
    eager calls and every replay match fe_prefill_ws: bitwise output, importance up to FP32
    atomic order (each replay zeroes the importance and the work-item counters with fill kernels,
    not memset nodes)."""
    b, hq, hk, n, d = 1, 8, 2, 2048, 128
    print("fe_prefill_static under graph capture: B=%d Hq=%d Hkv=%d N=%d D=%d bf16" % (b, hq, hk, n, d), flush=True)
    q, k, v = transposed_qkv(b, n, hq, hk, d, torch.bfloat16, 20261210)
    out_w, imp_w = _run(q, k, v, True, True, 0.05, 0, static=False)
    tol = 2e-6 * imp_w.abs() + 1e-6 * imp_w.abs().amax(-1, keepdim=True)
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    imp = torch.empty((b, hk, n), dtype=torch.float32, device=q.device)
    L = _lib.lib()
    args = _args(q, k, v, out, imp, True, True, 0.05, 0)
    _lib.check(L.fe_prefill_static(*args, torch.cuda.current_stream().cuda_stream), "fe_prefill_static")
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(3):
        _lib.check(L.fe_prefill_static(*args, torch.cuda.current_stream().cuda_stream), "fe_prefill_static")
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0
    assert torch.equal(out, out_w)
    assert bool(((imp - imp_w).abs() <= tol).all())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = L.fe_prefill_static(*args, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "fe_prefill_static (captured)")
    for r in range(3):
        out.zero_()
        imp.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        print("replay %d" % r, flush=True)
        assert torch.equal(out, out_w)
        assert bool(((imp - imp_w).abs() <= tol).all())
    del g


def test_static_entry_rejects_sizes_beyond_its_buffer():
    """B*Hq*N above FE_STATIC_BIAS_ROWS fails with FE_ERR_WORKSPACE before any HIP call
    (the pointers below are never dereferenced)."""
    L = _lib.lib()
    st = (ctypes.c_int64 * 4)(1, 1, 1, 1)
    p = ctypes.c_void_p(16)
    R = _lib.FE_STATIC_BIAS_ROWS
    for b, hq, n in [(1, 32, R // 32 + 1), (1, 1, R + 1), (R + 1, 1, 1), (2, 64, R // 64)]:
        rc = L.fe_prefill_static(p, p, p, p, p, b, hq, 1, n, 64, st, st, st, 1, 0.125, 1, 1, 1, 0.0, n, None)
        assert rc == FE_ERR_WORKSPACE, (b, hq, n, rc)
        msg = L.fe_last_error().decode()
        assert "static replay-bias buffer" in msg and str(R) in msg, msg


_RESERVE_SCRIPT = r"""
import sys
sys.path[:0] = sys.argv[1:]
import torch, flash_evict
from flash_evict import _lib
from flash_evict.prefill import _DTYPES
dev = torch.device("cuda", 0)
g = torch.Generator(device=dev).manual_seed(5)
q = torch.randn((1, 8, 1024, 128), device=dev, generator=g).to(torch.bfloat16)
k = torch.randn((1, 2, 1024, 128), device=dev, generator=g).to(torch.bfloat16)
v = torch.randn((1, 2, 1024, 128), device=dev, generator=g).to(torch.bfloat16)
for _ in range(2):
    out, imp = flash_evict.prefill(q, k, v)
torch.cuda.synchronize()
torch.cuda.empty_cache()
free_after_ws = torch.cuda.mem_get_info()[0]
L = _lib.lib()
st = _lib.strides
rc = L.fe_prefill_static(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), imp.data_ptr(), 1, 8, 2, 1024,
                         128, st(q), st(k), st(v), _DTYPES[q.dtype], 128 ** -0.5, 1, 1, 1, 0.0, 1024,
                         torch.cuda.current_stream().cuda_stream)
torch.cuda.synchronize()
torch.cuda.empty_cache()
free_after_static = torch.cuda.mem_get_info()[0]
print("RESERVED_BY_STATIC", rc, free_after_ws - free_after_static)
"""


@pytest.mark.gpu
def test_static_buffer_reserved_only_by_static_entry():
    """The static workspace (16 MiB + 4 KiB per GPU) lives in a code object of its own: a process
    holds it only once it calls fe_prefill_static, not from its first prefill() call. Checked in a
    fresh process (device free memory after prefill() calls, then after one static call)."""
    import os
    import subprocess
    import sys
    print("static buffer reservation: fresh process, prefill() twice, then fe_prefill_static once", flush=True)
    here = os.path.dirname(os.path.abspath(__file__))
    paths = [os.path.join(os.path.dirname(here), "flash-evict-prefill_amd"), os.path.dirname(here)]
    res = subprocess.run([sys.executable, "-c", _RESERVE_SCRIPT] + paths, capture_output=True, text=True,
                         timeout=110)
    line = [x for x in res.stdout.splitlines() if x.startswith("RESERVED_BY_STATIC")]
    assert res.returncode == 0 and line, res.stdout + res.stderr
    _, rc, delta = line[0].split()
    assert int(rc) == 0
    assert int(delta) >= 16 * 2**20, "fe_prefill_static reserved %d bytes: its buffer was already held" % int(delta)
