"""The two schedules of fe_prefill on the fast layouts agree: the fused single kernel
(fe_prefill, no workspace) and the split attention + replay kernels (fe_prefill_ws, the
path flash_evict.prefill takes). Both are checked against the oracle elsewhere through
prefill(); this pins the workspace-free entry point to the same results.

Where both schedules run the same attention kernel the output is bitwise identical (the
replay does not touch it) and the importance differs only by the order of FP32 atomic
additions. At tile dims 96 and 128 the split schedule runs the two-row-tile attention kernel,
whose reference max is the exact max of a row's first 32 keys instead of 64: outputs then
agree within the bound of two roundings of P and importance within FP32 summation error
(assert_schedules_agree derives both)."""
import pytest
import torch

from flash_evict import _lib
from flash_evict.prefill import _DTYPES

from _helpers import assert_schedules_agree, seeded_randn, split_runs_two_row_tiles, transposed_qkv

pytestmark = pytest.mark.gpu


def _ws_layout(b, h, n, score):
    """fe_prefill_workspace_bytes: B*Hq*N floats of replay biases (scoring calls), then 4 KiB
    of work-item counters for the dynamic schedule (eight queues per kernel, one counter per
    128-byte line) at the next 256-byte boundary."""
    bias = b * h * n * 4 if score else 0
    return (bias + 255) // 256 * 256 + 4096


def _run(q, k, v, causal, weighted, decay, window, use_ws, ws_bytes=None, score=True, scale=None):
    b, h, n, d = q.shape
    hk = k.shape[1]
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    imp = torch.empty((b, hk, n), dtype=torch.float32, device=q.device)
    L = _lib.lib()
    w = min(n, window or n)
    stream = torch.cuda.current_stream().cuda_stream
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), imp.data_ptr() if score else None, b, h, hk,
            n, d, _lib.strides(q), _lib.strides(k), _lib.strides(v), _DTYPES[q.dtype],
            d ** -0.5 if scale is None else scale, int(causal),
            int(weighted), int(score), decay, w)
    if use_ws:
        nbytes = L.fe_prefill_workspace_bytes(b, h, n, int(score))
        assert nbytes == _ws_layout(b, h, n, score)
        if ws_bytes is not None:
            nbytes = ws_bytes
        ws = torch.empty(max(nbytes, 4) // 4, dtype=torch.float32, device=q.device)
        rc = L.fe_prefill_ws(*args, ws.data_ptr(), nbytes, stream)
    else:
        rc = L.fe_prefill(*args, stream)
    _lib.check(rc, "prefill")
    torch.cuda.synchronize()
    return out, imp


CASES = [
    # b, hq, hk, n, d, dtype, causal, weighted, decay, window, layout
    (1, 32, 8, 4096, 128, torch.bfloat16, True, True, 0.1, 0, "transposed"),
    (2, 8, 2, 1000, 64, torch.float16, True, False, 0.0, 0, "contiguous"),
    (1, 28, 4, 3000, 128, torch.bfloat16, True, True, 0.0, 128, "contiguous"),
    (1, 4, 4, 777, 128, torch.bfloat16, False, True, 0.05, 300, "transposed"),
    (1, 8, 1, 65, 64, torch.float16, True, True, 0.0, 1, "contiguous"),
    # more work items than resident workgroups: the queues' heavy and light parts and stealing
    # (attention 1024 items, replay 2048 with every row replayed)
    (1, 32, 8, 16384, 128, torch.bfloat16, True, True, 0.0, 0, "contiguous"),
    # bf16 at tile dim 64 (D = 48: partial)
    (1, 8, 2, 1000, 64, torch.bfloat16, True, True, 0.1, 0, "transposed"),
    (2, 4, 2, 777, 48, torch.bfloat16, True, False, 0.0, 0, "contiguous"),
]


@pytest.mark.parametrize("b,hq,hk,n,d,dtype,causal,weighted,decay,window,layout", CASES)
def test_split_and_fused_schedules_agree(b, hq, hk, n, d, dtype, causal, weighted, decay, window, layout):
    print(f"schedules b={b} hq={hq} hk={hk} n={n} d={d} {dtype} causal={causal} window={window}", flush=True)
    if layout == "transposed":
        q, k, v = transposed_qkv(b, n, hq, hk, d, dtype, n + d)
    else:
        q = seeded_randn((b, hq, n, d), dtype, n)
        k = seeded_randn((b, hk, n, d), dtype, n + 1)
        v = seeded_randn((b, hk, n, d), dtype, n + 2)
    o1, i1 = _run(q, k, v, causal, weighted, decay, window, use_ws=False)
    o2, i2 = _run(q, k, v, causal, weighted, decay, window, use_ws=True)
    if not split_runs_two_row_tiles(d):
        assert torch.equal(o1, o2)
    assert_schedules_agree(o2, o1, i2, i1, v, hq, hk)


def test_small_workspace_falls_back_to_fused():
    q = seeded_randn((1, 8, 512, 128), torch.bfloat16, 1)
    k = seeded_randn((1, 2, 512, 128), torch.bfloat16, 2)
    v = seeded_randn((1, 2, 512, 128), torch.bfloat16, 3)
    o1, i1 = _run(q, k, v, True, True, 0.0, 0, use_ws=False)
    L = _lib.lib()
    out = torch.empty_like(q)
    imp = torch.empty((1, 2, 512), dtype=torch.float32, device="cuda")
    ws = torch.empty(16, dtype=torch.float32, device="cuda")
    rc = L.fe_prefill_ws(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), imp.data_ptr(), 1, 8, 2, 512,
                         128, _lib.strides(q), _lib.strides(k), _lib.strides(v), _DTYPES[q.dtype], 128 ** -0.5, 1, 1,
                         1, 0.0, 512, ws.data_ptr(), 64, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "fe_prefill_ws")
    torch.cuda.synchronize()
    assert torch.equal(out, o1)
    # same fused kernel; only the FP32 atomic order can differ between the two runs
    assert float((imp - i1).abs().max()) <= 2e-6 * float(i1.abs().max())


@pytest.mark.parametrize("b,hq,hk,n,d,dtype,causal,weighted,decay,window,layout", CASES)
def test_dynamic_and_static_schedules_agree(b, hq, hk, n, d, dtype, causal, weighted, decay, window, layout):
    """The dynamic schedule (the whole workspace: work items taken from a counter, heaviest
    first) against the static one (a workspace of the replay biases only: item = workgroup
    index). Each item is computed the same way whichever workgroup takes it, so the output is
    bitwise equal, with and without scoring, and the importance equal up to FP32 atomic order."""
    print(f"dynamic vs static b={b} hq={hq} hk={hk} n={n} d={d} {dtype} causal={causal} window={window}", flush=True)
    q = seeded_randn((b, hq, n, d), dtype, 3 * n + d)
    k = seeded_randn((b, hk, n, d), dtype, 3 * n + d + 1)
    v = seeded_randn((b, hk, n, d), dtype, 3 * n + d + 2)
    o_dyn, i_dyn = _run(q, k, v, causal, weighted, decay, window, use_ws=True)
    o_st, i_st = _run(q, k, v, causal, weighted, decay, window, use_ws=True, ws_bytes=b * hq * n * 4)
    assert torch.equal(o_dyn, o_st)
    assert float((i_dyn - i_st).abs().max()) <= 3e-6 * float(i_st.abs().max())
    # attention only: counters alone (dynamic) against no workspace (static)
    o_dyn0, _ = _run(q, k, v, causal, weighted, decay, window, use_ws=True, score=False)
    o_st0, _ = _run(q, k, v, causal, weighted, decay, window, use_ws=True, ws_bytes=0, score=False)
    assert torch.equal(o_dyn0, o_st0)
    assert torch.equal(o_dyn0, o_dyn)


def _last_plan():
    import ctypes
    buf = ctypes.create_string_buffer(256)
    _lib.check(_lib.lib().fe_last_plan(buf, len(buf)), "fe_last_plan")
    return buf.value.decode()


@pytest.mark.parametrize("d", [64, 32])
def test_small_grid_kernel_matches_the_eight_wave_kernel(d):
    """Tile dims 32 and 64 run the 4-wave small-grid attention kernel when the 8-wave kernel's
    items would fill at most one round of its resident workgroups. Both compute every row tile
    the same way (one row tile per wave, 64-key tiles), so batch 0 of a launch big enough for
    the 8-wave kernel equals the small launch of the same data bitwise; the importance differs
    only by FP32 atomic order. fe_last_plan names the kernels each launch ran."""
    hq, hk, n = 4, 2, 2048
    print(f"small-grid vs 8-wave attention kernel d={d} hq={hq} hk={hk} n={n}", flush=True)
    q = seeded_randn((40, hq, n, d), torch.bfloat16, 17 + d)
    k = seeded_randn((40, hk, n, d), torch.bfloat16, 18 + d)
    v = seeded_randn((40, hk, n, d), torch.bfloat16, 19 + d)
    o_small, i_small = _run(q[:1], k[:1], v[:1], True, True, 0.0, 0, use_ws=True)
    small_plan = _last_plan()
    o_big, i_big = _run(q, k, v, True, True, 0.0, 0, use_ws=True)
    big_plan = _last_plan()
    # every row replayed: the small launch replays as items of the attention launch (ascending
    # row groups); in the launch whose attention items fill every resident workgroup, the heaviest
    # row groups' replay runs as items, the others on the replay kernel
    assert small_plan == "attn_fast4<bf16,%d> with replay items" % d, small_plan
    assert big_plan == "attn_fast<bf16,%d> with replay items + replay_fast<bf16,%d>" % (d, d), big_plan
    assert torch.equal(o_small, o_big[:1])
    scale = i_big[:1].abs().amax(dim=-1, keepdim=True)
    assert ((i_small - i_big[:1]).abs() <= 2e-6 * i_big[:1].abs() + 1e-6 * scale).all()


@pytest.mark.parametrize("d,dtype", [(128, torch.bfloat16), (120, torch.float16), (96, torch.bfloat16)])
def test_small_grid_kernel_at_tile_dims_96_and_128(d, dtype):
    """Tile dims 96 and 128 run the 4-wave small-grid attention kernel instead of the two-row-tile
    kernel when the latter's 16-row-tile items would fill at most 1.5 rounds of its workgroups (one
    per CU). It computes every row tile as the fused single kernel does (one row tile per wave,
    reference max over the first 64 keys): output bitwise equal to fe_prefill's, importance up to
    FP32 atomic order."""
    b, hq, hk, n = 1, 8, 2, 3000
    print(f"small-grid attention kernel d={d} {dtype} b={b} hq={hq} hk={hk} n={n}", flush=True)
    q = seeded_randn((b, hq, n, d), dtype, 23 + d)
    k = seeded_randn((b, hk, n, d), dtype, 24 + d)
    v = seeded_randn((b, hk, n, d), dtype, 25 + d)
    o_ws, i_ws = _run(q, k, v, True, True, 0.0, 0, use_ws=True)
    plan = _last_plan()
    tile = (d + 31) // 32 * 32
    e = "bf16" if dtype == torch.bfloat16 else "f16"
    part = "" if d == tile else ",partial"
    # a causal launch this small replays as items of the attention launch
    assert plan == "attn_fast4<%s,%d%s> with replay items" % (e, tile, part), plan
    o_fu, i_fu = _run(q, k, v, True, True, 0.0, 0, use_ws=False)
    assert torch.equal(o_ws, o_fu)
    assert float((i_ws - i_fu).abs().max()) <= 3e-6 * float(i_fu.abs().max())


@pytest.mark.parametrize("b,hq,hk,n,d,dtype,causal,decay,window", [
    # (launches of more than 1.5 rounds of the two-row-tile kernel's items, below which the
    # small-grid kernel runs instead)
    (1, 32, 8, 8192, 128, torch.bfloat16, True, 0.1, 0),       # llama8k's schedule: 1050 rows replayed
    (2, 8, 2, 13000, 120, torch.float16, True, 0.0, 200),     # partial tile dim, ragged N, fp16
    (1, 16, 2, 12400, 96, torch.bfloat16, False, 0.0, 100),   # tile dim 96, non-causal
    # every row replayed: the heaviest row groups as items, the replay kernel for the others
    (1, 32, 8, 8192, 128, torch.bfloat16, True, 0.0, 0),
    (4, 12, 4, 5000, 104, torch.float16, True, 0.0, 0),
    # the one-row-tile kernel (fused_fast_kernel) at tile dims 32 and 64: 8 waves, the 4-wave
    # small grid (launches whose attention items fill every resident workgroup)
    (1, 32, 8, 8192, 64, torch.bfloat16, True, 0.1, 0),
    (1, 4, 2, 32768, 64, torch.float16, True, 0.0, 0),
    (1, 32, 8, 16384, 32, torch.bfloat16, False, 0.0, 300),
    (1, 16, 4, 8192, 56, torch.float16, True, 0.0, 100),
])
def test_replay_items_match_the_replay_kernel(b, hq, hk, n, d, dtype, causal, decay, window):
    """Short observation windows run the replay as work items of the attention launch (the whole
    workspace), on both fast attention kernels; longer ones run the heaviest row groups' replay
    as items and the others on the replay kernel; a workspace of the replay biases alone runs the
    separate replay kernel for every row. Same attention items and the same replay
    arithmetic: the output is bitwise equal and the importance equal up to FP32 atomic order.
    fe_last_plan names the schedule each launch ran."""
    print(f"replay items vs replay kernel b={b} hq={hq} hk={hk} n={n} d={d} {dtype} causal={causal} "
          f"decay={decay} window={window}", flush=True)
    q = seeded_randn((b, hq, n, d), dtype, 5 * n + d)
    k = seeded_randn((b, hk, n, d), dtype, 5 * n + d + 1)
    v = seeded_randn((b, hk, n, d), dtype, 5 * n + d + 2)
    o_it, i_it = _run(q, k, v, causal, True, decay, window, use_ws=True)
    plan_it = _last_plan()
    o_rk, i_rk = _run(q, k, v, causal, True, decay, window, use_ws=True, ws_bytes=b * hq * n * 4)
    plan_rk = _last_plan()
    # at most a quarter of the rows replayed (fe_replay_rows): all of them as items
    short = 4 * _lib.lib().fe_replay_rows(n, min(n, window or n), decay) <= n
    assert " with replay items" in plan_it, plan_it
    assert plan_it.endswith(" with replay items") == short, plan_it
    assert " + replay_fast<" in plan_rk and " with replay items" not in plan_rk, plan_rk
    assert torch.equal(o_it, o_rk)
    assert float((i_it - i_rk).abs().max()) <= 3e-6 * float(i_rk.abs().max())


@pytest.mark.parametrize("d,decay", [(128, 0.1), (128, 0.0), (64, 0.1), (64, 0.0)])
def test_replay_item_runs_its_dependency_when_the_wait_runs_out(monkeypatch, d, decay):
    """A replay item whose attention item has not published its biases within the wait's bound
    runs that attention item itself (attention items are idempotent: whoever runs one writes the
    same output and biases). FLASH_EVICT_REPLAY_WAIT=0 makes every replay item take that path at
    once; the results equal the replay kernel's (bitwise output, importance up to FP32 atomic
    order). Decay 0.1: every replayed row as items; decay 0: the heaviest row groups as items,
    the others on the replay kernel."""
    b, hq, hk, n = 1, 32, 8, 8192
    print(f"replay items running their dependencies b={b} hq={hq} hk={hk} n={n} d={d} decay={decay}", flush=True)
    q = seeded_randn((b, hq, n, d), torch.bfloat16, 71)
    k = seeded_randn((b, hk, n, d), torch.bfloat16, 72)
    v = seeded_randn((b, hk, n, d), torch.bfloat16, 73)
    o_rk, i_rk = _run(q, k, v, True, True, decay, 0, use_ws=True, ws_bytes=b * hq * n * 4)
    monkeypatch.setenv("FLASH_EVICT_REPLAY_WAIT", "0")
    o_it, i_it = _run(q, k, v, True, True, decay, 0, use_ws=True)
    assert " with replay items" in _last_plan()
    assert torch.equal(o_it, o_rk)
    assert float((i_it - i_rk).abs().max()) <= 3e-6 * float(i_rk.abs().max())
