"""Head dims other than 64 and 128 on the fast kernels (fe_attn_fast.hip: tile dims 32, 64,
96, ..., 256; a head dim that is a multiple of 8 below its tile dim runs the PARTIAL
instantiation, which reads zeros past channel D and stores D channels): the split schedule
(prefill, with its workspace) and the fused single kernel (fe_prefill without a workspace)
against the float64 oracle, and against each other: where both schedules run the same
attention kernel their outputs are bitwise identical and their importance differs only by
FP32 atomic order; at tile dims 96 and 128 the split schedule runs the two-row-tile kernel and
the schedules agree within the derived rounding bound (assert_schedules_agree). Other head
dims take the generic kernel."""
import pytest
import torch

import flash_evict
from flash_evict import prefill
from oracle.attention import chunked
from _helpers import (assert_importance_close, assert_schedules_agree, seeded_randn, split_runs_two_row_tiles,
                      transposed_qkv)
from test_schedules_gpu import _last_plan, _run

pytestmark = pytest.mark.gpu

CASES = [
    # n, hq, hk, dtype, causal, decay, window, layout
    (300, 4, 2, torch.bfloat16, True, 0.0, 0, "contiguous"),
    (777, 8, 2, torch.float16, True, 0.05, 0, "transposed"),
    (640, 6, 3, torch.bfloat16, False, 0.0, 200, "contiguous"),
    (65, 2, 1, torch.float16, True, 0.0, 1, "contiguous"),
]


@pytest.mark.parametrize("d", [32, 96, 24, 80, 120, 160, 200, 256])
@pytest.mark.parametrize("n,hq,hk,dtype,causal,decay,window,layout", CASES)
def test_fast_head_dims(d, n, hq, hk, dtype, causal, decay, window, layout):
    print(f"fast head dim d={d} n={n} hq={hq} hk={hk} {dtype} causal={causal} window={window}", flush=True)
    if layout == "transposed":
        q, k, v = transposed_qkv(1, n, hq, hk, d, dtype, n + d)
    else:
        q = seeded_randn((1, hq, n, d), dtype, n + d)
        k = seeded_randn((1, hk, n, d), dtype, n + d + 1)
        v = seeded_randn((1, hk, n, d), dtype, n + d + 2)
    out, imp = prefill(q, k, v, causal=causal, recency_decay=decay, observation_window=window)
    ref_out, ref_imp = chunked(q, k, v, causal=causal, recency_decay=decay, observation_window=window,
                               block=512, dtype=torch.float64)
    assert (out.double() - ref_out.to(out.device)).abs().max().item() <= (2e-2 if dtype == torch.bfloat16 else 5e-3)
    assert_importance_close(imp, ref_imp, rtol=1e-3, floor=1e-30)
    o2, i2 = _run(q, k, v, causal, True, decay, window, use_ws=False)
    if not split_runs_two_row_tiles(d):
        assert torch.equal(out, o2)
    assert_schedules_agree(out, o2, imp, i2, v, hq, hk)


@pytest.mark.parametrize("d", [8, 40, 80, 120, 200, 248])
def test_partial_head_dim_reads_stop_at_d(d):
    # K and V rows of 2D channels whose channels past D are NaN: a read past channel D would
    # put NaN into the logits (K) or, through the output store, into a neighbouring row
    print(f"partial head dim d={d}: NaN past channel D", flush=True)
    n, hq, hk = 333, 4, 2
    q = seeded_randn((1, hq, n, d), torch.bfloat16, 70 + d)
    wide_k = torch.full((1, hk, n, 2 * d), float("nan"), dtype=torch.bfloat16, device="cuda")
    wide_v = torch.full((1, hk, n, 2 * d), float("nan"), dtype=torch.bfloat16, device="cuda")
    wide_k[..., :d] = seeded_randn((1, hk, n, d), torch.bfloat16, 71 + d)
    wide_v[..., :d] = seeded_randn((1, hk, n, d), torch.bfloat16, 72 + d)
    k, v = wide_k[..., :d], wide_v[..., :d]
    assert k.stride(2) == 2 * d and k.data_ptr() % 16 == 0
    for use_ws in (True, False):
        out, imp = _run(q, k, v, True, True, 0.0, 0, use_ws=use_ws)
        assert torch.isfinite(out).all() and torch.isfinite(imp).all()
        ref_out, ref_imp = chunked(q, k.contiguous(), v.contiguous(), block=512, dtype=torch.float64)
        assert (out.double() - ref_out.to(out.device)).abs().max().item() <= 2e-2
        assert_importance_close(imp, ref_imp, rtol=1e-3, floor=1e-30)


@pytest.mark.parametrize("d,scale,decay", [
    (64, 0.69, 0.0),       # |scale| * log2 e just below 1
    (64, 0.7, 0.02),       # just above 1
    (48, None, 0.0),
    (32, -0.3, 0.05),
    (40, -1.0, 0.02),
])
def test_replay_scales_bf16(d, scale, decay):
    """bf16 replay at tile dims 32 and 64 under the split schedule for scales around and above
    1/log2(e) and negative ones, with and without a recency decay: against the float64 oracle
    and against the fused single kernel (same attention kernel: bitwise-equal outputs)."""
    n, hq, hk = 1500, 8, 2
    print(f"bf16 replay d={d} scale={scale} decay={decay}", flush=True)
    q = seeded_randn((1, hq, n, d), torch.bfloat16, 90 + d)
    k = seeded_randn((1, hk, n, d), torch.bfloat16, 91 + d)
    v = seeded_randn((1, hk, n, d), torch.bfloat16, 92 + d)
    out, imp = prefill(q, k, v, scale=scale, recency_decay=decay)
    tile = (d + 31) // 32 * 32
    plan = _last_plan()
    # a launch this small replays as items of the attention launch (causal, tile dims 32 and 64)
    assert plan == "attn_fast4<bf16,%d%s> with replay items" % (tile, "" if d == tile else ",partial"), plan
    ref_out, ref_imp = chunked(q, k, v, scale=scale, recency_decay=decay, block=512, dtype=torch.float64)
    assert (out.double() - ref_out.to(out.device)).abs().max().item() <= 2e-2
    assert_importance_close(imp, ref_imp, rtol=1e-3, floor=1e-30)
    o2, i2 = _run(q, k, v, True, True, decay, 0, use_ws=False, scale=(d ** -0.5 if scale is None else scale))
    assert torch.equal(out, o2)
    assert_schedules_agree(out, o2, imp, i2, v, hq, hk)


def test_fast_head_dim_kernels_listed():
    res = {r["kernel"]: r for r in flash_evict.kernel_resources()}
    for d in (32, 96, 160, 256):
        for part in ("", ",partial"):
            for name in ("attn_fast<bf16,%d%s>" % (d, part), "fused_fast<bf16,%d%s>" % (d, part),
                         "replay_fast<bf16,%d%s>" % (d, part)):
                assert name in res
                assert res[name]["scratch_bytes_per_thread"] == 0
    # D = 96 runs twelve waves (three per SIMD), D = 32 eight, D = 256 four (one per SIMD)
    assert res["attn_fast<bf16,96>"]["registers_per_thread"] <= 168
    assert res["attn_fast<bf16,96>"]["max_threads_per_block"] >= 768
    assert res["attn_fast<bf16,256>"]["max_threads_per_block"] >= 256
