"""Head dims 32 and 96 on the fast kernels (fe_attn_fast.hip instantiates D in {32, 64, 96,
128}; other head dims take the generic kernel): the split schedule (prefill, with its
workspace) and the fused single kernel (fe_prefill without a workspace) against the float64
oracle, and against each other. The attention output of the two schedules is bitwise
identical and their importance differs only by FP32 atomic order, as at D = 64 and 128."""
import pytest
import torch

import flash_evict
from flash_evict import prefill
from oracle.attention import chunked
from _helpers import assert_importance_close, seeded_randn, transposed_qkv
from test_schedules_gpu import _run

pytestmark = pytest.mark.gpu

CASES = [
    # n, hq, hk, dtype, causal, decay, window, layout
    (300, 4, 2, torch.bfloat16, True, 0.0, 0, "contiguous"),
    (777, 8, 2, torch.float16, True, 0.05, 0, "transposed"),
    (640, 6, 3, torch.bfloat16, False, 0.0, 200, "contiguous"),
    (65, 2, 1, torch.float16, True, 0.0, 1, "contiguous"),
]


@pytest.mark.parametrize("d", [32, 96])
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
    assert torch.equal(out, o2)
    assert float((imp - i2).abs().max()) <= 2e-6 * float(i2.abs().max())


def test_fast_head_dim_kernels_listed():
    res = {r["kernel"]: r for r in flash_evict.kernel_resources()}
    for d in (32, 96):
        for name in ("attn_fast<bf16,%d>" % d, "fused_fast<bf16,%d>" % d, "replay_fast<bf16,%d>" % d):
            assert name in res
            assert res[name]["scratch_bytes_per_thread"] == 0
    # D = 96 runs twelve waves (three per SIMD), D = 32 eight
    assert res["attn_fast<bf16,96>"]["registers_per_thread"] <= 168
    assert res["attn_fast<bf16,96>"]["max_threads_per_block"] >= 768
