"""GPU parity on the five workload configurations of the project brief.

Tolerances (stated per config): attention output max-abs-err <= 2e-2 (bf16) / 5e-3 (fp16);
importance relative error <= 1e-3 (atomic reordering); selected index sets identical except
for near-ties within that tolerance. The oracle runs in FP32 -- on the CPU for the small
configs, and (same code, oracle/attention.chunked) on the GPU in float32 for the large ones.
"""
import math

import pytest
import torch

import flash_evict
from oracle.attention import chunked, materialized
from oracle import select as osel
from _helpers import assert_same_selection, seeded_randn

pytestmark = pytest.mark.gpu


def rel_err(a, b):
    return float((a.double() - b.double()).abs().max() / b.double().abs().max().clamp_min(1e-30))


def test_tiny_fp16_dense():
    print("config tiny", flush=True)
    g = 731
    q = seeded_randn((1, 4, 512, 64), torch.float16, g)
    k = seeded_randn((1, 4, 512, 64), torch.float16, g + 1)
    v = seeded_randn((1, 4, 512, 64), torch.float16, g + 2)
    out, imp, idx, evicted = flash_evict.evict(q, k, v, 64)
    ref_out, ref_imp = materialized(q.cpu(), k.cpu(), v.cpu())
    assert (out.float().cpu() - ref_out).abs().max() <= 5e-3
    torch.testing.assert_close(imp.cpu(), ref_imp, rtol=1e-3, atol=1e-5)
    _, ref_keep = osel.select_tokens(ref_imp.numpy(), 64)
    assert_same_selection(~evicted, torch.from_numpy(ref_keep), ref_imp, 64, rtol=1e-3)
    assert (~evicted).sum(-1).eq(64).all()


def test_edge_noncausal_noncontiguous_extreme_zero_rows():
    print("config edge", flush=True)
    b, n, hq, hk, d = 2, 4000, 8, 2, 128
    q = seeded_randn((b, n, hq, d), torch.float16, 20260910, scale=30).transpose(1, 2)
    k = seeded_randn((b, n, hk, d), torch.float16, 20260911, scale=30).transpose(1, 2)
    v = seeded_randn((b, n, hk, d), torch.float16, 20260912).transpose(1, 2).clone()
    gz = torch.Generator().manual_seed(5)
    zero_rows = torch.randperm(n, generator=gz)[: n // 10]
    v[:, :, zero_rows.cuda()] = 0
    v = v.transpose(1, 2).contiguous().transpose(1, 2)      # noncontiguous [B,N,H,D] view again
    assert not q.is_contiguous() and not k.is_contiguous() and not v.is_contiguous()
    budget = n // 10
    out, imp, idx, evicted = flash_evict.evict(q, k, v, budget, causal=False, value_weighted=False)
    # H2O mass: every query row sums to 1, so each (b, kv head) row sums to G * N
    torch.testing.assert_close(imp.sum(-1).cpu().double(), torch.full((b, hk), float(n * hq // hk), dtype=torch.float64),
                               rtol=1e-5, atol=0)
    ref_out, ref_imp = chunked(q.float(), k.float(), v.float(), causal=False, value_weighted=False, block=512)
    assert torch.isfinite(out).all() and torch.isfinite(imp).all()
    assert (out.float() - ref_out).abs().max() <= 5e-3
    assert rel_err(imp, ref_imp) <= 1e-3
    _, ref_keep = osel.select_tokens(ref_imp.cpu().numpy(), budget)
    assert_same_selection(~evicted, torch.from_numpy(ref_keep), ref_imp.cpu(), budget, atol=1e-2, rtol=1e-3)


def test_edge_and_llama_configs_through_workspace_free_entry_point():
    """The same two configs through fe_prefill (the single fused kernel, no workspace)."""
    from test_schedules_gpu import _run
    print("config edge + llama8k, fe_prefill", flush=True)
    b, n, hq, hk, d = 2, 4000, 8, 2, 128
    q = seeded_randn((b, n, hq, d), torch.float16, 20260910, scale=30).transpose(1, 2)
    k = seeded_randn((b, n, hk, d), torch.float16, 20260911, scale=30).transpose(1, 2)
    v = seeded_randn((b, n, hk, d), torch.float16, 20260912).transpose(1, 2).clone()
    v[:, :, torch.randperm(n, generator=torch.Generator().manual_seed(5))[: n // 10].cuda()] = 0
    v = v.transpose(1, 2).contiguous().transpose(1, 2)
    out, imp = _run(q, k, v, False, False, 0.0, 0, use_ws=False)
    ref_out, ref_imp = chunked(q.float(), k.float(), v.float(), causal=False, value_weighted=False, block=512)
    assert (out.float() - ref_out).abs().max() <= 5e-3
    assert rel_err(imp, ref_imp) <= 1e-3

    n, hq, hk = 8192, 32, 8
    q, k = _outlier_qk(n, hq, hk, d, 20260910)
    v = seeded_randn((1, hk, n, d), torch.bfloat16, 20260913)
    out, imp = _run(q, k, v, True, True, 0.1, 0, use_ws=False)
    ref_out, ref_imp = chunked(q, k, v, block=1024, recency_decay=0.1)
    assert (out.float() - ref_out).abs().max() <= 2e-2
    assert rel_err(imp, ref_imp) <= 1e-3


def _outlier_qk(n, hq, hk, d, seed):
    q = torch.randn((1, hq, n, d), generator=torch.Generator().manual_seed(seed))
    k = torch.randn((1, hk, n, d), generator=torch.Generator().manual_seed(seed + 1))
    ch = torch.randperm(d, generator=torch.Generator().manual_seed(seed + 2))[:4]
    q[..., ch] *= 8
    k[..., ch] *= 8
    return q.to(torch.bfloat16).cuda(), k.to(torch.bfloat16).cuda()


def test_llama_8k_outliers():
    print("config llama8k", flush=True)
    n, hq, hk, d = 8192, 32, 8, 128
    q, k = _outlier_qk(n, hq, hk, d, 20260910)
    v = seeded_randn((1, hk, n, d), torch.bfloat16, 20260913)
    kw = dict(recency_decay=0.1)
    out, imp, idx, evicted = flash_evict.evict(q, k, v, 1024, reserved_recent=64, **kw)
    ref_out, ref_imp = chunked(q, k, v, block=1024, **kw)          # FP32 on the GPU
    assert (out.float() - ref_out).abs().max() <= 2e-2
    assert rel_err(imp, ref_imp) <= 1e-3
    _, ref_keep = osel.select_tokens(ref_imp.cpu().numpy(), 1024, reserved_recent=64)
    assert_same_selection(~evicted, torch.from_numpy(ref_keep), ref_imp.cpu(), 1024, 64, rtol=1e-3)
    assert (~evicted)[..., -64:].all()


def test_qwen_32k_window_pool():
    print("config qwen32k", flush=True)
    n, hq, hk, d = 32768, 28, 4, 128
    q = seeded_randn((1, hq, n, d), torch.bfloat16, 20260910)
    k = seeded_randn((1, hk, n, d), torch.bfloat16, 20260911)
    v = seeded_randn((1, hk, n, d), torch.bfloat16, 20260912)
    kw = dict(observation_window=128)
    out, imp, idx, evicted = flash_evict.evict(q, k, v, 2048, reserved_recent=64, pool_kernel=5, **kw)
    # importance comes only from the last 128 queries: cheap to recompute exactly
    _, ref_imp = chunked(q, k, v, block=128, want_out=False, **kw)
    assert rel_err(imp, ref_imp) <= 1e-3
    # full attention output for all N rows: check first, middle and last blocks
    rows = [(0, 256), (16384 - 128, 16384 + 128), (n - 256, n)]
    ref_out, _ = chunked(q, k, v, block=256, query_rows=rows, value_weighted=False, **kw)
    for r0, r1 in rows:
        assert (out[:, :, r0:r1].float() - ref_out[:, :, r0:r1]).abs().max() <= 2e-2, (r0, r1)
    assert torch.isfinite(out).all()
    _, ref_keep = osel.select_tokens(ref_imp.cpu().numpy(), 2048, reserved_recent=64, pool_kernel=5)
    pooled = torch.nn.functional.avg_pool1d(ref_imp[..., :n - 64].reshape(-1, 1, n - 64).cpu(), 5, 1, 2)
    assert_same_selection(~evicted, torch.from_numpy(ref_keep), torch.cat(
        (pooled.reshape(1, hk, n - 64), ref_imp[..., n - 64:].cpu()), -1), 2048, 64, rtol=1e-3)


def test_long_131k_planted_keys():
    print("config long131k", flush=True)
    n, hq, hk, d = 131072, 32, 8, 128
    g = torch.Generator().manual_seed(20260910)
    q = torch.randn((1, hq, n, d), generator=g)
    k = torch.randn((1, hk, n, d), generator=g)
    v = torch.randn((1, hk, n, d), generator=g)
    u = torch.randn((hk, d), generator=g)
    u = u / u.norm(dim=-1, keepdim=True)
    a = bb = math.sqrt(6 * math.sqrt(d))          # a*b/sqrt(D) = 6
    gq = hq // hk
    q[0, :, n - 128:] += a * u.repeat_interleave(gq, 0)[:, None, :]
    p0 = n // 4
    k[0, :, p0:p0 + 64] = bb * u[:, None, :] + torch.randn((hk, 64, d), generator=g)
    q, k, v = (t.to(torch.bfloat16).cuda() for t in (q, k, v))
    out, imp, idx, evicted = flash_evict.evict(q, k, v, 1024, reserved_recent=64, recency_decay=0.1)
    assert torch.isfinite(out).all() and torch.isfinite(imp).all()
    keep = ~evicted
    assert keep[..., p0:p0 + 64].all(), keep[..., p0:p0 + 64].sum(-1)
    assert keep.sum(-1).eq(1024).all() and keep[..., -64:].all()
    assert torch.equal(idx, idx.sort(-1).values)
    # spot-check: the output of the last query block against the FP32 oracle
    ref_out, _ = chunked(q[:, :4], k[:, :1], v[:, :1], block=128, query_rows=[(n - 128, n)], value_weighted=False)
    assert (out[:, :4, n - 128:].float() - ref_out[:, :, n - 128:]).abs().max() <= 2e-2
