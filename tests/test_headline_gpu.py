"""GPU parity at the benchmarked headline workload (bench.py's `headline` config).

evict() runs with exactly the arguments bench.py times -- B=1, Hq=32, Hkv=8, N=32768,
D=128, bf16, causal, budget 1024, recency_decay 0.1, reserved_recent 64, all-query
window, seeded N(0,1) inputs drawn on the device as bench.py draws them -- and every
output is compared with the FP32 oracle (oracle/attention.chunked, a restatement of the
reference's materialized path, flash_evict/reference.py:5-25), run in float32 on the GPU:

  * out: every row of every head, max-abs-err <= 2e-2 (bf16 bar of the reference tests
    and of the project's north star);
  * importance: element-wise |kernel - oracle| <= 1e-3 * |oracle| + 1e-30. The oracle
    covers the last 1100 query rows. Earlier rows have recency weight
    exp(-0.1 * (N-1-q)) <= exp(-110), which is exactly 0.0 in FP32 (in the reference
    too), so they add exactly nothing and the restricted oracle is the full one;
  * selection: the kept set equals the oracle's except for near-ties within the
    importance tolerance; the evict mask is the complement of the kept indices.

The same seeded workload with decay 0 (every row replayed: bench.py's full-replay record)
is checked the same way, its importance against the full-row oracle; and the headline shape
in fp16 (the f16 kernels, whose overflow guard is 2^15), output within the fp16 bar 5e-3.
"""
import pytest
import torch

import flash_evict
from oracle.attention import chunked
from oracle import select as osel
from _helpers import assert_same_selection, assert_importance_close, out_err_all_rows

pytestmark = pytest.mark.gpu

B, HQ, HKV, N, D = 1, 32, 8, 32768, 128
SEED = 20260910          # bench.py's generator seed


def _bench_inputs(dtype=torch.bfloat16):
    """q, k, v exactly as bench.py draws them (device generator, same order)."""
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(SEED)
    q = torch.randn((B, HQ, N, D), device=dev, dtype=dtype, generator=gen)
    k = torch.randn((B, HKV, N, D), device=dev, dtype=dtype, generator=gen)
    v = torch.randn((B, HKV, N, D), device=dev, dtype=dtype, generator=gen)
    return q, k, v


def test_headline_evict_matches_oracle():
    print("headline evict(): B=1 Hq=32 Hkv=8 N=32768 D=128 bf16 decay 0.1 budget 1024 recent 64", flush=True)
    q, k, v = _bench_inputs()
    budget, recent, decay = 1024, 64, 0.1
    with torch.inference_mode():
        out, imp, idx, evicted = flash_evict.evict(q, k, v, budget, reserved_recent=recent, pool_kernel=1,
                                                   recency_decay=decay, observation_window=0)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all() and torch.isfinite(imp).all()

    # importance: the last 1100 rows carry every nonzero FP32 weight
    _, ref_imp = chunked(q, k, v, block=1100, want_out=False, recency_decay=decay,
                         query_rows=[(N - 1100, N)])
    rel = assert_importance_close(imp, ref_imp, rtol=1e-3, floor=1e-30)
    print("importance element-wise max rel err %.3e" % rel, flush=True)

    worst = out_err_all_rows(out, q, k, v)
    print("out max-abs-err over all %d rows x %d heads: %.4f" % (N, HQ, worst), flush=True)
    assert worst <= 2e-2

    # selection against the oracle's rule on the oracle's scores
    _, ref_keep = osel.select_tokens(ref_imp.cpu().numpy(), budget, reserved_recent=recent)
    keep = ~evicted
    assert_same_selection(keep, torch.from_numpy(ref_keep), ref_imp.cpu(), budget, recent, rtol=1e-3)
    assert keep.sum(-1).eq(budget).all() and keep[..., -recent:].all()
    assert torch.equal(idx, idx.sort(-1).values)
    assert torch.equal(keep, torch.zeros_like(keep).scatter_(-1, idx, True))
    # and bit-exact against the oracle's rule on the kernel's own scores
    oidx, okeep = osel.select_tokens(imp.cpu().numpy(), budget, reserved_recent=recent)
    assert torch.equal(idx.cpu(), torch.from_numpy(oidx))
    assert torch.equal(keep.cpu(), torch.from_numpy(okeep))


def test_headline_full_replay_matches_oracle():
    """bench.py's full-replay record: the same inputs and selection arguments with decay 0
    (all 32768 rows replayed)."""
    print("headline full replay: decay 0, budget 1024, recent 64", flush=True)
    q, k, v = _bench_inputs()
    budget, recent = 1024, 64
    with torch.inference_mode():
        out, imp, idx, evicted = flash_evict.evict(q, k, v, budget, reserved_recent=recent, recency_decay=0.0)
    torch.cuda.synchronize()
    _, ref_imp = chunked(q, k, v, block=2048, want_out=False)
    rel = assert_importance_close(imp, ref_imp, rtol=1e-3, floor=1e-30)
    print("importance element-wise max rel err %.3e" % rel, flush=True)
    # every query row sums to one: each (b, kv head) row of the H2O mass would be G*N; with
    # value weighting divide the norms back out
    vn = v.float().abs().sum(-1)
    mass = (imp / vn).sum(-1).double()
    torch.testing.assert_close(mass, torch.full_like(mass, float(N * HQ // HKV)), rtol=1e-4, atol=0)
    _, ref_keep = osel.select_tokens(ref_imp.cpu().numpy(), budget, reserved_recent=recent)
    assert_same_selection(~evicted, torch.from_numpy(ref_keep), ref_imp.cpu(), budget, recent, rtol=1e-3)
    # the output is bitwise independent of the scoring options
    with torch.inference_mode():
        out_ns, _ = flash_evict.prefill(q, k, v, score=False)
    assert torch.equal(out, out_ns)


def test_headline_shape_fp16_matches_oracle():
    """The headline shape and arguments in fp16: the f16 instantiations of the attention,
    replay and selection kernels at full size."""
    print("headline shape fp16: decay 0.1, budget 1024, recent 64", flush=True)
    q, k, v = _bench_inputs(torch.float16)
    budget, recent, decay = 1024, 64, 0.1
    with torch.inference_mode():
        out, imp, idx, evicted = flash_evict.evict(q, k, v, budget, reserved_recent=recent, pool_kernel=1,
                                                   recency_decay=decay, observation_window=0)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16
    assert torch.isfinite(out).all() and torch.isfinite(imp).all()
    _, ref_imp = chunked(q, k, v, block=1100, want_out=False, recency_decay=decay, query_rows=[(N - 1100, N)])
    rel = assert_importance_close(imp, ref_imp, rtol=1e-3, floor=1e-30)
    print("importance element-wise max rel err %.3e" % rel, flush=True)
    worst = out_err_all_rows(out, q, k, v)
    print("out max-abs-err over all %d rows x %d heads: %.4f" % (N, HQ, worst), flush=True)
    assert worst <= 5e-3
    _, ref_keep = osel.select_tokens(ref_imp.cpu().numpy(), budget, reserved_recent=recent)
    keep = ~evicted
    assert_same_selection(keep, torch.from_numpy(ref_keep), ref_imp.cpu(), budget, recent, rtol=1e-3)
    assert keep.sum(-1).eq(budget).all() and keep[..., -recent:].all()
    oidx, okeep = osel.select_tokens(imp.cpu().numpy(), budget, reserved_recent=recent)
    assert torch.equal(idx.cpu(), torch.from_numpy(oidx))
    assert torch.equal(keep.cpu(), torch.from_numpy(okeep))
