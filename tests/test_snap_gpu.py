"""SnapKV baseline path on the GPU: fe_snap_scores against the oracle (FP32 scores,
tolerance below), snap_select / flash_snap selections against the oracle's selection, and
torch's fused attention against the attention oracle.

Tolerance of the scores: |gpu - oracle| <= 1e-2 * |oracle| + 1e-6 elementwise, and a mean
relative error below 1e-4. Both sides round an FP32 dot product to the input dtype; their
accumulation orders differ, so a logit near a rounding boundary can land one bf16 ulp
apart (about 0.5% of that row's probability of that key), which the elementwise bound
covers; everything else agrees to FP32 rounding."""
import pytest
import torch

from flash_evict.baselines import flash_attention, flash_snap, snap_scores, snap_select
from oracle import select as osel
from oracle import snap as osnap
from oracle.attention import chunked, materialized

from _helpers import assert_same_selection, seeded_randn

pytestmark = pytest.mark.gpu


def _qk(b, hq, hk, n, d, dtype, seed, layout="contiguous"):
    if layout == "transposed":
        q = seeded_randn((b, n, hq, d), dtype, seed).transpose(1, 2)
        k = seeded_randn((b, n, hk, d), dtype, seed + 1).transpose(1, 2)
    elif layout == "channel_stride2":
        q = seeded_randn((b, hq, n, 2 * d), dtype, seed)[..., ::2]
        k = seeded_randn((b, hk, n, 2 * d), dtype, seed + 1)[..., ::2]
    else:
        q = seeded_randn((b, hq, n, d), dtype, seed)
        k = seeded_randn((b, hk, n, d), dtype, seed + 1)
    return q, k


def _check_scores(got, ref, w):
    got = got.cpu().double()
    ref = ref.double()
    err = (got - ref).abs()
    assert (err <= 1e-2 * ref.abs() + 1e-6).all(), float((err / (ref.abs() + 1e-6)).max())
    assert float((err / (ref.abs() + 1e-6)).mean()) < 1e-4
    torch.testing.assert_close(got.sum(-1), torch.full(got.shape[:-1], float(w), dtype=torch.float64),
                               rtol=1e-4, atol=1e-4)


CASES = [
    # b, hq, hk, n, d, window, dtype, layout
    (1, 6, 2, 137, 32, 32, torch.bfloat16, "contiguous"),       # reference test shape
    (1, 6, 2, 137, 32, 137, torch.bfloat16, "contiguous"),      # full window
    (1, 32, 8, 4096, 128, 32, torch.bfloat16, "transposed"),
    (2, 8, 2, 1000, 64, 128, torch.float16, "contiguous"),
    (1, 28, 4, 8192, 128, 128, torch.bfloat16, "transposed"),   # Qwen-like G = 7
    (1, 4, 4, 300, 80, 7, torch.bfloat16, "contiguous"),
    (1, 4, 2, 200, 48, 16, torch.float16, "channel_stride2"),   # element loads
    (1, 2, 1, 129, 256, 40, torch.bfloat16, "contiguous"),
    (1, 2, 2, 96, 200, 33, torch.bfloat16, "channel_stride2"),
    (1, 2, 1, 50, 64, 500, torch.bfloat16, "contiguous"),       # window > N
    (1, 2, 1, 1, 64, 1, torch.bfloat16, "contiguous"),          # N = 1
]


@pytest.mark.parametrize("b,hq,hk,n,d,w,dtype,layout", CASES)
def test_snap_scores_match_oracle(b, hq, hk, n, d, w, dtype, layout):
    print(f"snap_scores b={b} hq={hq} hk={hk} n={n} d={d} w={w} {dtype} {layout}", flush=True)
    q, k = _qk(b, hq, hk, n, d, dtype, 1000 + n + d, layout)
    got = snap_scores(q, k, w)
    torch.cuda.synchronize()
    ref = osnap.snap_scores(q.cpu(), k.cpu(), w)
    _check_scores(got, ref, min(w, n))


def test_snap_scores_headline_size():
    """Headline shape (B=1, Hq=32, Hkv=8, N=32768, D=128), window 32 and 128."""
    q, k = _qk(1, 32, 8, 32768, 128, torch.bfloat16, 20260910, "transposed")
    for w in (32, 128):
        print(f"snap_scores headline window={w}", flush=True)
        got = snap_scores(q, k, w)
        torch.cuda.synchronize()
        _check_scores(got, osnap.snap_scores(q.cpu(), k.cpu(), w), w)


def test_snap_select_matches_oracle():
    q, k = _qk(1, 32, 8, 4096, 128, torch.bfloat16, 7, "transposed")
    s = snap_scores(q, k, 32)
    for budget, window, kernel in [(409, 32, 5), (64, 128, 5), (1, 32, 5), (4096, 32, 5), (5000, 32, 3),
                                   (100, 32, 1)]:
        idx, keep = snap_select(s, budget, window, kernel)
        ridx, rkeep = osel.snap_select(s.cpu().numpy(), budget, window, kernel)
        assert idx.shape == tuple(ridx.shape) and idx.dtype == torch.int64
        assert torch.equal(idx.cpu(), torch.from_numpy(ridx))
        assert torch.equal(keep.cpu(), torch.from_numpy(rkeep))


def test_flash_snap_end_to_end():
    """The reference's test_window_baseline (tests/test_baselines.py:7-24) on the GPU path,
    with the oracle standing in for the kv_distill comparison."""
    q = seeded_randn((1, 6, 137, 32), torch.bfloat16, 17)
    k = seeded_randn((1, 2, 137, 32), torch.bfloat16, 18)
    v = seeded_randn((1, 2, 137, 32), torch.bfloat16, 19)
    out, scores, indices, mask = flash_snap(q, k, v, 48, 32)
    expected, _ = materialized(q.cpu(), k.cpu(), v.cpu())
    torch.testing.assert_close(out.float().cpu(), expected, atol=.015, rtol=.015)
    assert (~mask).sum(-1).eq(48).all()
    assert not mask[..., -32:].any()
    _, hh = materialized(q.cpu(), k.cpu(), v.cpu(), value_weighted=False)
    torch.testing.assert_close(snap_scores(q, k, 137).cpu(), hh / 3, atol=.025, rtol=.005)
    ref = osnap.snap_scores(q.cpu(), k.cpu(), 32)
    _, rkeep = osel.snap_select(ref.numpy(), 48, 32)
    # the selection ranks the pooled scores of the tokens before the pinned window
    pooled = torch.cat([torch.from_numpy(osel.avg_pool(ref[..., :137 - 32].numpy(), 5)), ref[..., 137 - 32:]], -1)
    assert_same_selection(~mask, torch.from_numpy(rkeep), pooled, 48, recent=32, atol=1e-5, rtol=1e-2)


@pytest.mark.parametrize("hq,hk,n,d", [(8, 2, 1024, 128), (28, 4, 2048, 128), (4, 4, 333, 64)])
def test_flash_attention_matches_oracle(hq, hk, n, d):
    q = seeded_randn((1, hq, n, d), torch.bfloat16, n)
    k = seeded_randn((1, hk, n, d), torch.bfloat16, n + 1)
    v = seeded_randn((1, hk, n, d), torch.bfloat16, n + 2)
    out = flash_attention(q, k, v)
    ref, _ = chunked(q.cpu(), k.cpu(), v.cpu(), value_weighted=False)
    assert (out.float().cpu() - ref).abs().max() <= 2e-2
