"""GPU selection kernels (fe_select: pool, radix select, mask + ascending indices) against the
host routine and the oracle. Integer/index results must be bit-exact."""
import pytest
import torch

from flash_evict import select_tokens
from flash_evict.prefill import _select
from oracle import select as osel

pytestmark = pytest.mark.gpu


CASES = [
    # rows, n, budget, recent, pool, tie-heavy
    (1, 1, 1, 0, 1, False), (1, 1, 1, 1, 3, False), (3, 20, 4, 2, 1, False), (2, 137, 48, 32, 5, False),
    (8, 32768, 1024, 64, 1, False), (8, 32768, 3277, 0, 1, False), (4, 32768, 2048, 64, 5, False),
    (5, 4000, 400, 0, 1, True), (2, 5000, 2500, 100, 3, True), (7, 2049, 2049, 0, 1, False),
    (6, 3000, 1000, 1000, 7, False), (1, 131072, 1024, 64, 1, False), (3, 70000, 17, 5, 9, True),
]


@pytest.mark.parametrize("rows,n,budget,recent,pool,ties", CASES)
def test_gpu_matches_host_and_oracle(rows, n, budget, recent, pool, ties):
    print(f"select rows={rows} n={n} budget={budget} recent={recent} pool={pool} ties={ties}", flush=True)
    g = torch.Generator().manual_seed(n + rows)
    if ties:
        x = torch.randint(0, 7, (rows, n), generator=g).float()
    else:
        x = torch.rand((rows, n), generator=g) * 10
    idx_d, keep_d = select_tokens(x.cuda(), budget, recent=recent, pool_kernel=pool)
    idx_h, keep_h = select_tokens(x, budget, recent=recent, pool_kernel=pool)
    assert torch.equal(idx_d.cpu(), idx_h) and torch.equal(keep_d.cpu(), keep_h)
    if n <= 40000:
        oidx, okeep = osel.select_tokens(x.numpy(), budget, recent=recent, pool_kernel=pool)
        assert torch.equal(idx_h, torch.from_numpy(oidx)) and torch.equal(keep_h, torch.from_numpy(okeep))
    else:
        # large rows: sortedness, counts, suffix and threshold property (size-independent)
        assert torch.equal(idx_h, idx_h.sort(-1).values)
        assert keep_h.sum(-1).eq(budget).all() and (recent == 0 or keep_h[:, n - recent:].all())
        past = x[:, :n - recent]
        if pool > 1 and budget > recent:       # selection ranks the pooled scores
            past = torch.nn.functional.avg_pool1d(past[:, None], pool, stride=1, padding=pool // 2)[:, 0]
        kept_min = torch.where(keep_h[:, :n - recent], past, torch.full_like(past, float("inf"))).min(-1).values
        drop_max = torch.where(~keep_h[:, :n - recent], past, torch.full_like(past, -float("inf"))).max(-1).values
        assert (kept_min >= drop_max).all()


def test_evict_mask_and_scaled_synthetic():
    print("select scaled synthetic 256 x 131072", flush=True)
    x = torch.rand((256, 131072), generator=torch.Generator().manual_seed(1), device="cpu").cuda()
    idx, keep = _select(x, 1024, 64, 1, invert=False)
    idx2, evicted = _select(x, 1024, 64, 1, invert=True)
    assert torch.equal(idx, idx2) and torch.equal(evicted, ~keep)
    hidx, hkeep = _select(x.cpu(), 1024, 64, 1, invert=False)
    assert torch.equal(idx.cpu(), hidx) and torch.equal(keep.cpu(), hkeep)


def test_noncontiguous_and_special_values():
    base = torch.randn(4, 300, 3, generator=torch.Generator().manual_seed(2))
    x = base.cuda()[..., 1]
    assert not x.is_contiguous()
    idx, keep = select_tokens(x, 50, reserved_recent=10, pool_kernel=3)
    hidx, hkeep = select_tokens(base[..., 1], 50, reserved_recent=10, pool_kernel=3)
    assert torch.equal(idx.cpu(), hidx) and torch.equal(keep.cpu(), hkeep)
    s = torch.tensor([0.0, -0.0, float("nan"), -float("inf"), float("inf"), 1.0, -0.0, 0.0]).cuda()
    assert select_tokens(s, 3)[0].tolist() == [2, 4, 5]
    assert select_tokens(s, 5)[0].tolist() == [0, 1, 2, 4, 5]
    lead = torch.randn(2, 3, 4, 64).cuda()
    idx, keep = select_tokens(lead, 8, recent=2)
    assert idx.shape == (2, 3, 4, 8) and keep.shape == (2, 3, 4, 64)
    assert torch.equal(idx.cpu(), select_tokens(lead.cpu(), 8, recent=2)[0])
