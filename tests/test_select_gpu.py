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
    (2, 5000, 300, 10, 11, False), (2, 3000, 200, 0, 201, False), (2, 20000, 700, 3, 5, True),
    # pooling tiles of 1024 and 4096 outputs (the launch halves the tile until the grid has 1024
    # blocks; the small cases above take 256)
    (64, 20064, 1000, 64, 5, False), (300, 16448, 500, 64, 3, False),
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


def _host_equal(x, budget, recent=0, pool=1):
    idx_d, keep_d = select_tokens(x.cuda(), budget, recent=recent, pool_kernel=pool)
    idx_h, keep_h = select_tokens(x, budget, recent=recent, pool_kernel=pool)
    assert torch.equal(idx_d.cpu(), idx_h) and torch.equal(keep_d.cpu(), keep_h)


@pytest.mark.parametrize("n,budget,recent", [(16384, 1024, 0), (16385, 1024, 0), (16384 + 64, 1024, 64),
                                             (16385 + 64, 1024, 64), (9000, 900, 0)])
def test_schedule_boundary(n, budget, recent):
    """The last row length staged whole in LDS and the first sampled one (past = n - recent)."""
    print(f"select boundary n={n} budget={budget} recent={recent}", flush=True)
    x = torch.rand((3, n), generator=torch.Generator().manual_seed(n)) * 10
    _host_equal(x, budget, recent)


@pytest.mark.parametrize("n,decay", [(131072, 0.1), (65536, 0.01), (200003, 1.0)])
def test_sampled_schedule_on_importance_like_rows(n, decay):
    """Rows shaped like decayed importance: a dense run of large scores at the end of the row,
    a noise floor elsewhere, an attention sink at token 0."""
    print(f"select importance-like n={n} decay={decay}", flush=True)
    g = torch.Generator().manual_seed(n)
    t = torch.arange(n - 1, -1, -1, dtype=torch.float64)
    x = ((-decay * t).exp() + torch.rand((4, n), generator=g, dtype=torch.float64) * 1e-3).float()
    x[:, 0] = 5.0
    for budget, recent in ((1024, 64), (1024, 0), (17, 5), (n // 10, 64)):
        _host_equal(x, budget, recent)


@pytest.mark.parametrize("n", [70000, 131072])
def test_sampled_schedule_ties_at_threshold(n):
    """Quantised scores (about n/1000 equal keys per value): the bracket holds the threshold,
    many candidates tie at it, and they are kept by index, lowest first."""
    print(f"select ties at threshold n={n}", flush=True)
    g = torch.Generator().manual_seed(n + 7)
    x = (torch.rand((3, n), generator=g) * 1000).floor() / 1000
    for budget, recent in ((1024, 64), (5000, 0), (333, 3)):
        _host_equal(x, budget, recent)


@pytest.mark.parametrize("n,n_tied", [(70000, 5), (70000, 64), (131072, 65), (131072, 9)])
def test_sampled_schedule_few_ties_at_threshold(n, n_tied):
    """Distinct scores except n_tied equal ones straddling the budget: 3 of them rank inside
    it, so the 3 lowest-index copies are kept. Up to 64 tied candidates are ranked by index
    from an LDS list, more by a radix select over their indices."""
    print(f"select few ties n={n} tied={n_tied}", flush=True)
    g = torch.Generator().manual_seed(n + n_tied)
    recent = 64
    budget = 1024
    K = budget - recent
    x = torch.randperm(n, generator=g).float() / n                # distinct scores
    past = x[: n - recent]
    order = past.argsort(descending=True)
    tied = order[K - 3: K - 3 + n_tied]                            # ranks K-3 .. K-4+n_tied
    past[tied] = past[order[K - 1]].item()
    _host_equal(x.unsqueeze(0).repeat(2, 1), budget, recent)
    idx_h, _ = select_tokens(x.unsqueeze(0), budget, recent=recent)
    kept_tied = sorted(set(idx_h[0].tolist()) & set(tied.tolist()))
    assert kept_tied == sorted(tied.tolist())[:3]


def test_sampled_schedule_denormals_and_zeros():
    """Long rows whose threshold falls among FP32 denormals and signed zeros: the sampled
    schedule classifies by float compares, which must order denormals and tie -0 with +0."""
    print("select denormals and zeros", flush=True)
    g = torch.Generator().manual_seed(21)
    n = 40000
    tiny = torch.tensor(1e-40, dtype=torch.float32)              # a denormal
    x = (torch.randint(-200, 200, (4, n), generator=g).float() * tiny)
    x[1, ::3] = -0.0
    x[2] = torch.where(torch.rand((n,), generator=g) < 0.5, -tiny * 3, tiny * 3)
    x[3, ::7] = float("nan")
    for budget, recent in ((1024, 64), (20000, 0), (39999, 1)):
        _host_equal(x, budget, recent)


def test_rows_past_the_bitmap():
    """Rows longer than the sampled schedule's kept-key bitmap (2^18 past scores) take the
    radix passes over HBM."""
    print("select rows past the bitmap", flush=True)
    x = torch.rand((2, 300000), generator=torch.Generator().manual_seed(9))
    _host_equal(x, 1024, 64)


def test_sampled_schedule_fallbacks():
    """Brackets that cannot hold the threshold (a large budget, heavy ties) take the radix
    passes over HBM: the same result. Long rows need no workspace without pooling."""
    print("select fallbacks", flush=True)
    g = torch.Generator().manual_seed(3)
    x = torch.rand((2, 50000), generator=g)
    _host_equal(x, 40000, 100)                                    # large K
    _host_equal(torch.randint(0, 3, (2, 80000), generator=g).float(), 5000, 0)   # ties
    import ctypes
    from flash_evict import _lib
    L = _lib.lib()
    xd = x.cuda()
    idx = torch.empty((2, 1024), dtype=torch.int64, device="cuda")
    keep = torch.empty((2, 50000), dtype=torch.bool, device="cuda")
    assert L.fe_select_workspace_bytes(2, 50000, 1024, 0, 1) == 0
    _lib.check(L.fe_select(xd.data_ptr(), 2, 50000, 50000, 1024, 0, 1, idx.data_ptr(), keep.data_ptr(), 0,
                           None, 0, torch.cuda.current_stream().cuda_stream), "fe_select")
    hidx, hkeep = select_tokens(x, 1024)
    assert torch.equal(idx.cpu(), hidx) and torch.equal(keep.cpu(), hkeep)


def test_sampled_schedule_special_values():
    print("select special values, long rows", flush=True)
    g = torch.Generator().manual_seed(4)
    x = torch.randn((3, 70001), generator=g)
    x[0, ::997] = float("nan")
    x[1, ::1013] = float("inf")
    x[1, 5::1013] = -float("inf")
    x[2, ::2] = -0.0
    x[2, 1::2] = 0.0
    for budget, recent in ((1024, 64), (3000, 0)):
        _host_equal(x, budget, recent)
