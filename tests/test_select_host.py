"""select_tokens on CPU tensors (the library's native host routine, fe_select_host),
mirroring the reference's CPU tests (tests/test_prefill.py:77-84,149-159) and checked
against the oracle (oracle/select.py)."""
import numpy as np
import pytest
import torch

import flash_evict
from flash_evict import select_tokens
from flash_evict.prefill import _select
from oracle import select as osel


def test_selection_contract():
    # tests/test_prefill.py:77-84
    scores = torch.arange(20.).reshape(1, 1, 20)
    idx, keep = select_tokens(scores, 4, recent=2)
    assert idx.tolist() == [[[16, 17, 18, 19]]]
    assert keep.sum() == 4
    assert idx.dtype == torch.int64 and keep.dtype == torch.bool
    for budget in (0, 21, True, 2.5):
        with pytest.raises(ValueError):
            select_tokens(scores, budget)
    with pytest.raises(ValueError):
        select_tokens(scores, 2, recent=3)


def test_pinning_and_pooling_contract():
    # tests/test_prefill.py:149-159, with SnapKV selection restated in the oracle
    torch.manual_seed(1)
    scores = torch.randn(1, 3, 137)
    idx, keep = select_tokens(scores, 48, reserved_recent=32, pool_kernel=5)
    expected, expected_keep = osel.snap_select(scores.numpy(), 48, 32, 5)
    assert torch.equal(idx, torch.from_numpy(expected)) and torch.equal(keep, torch.from_numpy(expected_keep))
    _, tail = select_tokens(scores, 64, reserved_recent=64, pool_kernel=5)
    assert tail.sum() == 3 * 64 and tail[..., -64:].all()
    for kwargs in ({"recent": True}, {"pool_kernel": 2}, {"recent": 1, "reserved_recent": 2}):
        with pytest.raises(ValueError):
            select_tokens(scores, 64, **kwargs)


def test_value_norm_known_answer():
    # tests/test_quality_adapter.py:18-24: top-2 value L1 norms and the suffix control
    v = torch.tensor([1., -9., 3., -7., 2.]).view(1, 1, 5, 1).expand(1, 2, 5, 2)
    idx, _ = select_tokens(v.abs().sum(-1), 2)
    assert idx.tolist() == [[[1, 3], [1, 3]]]
    idx, _ = select_tokens(v.abs().sum(-1), 2, recent=2)
    assert idx.tolist() == [[[3, 4], [3, 4]]]


@pytest.mark.parametrize("seed", range(40))
def test_host_matches_oracle(seed):
    g = torch.Generator().manual_seed(seed)
    lead = [(3,), (2, 3), (1, 1, 2), ()][seed % 4]
    n = int(torch.randint(1, 700, (1,), generator=g))
    if seed % 3 == 0:
        x = torch.randint(0, 5, lead + (n,), generator=g).float()       # heavy ties
    else:
        x = torch.randn(lead + (n,), generator=g)
    budget = int(torch.randint(1, n + 1, (1,), generator=g))
    recent = int(torch.randint(0, budget + 1, (1,), generator=g))
    pk = [1, 3, 5, 7][seed % 4]
    idx, keep = select_tokens(x, budget, recent=recent, pool_kernel=pk)
    oidx, okeep = osel.select_tokens(x.numpy(), budget, recent=recent, pool_kernel=pk)
    assert torch.equal(idx, torch.from_numpy(oidx))
    assert torch.equal(keep, torch.from_numpy(okeep))
    assert idx.shape == lead + (budget,) and keep.shape == lead + (n,)


def test_noncontiguous_and_dtypes():
    g = torch.Generator().manual_seed(7)
    base = torch.randn(4, 300, 3, generator=g)
    x = base[..., 1]                       # stride 3 along tokens
    idx, keep = select_tokens(x, 50, reserved_recent=10, pool_kernel=3)
    oidx, okeep = osel.select_tokens(x.contiguous().numpy(), 50, reserved_recent=10, pool_kernel=3)
    assert torch.equal(idx, torch.from_numpy(oidx)) and torch.equal(keep, torch.from_numpy(okeep))
    rows = torch.randn(6, 200, generator=g)[::2]    # row stride 400
    idx, _ = select_tokens(rows, 20)
    assert torch.equal(idx, torch.from_numpy(osel.select_tokens(rows.contiguous().numpy(), 20)[0]))
    for dt in (torch.float16, torch.bfloat16, torch.float64):
        y = torch.randn(2, 128, generator=g).to(dt)
        idx, _ = select_tokens(y, 16)
        assert torch.equal(idx, torch.from_numpy(osel.select_tokens(y.float().numpy(), 16)[0]))


def test_special_values():
    x = torch.tensor([0.0, -0.0, float("nan"), -float("inf"), float("inf"), 1.0, -0.0, 0.0])
    assert select_tokens(x, 3)[0].tolist() == [2, 4, 5]
    assert select_tokens(x, 5)[0].tolist() == [0, 1, 2, 4, 5]


def test_eviction_mask_is_inverse_of_keep():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 4, 333, generator=g)
    idx, keep = _select(x, 40, 8, 5, invert=False)
    idx2, evicted = _select(x, 40, 8, 5, invert=True)
    assert torch.equal(idx, idx2) and torch.equal(evicted, ~keep)


def test_budget_equal_recent_and_full_budget():
    x = torch.randn(3, 50)
    idx, keep = select_tokens(x, 10, recent=10, pool_kernel=5)
    assert torch.equal(idx, torch.arange(40, 50).expand(3, 10)) and keep[:, 40:].all() and not keep[:, :40].any()
    idx, keep = select_tokens(x, 50)
    assert torch.equal(idx, torch.arange(50).expand(3, 50)) and keep.all()
    idx, keep = select_tokens(x, 50, recent=50)
    assert torch.equal(idx, torch.arange(50).expand(3, 50)) and keep.all()


def test_empty_leading_dims():
    x = torch.randn(0, 4, 12)
    idx, keep = select_tokens(x, 3)
    assert idx.shape == (0, 4, 3) and keep.shape == (0, 4, 12)


def test_evict_and_prefill_validate_before_device_check():
    q = torch.randn(1, 2, 8, 16)
    k = torch.randn(1, 1, 8, 16)
    with pytest.raises(ValueError, match="evict requires importance scoring"):
        flash_evict.evict(q, k, k, 4, score=False)
    with pytest.raises(ValueError, match="CUDA fp16 or bf16 inputs required"):
        flash_evict.prefill(q.half(), k.half(), k.half())
    with pytest.raises(ValueError, match="shape"):
        flash_evict.prefill(q[0], k[0], k[0])
    with pytest.raises(ValueError, match="nonempty"):
        flash_evict.prefill(q, k[:, :, :4], k[:, :, :4])
    with pytest.raises(ValueError, match="divisible"):
        flash_evict.prefill(torch.randn(1, 3, 8, 16), torch.randn(1, 2, 8, 16), torch.randn(1, 2, 8, 16))
    with pytest.raises(ValueError, match="<= 256"):
        flash_evict.prefill(torch.randn(1, 2, 8, 300), torch.randn(1, 1, 8, 300), torch.randn(1, 1, 8, 300))
    with pytest.raises(ValueError, match="same device and dtype"):
        flash_evict.prefill(q.half(), k.float(), k.half())
