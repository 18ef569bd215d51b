"""Pins the KV compaction gather oracle (oracle/gather.py) and checks the host side of
flash_evict.gather_tokens (argument rules), on the CPU.

The oracle is checked against torch.gather (a library routine) on in-range indices,
against brute-force loops including out-of-range indices, and against the two identities
the reference's call sites rely on: indices arange(N) return the cache, and the
uniform_recent indices arange(N-K, N).expand(B, H, K) (quality_adapter.py:41-43) return
the suffix slice.
"""
import numpy as np
import pytest
import torch

from oracle import gather as og


def _cache(b, h, n, d, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn((b, h, n, d), generator=g)


def test_identity_indices_return_the_cache():
    x = _cache(2, 3, 17, 5, 1)
    idx = torch.arange(17).expand(2, 3, 17)
    assert np.array_equal(og.gather_tokens(x.numpy(), idx.numpy()), x.numpy())


def test_uniform_recent_indices_return_the_suffix():
    x = _cache(1, 4, 40, 8, 2)
    budget = 9
    idx = torch.arange(40 - budget, 40).expand(1, 4, budget)
    assert np.array_equal(og.gather_tokens(x.numpy(), idx.numpy()), x[:, :, 40 - budget:].numpy())


@pytest.mark.parametrize("b,h,n,d,k", [(1, 1, 1, 1, 1), (2, 3, 50, 7, 13), (1, 8, 300, 16, 300), (3, 2, 9, 4, 20)])
def test_matches_torch_gather(b, h, n, d, k):
    x = _cache(b, h, n, d, n + k)
    g = torch.Generator().manual_seed(k)
    idx = torch.randint(0, n, (b, h, k), generator=g)
    ref = x.gather(2, idx[..., None].expand(b, h, k, d))
    assert np.array_equal(og.gather_tokens(x.numpy(), idx.numpy()), ref.numpy())


def test_brute_force_with_out_of_range_indices():
    x = _cache(2, 2, 6, 3, 5)
    idx = torch.tensor([[[0, 5, -1, 6], [2, 2, 100, 1]], [[5, 4, 3, -7], [0, 1, 2, 3]]])
    got = og.gather_tokens(x.numpy(), idx.numpy())
    for b in range(2):
        for h in range(2):
            for j in range(4):
                t = int(idx[b, h, j])
                want = x[b, h, t].numpy() if 0 <= t < 6 else np.zeros(3, np.float32)
                assert np.array_equal(got[b, h, j], want)


def test_planted_head_swap_is_caught():
    """Applying the indices of head h to head h+1 (a plausible indexing slip) must fail
    the torch.gather check."""
    x = _cache(1, 3, 30, 4, 9)
    idx = torch.randint(0, 30, (1, 3, 7), generator=torch.Generator().manual_seed(3))
    wrong = og.gather_tokens(x.numpy(), idx.roll(1, dims=1).numpy())
    ref = x.gather(2, idx[..., None].expand(1, 3, 7, 4)).numpy()
    assert not np.array_equal(wrong, ref)


def test_gather_tokens_rejects_bad_arguments():
    from flash_evict import gather_tokens
    x = torch.zeros(1, 2, 8, 4)
    with pytest.raises(ValueError):
        gather_tokens(x[0], torch.zeros(1, 2, 3, dtype=torch.int64))
    with pytest.raises(ValueError):
        gather_tokens(x, torch.zeros(1, 3, 3, dtype=torch.int64))
    with pytest.raises(ValueError):
        gather_tokens(x, torch.zeros(1, 2, 3, dtype=torch.int32))
    with pytest.raises(ValueError):   # CPU tensors: no host fallback
        gather_tokens(x, torch.zeros(1, 2, 3, dtype=torch.int64))
