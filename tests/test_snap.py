"""Pins the SnapKV score oracle (oracle/snap.py) on the CPU.

Checks, each independent of the oracle's own formula: the reference's own relation
(tests/test_baselines.py:19-20: a full observation window gives the H2O mass of the
attention oracle divided by G), mass conservation (every window row is a probability
distribution, so the scores of a KV head sum to W), the q = 0 closed form (uniform
causal rows), and float64 loops on tiny inputs. Planted mistakes (GQA sum instead of
mean, a missing causal mask) must fail those checks.
"""
import pytest
import torch

from oracle import snap as osnap
from oracle.attention import materialized


def _qkv(b, hq, hk, n, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((b, hq, n, d), generator=g).to(dtype)
    k = torch.randn((b, hk, n, d), generator=g).to(dtype)
    v = torch.randn((b, hk, n, d), generator=g).to(dtype)
    return q, k, v


def test_full_window_is_h2o_mass_over_groups():
    """tests/test_baselines.py:19-20 of the reference, on the CPU oracles."""
    torch.manual_seed(17)
    q, k, v = _qkv(1, 6, 2, 137, 32, torch.bfloat16, 17)
    _, hh = materialized(q, k, v, value_weighted=False)
    torch.testing.assert_close(osnap.snap_scores(q, k, 137), hh / 3, atol=.025, rtol=.005)


@pytest.mark.parametrize("n,w", [(137, 32), (64, 64), (300, 1), (50, 500)])
def test_mass_conservation(n, w):
    q, k, _ = _qkv(2, 4, 2, n, 16, torch.bfloat16, n + w)
    s = osnap.snap_scores(q, k, w)
    torch.testing.assert_close(s.sum(-1), torch.full((2, 2), float(min(w, n))), rtol=1e-5, atol=1e-5)
    assert (s >= 0).all()


def test_zero_queries_closed_form():
    n, w = 40, 9
    q = torch.zeros((1, 4, n, 8), dtype=torch.float16)
    _, k, _ = _qkv(1, 4, 2, n, 8, torch.float16, 3)
    s = osnap.snap_scores(q, k, w)
    want = torch.tensor([sum(1.0 / (t + 1) for t in range(max(j, n - w), n)) for j in range(n)])
    torch.testing.assert_close(s[0, 0].double(), want.double(), rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(s[0, 1].double(), want.double(), rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("hq,hk,n,d,w,dtype", [(2, 1, 7, 4, 3, torch.bfloat16), (4, 2, 11, 8, 11, torch.float16),
                                               (3, 3, 6, 16, 2, torch.bfloat16)])
def test_brute_force(hq, hk, n, d, w, dtype):
    q, k, _ = _qkv(1, hq, hk, n, d, dtype, n * d)
    q = q * 3
    got = osnap.snap_scores(q, k, w).double()
    want = osnap.snap_scores_brute(q, k, w)
    torch.testing.assert_close(got, want, rtol=2e-5, atol=1e-7)


def test_planted_mistakes_are_caught():
    n, w = 40, 9
    q, k, _ = _qkv(1, 4, 2, n, 8, torch.float16, 5)
    s = osnap.snap_scores(q, k, w)
    summed = s * 2                                       # GQA sum instead of mean
    assert not torch.allclose(summed.sum(-1), torch.full((1, 2), float(w)))
    qz = torch.zeros_like(q)
    nocausal = torch.full((n,), w / n)                   # every window row uniform over all keys
    want = torch.tensor([sum(1.0 / (t + 1) for t in range(max(j, n - w), n)) for j in range(n)])
    assert not torch.allclose(nocausal.double(), want.double(), atol=1e-3)
    assert torch.allclose(osnap.snap_scores(qz, k, w)[0, 0].double(), want.double(), atol=1e-6)
