"""GPU parity tests mirroring the reference's tests/test_prefill.py (anishesg/flash-evict-prefill).

Each test follows the reference test of the same name (file:line noted) with the
materialized oracle restated in oracle/attention.py. Inputs are drawn on the CPU from
seeded generators so the oracle and the kernel see identical values. Tolerances are the
reference's own.
"""
import math

import pytest
import torch

from flash_evict import evict, prefill, select_tokens
from oracle import analytic
from oracle.attention import materialized
from oracle import select as oselect
from _helpers import assert_same_selection, seeded_randn, transposed_qkv

pytestmark = pytest.mark.gpu


def _oracle(q, k, v, **kw):
    return materialized(q.cpu(), k.cpu(), v.cpu(), **kw)


# tests/test_prefill.py:14-41
@pytest.mark.parametrize("n,h,hk,d,dtype,causal", [
    (512, 4, 4, 64, torch.float16, True),
    (1024, 4, 2, 64, torch.bfloat16, True),
    (4096, 4, 2, 128, torch.bfloat16, True),
    (137, 6, 2, 80, torch.float16, False),
    (65, 4, 1, 32, torch.bfloat16, True),
    (1, 2, 1, 16, torch.float16, True),
])
def test_exact(n, h, hk, d, dtype, causal):
    print(f"test_exact n={n} h={h} hk={hk} d={d} {dtype} causal={causal}", flush=True)
    q, k, v = transposed_qkv(1, n, h, hk, d, dtype, seed=731)
    out, importance = prefill(q, k, v, causal=causal)
    torch.cuda.synchronize()
    expected, scores = _oracle(q, k, v, causal=causal)
    atol = 0.012 if dtype == torch.bfloat16 else 0.002
    torch.testing.assert_close(out.float().cpu(), expected, atol=atol, rtol=0.006)
    torch.testing.assert_close(importance.cpu(), scores, atol=3e-3, rtol=3e-4)
    for rate in (.05, .1, .2):
        budget = max(1, math.ceil(n * rate))
        idx, keep = select_tokens(importance, budget)
        refidx, refkeep = select_tokens(scores, budget)          # host path on the oracle
        oidx, okeep = oselect.select_tokens(scores.numpy(), budget)
        assert torch.equal(refkeep, torch.from_numpy(okeep))
        assert torch.equal(refidx, torch.from_numpy(oidx))
        assert_same_selection(keep, refkeep, scores, budget, atol=3e-3, rtol=3e-4)
        if torch.equal(keep.cpu(), refkeep):
            assert torch.equal(idx.cpu(), refidx)
    # H2O mass (value_weighted=False), and conservation sum_k mass = N * Hq / Hkv.
    _, hh = prefill(q, k, v, causal=causal, value_weighted=False)
    _, hh_ref = _oracle(q, k, v, causal=causal, value_weighted=False)
    torch.testing.assert_close(hh.cpu(), hh_ref, atol=3e-5, rtol=3e-4)
    torch.testing.assert_close(hh.sum(-1).cpu(), torch.full((1, hk), n * h / hk), rtol=1e-5, atol=1e-4)


# tests/test_prefill.py:44-59
def test_extreme_logits_batches_and_zero_values():
    print("test_extreme_logits_batches_and_zero_values", flush=True)
    q = seeded_randn((2, 4, 97, 64), torch.float16, 11, scale=15)
    k = seeded_randn((2, 2, 97, 64), torch.float16, 12, scale=15)
    v = seeded_randn((2, 2, 97, 64), torch.float16, 13)
    out, scores, idx, mask = evict(q, k, v, 17, recent=5)
    ref, refscore = _oracle(q, k, v)
    torch.testing.assert_close(out.float().cpu(), ref, atol=0.004, rtol=0.006)
    torch.testing.assert_close(scores.cpu(), refscore, atol=0.01, rtol=0.001)
    assert torch.isfinite(scores).all()
    assert (~mask).sum(-1).eq(17).all()
    assert not mask[..., -5:].any()
    assert idx.shape == (2, 2, 17) and idx.dtype == torch.int64
    assert torch.equal(idx, torch.sort(idx, -1).values)
    zero, zeroscore = prefill(q, k, torch.zeros_like(v))
    assert zero.count_nonzero() == 0 and zeroscore.count_nonzero() == 0
    plain, none = prefill(q, k, v, score=False)
    assert none is None
    assert torch.equal(plain, out)


# tests/test_prefill.py:87-102
@pytest.mark.parametrize("n", [8192, 32768, 131072])
def test_long_uniform_analytic(n):
    print(f"test_long_uniform_analytic n={n}", flush=True)
    q = torch.zeros(1, 2, n, 16, device="cuda", dtype=torch.bfloat16)
    k = torch.zeros(1, 1, n, 16, device="cuda", dtype=q.dtype)
    v = seeded_randn((1, 1, n, 16), torch.bfloat16, 5)
    out, scores = prefill(q, k, v)
    vc = v.cpu()
    expected_out = analytic.zero_qk_output(vc).expand(1, 2, n, 16)
    expected_scores = (vc.double().abs().sum(-1) * analytic.zero_qk_mass(n, 2)).float()
    torch.testing.assert_close(out.float().cpu(), expected_out.float(), atol=.008, rtol=.008)
    torch.testing.assert_close(scores.cpu(), expected_scores, atol=.002, rtol=.0003)


# tests/test_prefill.py:105-131
@pytest.mark.parametrize("n,decay,window", [
    (512, .01, 0), (1024, .1, 0), (4096, 1., 0), (4096, .1, 0),
    (137, 0., 32), (1024, 0., 64), (4096, 0., 128),
    (137, .1, 65), (65, 1., 128), (1, .1, 32),
])
@pytest.mark.parametrize("value_weighted", [True, False])
def test_query_weighted_exact(n, decay, window, value_weighted):
    print(f"test_query_weighted_exact n={n} decay={decay} window={window} vw={value_weighted}", flush=True)
    q, k, v = transposed_qkv(1, n, 4, 2, 64, torch.bfloat16, seed=97 + n)
    kwargs = dict(recency_decay=decay, observation_window=window, value_weighted=value_weighted)
    out, scores = prefill(q, k, v, **kwargs)
    expected, ref = _oracle(q, k, v, **kwargs)
    torch.testing.assert_close(out.float().cpu(), expected, atol=.012, rtol=.006)
    torch.testing.assert_close(scores.cpu(), ref, atol=3e-5, rtol=4e-4)
    plain, _ = prefill(q, k, v, score=False)
    assert torch.equal(out, plain)
    if not value_weighted:
        pos = torch.arange(n)
        weight = (decay * (pos.float() - (n - 1))).exp()
        if window:
            weight *= pos >= n - window
        torch.testing.assert_close(scores.sum(-1).cpu(), weight.sum().expand(1, 2) * 2, rtol=1e-5, atol=1e-4)
    budget = min(n, 128)
    recent = min(64, budget)
    _, keep = select_tokens(scores, budget, reserved_recent=recent)
    _, reference_keep = select_tokens(ref, budget, reserved_recent=recent)
    assert_same_selection(keep, reference_keep, ref, budget, recent, atol=3e-5, rtol=4e-4)
    assert keep.sum(-1).eq(budget).all() and keep[..., -recent:].all()


# tests/test_prefill.py:134-146
@pytest.mark.parametrize("decay,window", [(.01, 0), (0., 128), (.1, 65)])
def test_long_weighted_analytic(decay, window):
    print(f"test_long_weighted_analytic decay={decay} window={window}", flush=True)
    n = 131072
    q = torch.zeros(1, 2, n, 16, device="cuda", dtype=torch.bfloat16)
    k = torch.zeros(1, 1, n, 16, device="cuda", dtype=q.dtype)
    v = torch.ones_like(k)
    _, scores = prefill(q, k, v, recency_decay=decay, observation_window=window)
    expected = analytic.zero_qk_mass(n, 2, decay, window) * 16
    torch.testing.assert_close(scores[0, 0].cpu(), expected.float(), atol=1e-7, rtol=5e-4)
