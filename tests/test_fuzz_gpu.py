"""Seeded randomized parity sweep of prefill/evict against the oracle.

Each case draws its shape and options from a seeded generator: batch, KV heads and GQA group
(1, 2, 4 or 7), N from 1 to 700 (tile edges included), head dims 16..256 (the fast kernels for
multiples of 8 up to 256, on full and partial tiles; at these sizes every launch is below one
round of the two-row-tile kernel's work items, so 72..128 run the small-grid kernel; the generic
kernel for 100), fp16/bf16, causal or not, softmax scale (default, small,
negative), recency decay
(including decays large enough that the replay keeps only a few rows), observation window,
value weighting, contiguous or transposed layouts, and a selection budget, reserved suffix and
pool kernel. The attention output and importance are compared with the dense FP32 oracle
(oracle/attention.materialized, restating reference.py:5-25) at the reference's tolerances;
evict's selection with the oracle's selection (oracle/select, restating prefill.py:140-170)
on the same importance."""
import random

import pytest
import torch

from flash_evict import evict, prefill, select_tokens
from oracle import select as oselect
from oracle.attention import materialized

from _helpers import assert_same_selection, seeded_randn

pytestmark = pytest.mark.gpu


def draw(seed):
    r = random.Random(seed)
    n = r.choice([1, 2, 31, 63, 64, 65, 127, 200, 333, 512, 700])
    budget = r.randint(1, n)
    return dict(
        b=r.choice([1, 1, 2]), hk=r.choice([1, 2, 4]), g=r.choice([1, 2, 4, 7]), n=n,
        d=r.choice([16, 32, 48, 64, 64, 80, 96, 100, 120, 128, 128, 160, 256]), dtype=r.choice([torch.float16, torch.bfloat16]),
        causal=r.random() < 0.8, scale=r.choice([None, None, 0.05, 0.3, -0.2]),
        decay=r.choice([0.0, 0.0, 0.05, 0.5, 3.0, 50.0]), window=r.choice([0, 0, 1, 17, 64, n + 5]),
        weighted=r.random() < 0.7, transposed=r.random() < 0.5, budget=budget,
        recent=r.randint(0, budget), pool=r.choice([1, 1, 3, 5]))


def inputs(c, seed):
    b, hq, hk, n, d = c["b"], c["g"] * c["hk"], c["hk"], c["n"], c["d"]
    if c["transposed"]:
        q = seeded_randn((b, n, hq, d), c["dtype"], seed).transpose(1, 2)
        k = seeded_randn((b, n, hk, d), c["dtype"], seed + 1).transpose(1, 2)
        v = seeded_randn((b, n, hk, d), c["dtype"], seed + 2).transpose(1, 2)
    else:
        q = seeded_randn((b, hq, n, d), c["dtype"], seed)
        k = seeded_randn((b, hk, n, d), c["dtype"], seed + 1)
        v = seeded_randn((b, hk, n, d), c["dtype"], seed + 2)
    return q, k, v


@pytest.mark.parametrize("seed", range(48))
def test_random_case_matches_oracle(seed):
    c = draw(seed)
    print("fuzz seed=%d %s" % (seed, c), flush=True)
    q, k, v = inputs(c, 1000 + 7 * seed)
    kw = dict(causal=c["causal"], value_weighted=c["weighted"], scale=c["scale"], recency_decay=c["decay"],
              observation_window=c["window"])
    out, imp = prefill(q, k, v, **kw)
    ref_out, ref_imp = materialized(q.cpu(), k.cpu(), v.cpu(), **kw)
    # the reference's tolerances (tests/test_prefill.py: bf16 .012/.006, fp16 .002/.006)
    atol = .012 if c["dtype"] == torch.bfloat16 else .002
    torch.testing.assert_close(out.float().cpu(), ref_out, atol=atol, rtol=.006)
    big = float(ref_imp.abs().max())
    torch.testing.assert_close(imp.cpu(), ref_imp, atol=3e-5 + 1e-6 * big, rtol=4e-4)

    # evict: the same output, and its selection of its own importance
    out2, imp2, idx, evicted = evict(q, k, v, c["budget"], reserved_recent=c["recent"], pool_kernel=c["pool"],
                                     **kw)
    assert torch.equal(out2, out)
    torch.testing.assert_close(imp2, imp, atol=1e-6 * big + 1e-7, rtol=2e-6)   # FP32 atomic order
    keep = ~evicted
    assert idx.shape[-1] == c["budget"] and keep.sum(-1).eq(c["budget"]).all()
    assert keep.gather(-1, idx).all() and (idx[..., 1:] > idx[..., :-1]).all()
    if c["recent"]:
        assert keep[..., -c["recent"]:].all()
    # the selection kernel on the oracle's importance equals the oracle's selection exactly
    ref_idx, ref_keep = oselect.select_tokens(ref_imp.numpy(), c["budget"], reserved_recent=c["recent"],
                                              pool_kernel=c["pool"])
    got_idx, got_keep = select_tokens(ref_imp.cuda(), c["budget"], reserved_recent=c["recent"],
                                      pool_kernel=c["pool"])
    assert torch.equal(got_idx.cpu(), torch.from_numpy(ref_idx))
    assert torch.equal(got_keep.cpu(), torch.from_numpy(ref_keep))
    # ... and on the kernel's own importance it differs only at near-ties (unpooled scores)
    if c["pool"] == 1 or c["budget"] == c["recent"]:
        assert_same_selection(keep, torch.from_numpy(ref_keep), ref_imp, c["budget"], c["recent"],
                              atol=3e-5 + 1e-6 * big, rtol=4e-4)
