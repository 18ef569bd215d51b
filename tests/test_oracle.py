"""Pins the CPU oracle (oracle/) against things other than itself.

Each check is chosen so that a plausible mistake in the oracle -- a dropped term, a wrong
sign or index, GQA mean instead of sum, natural vs base-2 exponent -- fails at least one
of them; the `test_planted_*` tests plant such mistakes in a copy of the oracle's output
and confirm the checks catch them.
"""
import json
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import analytic, brute
from oracle import select as osel
from oracle.attention import chunked, materialized

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def known():
    with open(os.path.join(GOLDEN, "known_answers.json")) as f:
        return json.load(f)


def logits_as_qk(logits):
    """q = I and k = logits^T reproduce `logits` as q k^T (scale 1)."""
    lg = torch.tensor(logits, dtype=torch.float32)
    n = lg.shape[0]
    q = torch.eye(n)[None, None]
    k = lg.t().contiguous()[None, None]
    return q, k


# ---- known answers of the reference (tests/test_prefill.py:62-74, RESEARCH_NOTES.md:47-52)

def test_known_normalization_counterexample():
    ka = known()["normalization_counterexample"]
    q, k = logits_as_qk(ka["logits"])
    v = torch.ones_like(k)
    _, mass = materialized(q, k, v, causal=False, value_weighted=False, scale=1.0)
    torch.testing.assert_close(mass[0, 0], torch.tensor(ka["softmax_column_sums"]), rtol=1e-6, atol=1e-6)


def test_known_causal_counterexample():
    ka = known()["causal_counterexample"]
    w = torch.tensor(ka["weights"])
    logits = torch.where(w > 0, w.clamp_min(1e-30).log(), torch.zeros_like(w))
    q, k = logits_as_qk(logits.tolist())
    v = torch.ones_like(k) / 2          # ||v||_1 = 1 with D = 2
    _, mass = materialized(q, k, v, causal=True, scale=1.0)
    torch.testing.assert_close(mass[0, 0], torch.tensor(ka["importance"]), rtol=1e-6, atol=1e-6)
    assert int(mass[0, 0].argmax()) == ka["kept_top1"]
    assert int(w.sum(0).argmax()) == ka["unnormalized_top1"]


# ---- brute-force loops (float64) on tiny inputs

BRUTE_CASES = [
    dict(b=1, hq=2, hk=1, n=7, d=4, causal=True, vw=True, decay=0.0, win=0),
    dict(b=2, hq=4, hk=2, n=9, d=3, causal=False, vw=True, decay=0.3, win=0),
    dict(b=1, hq=3, hk=3, n=8, d=5, causal=True, vw=False, decay=0.1, win=3),
    dict(b=1, hq=6, hk=2, n=6, d=2, causal=True, vw=True, decay=1.0, win=4),
    dict(b=1, hq=2, hk=1, n=1, d=3, causal=True, vw=True, decay=0.5, win=1),
]


@pytest.mark.parametrize("c", BRUTE_CASES)
def test_materialized_matches_brute_force(c):
    g = torch.Generator().manual_seed(c["n"] * 31 + c["hq"])
    q = torch.randn(c["b"], c["hq"], c["n"], c["d"], generator=g)
    k = torch.randn(c["b"], c["hk"], c["n"], c["d"], generator=g)
    v = torch.randn(c["b"], c["hk"], c["n"], c["d"], generator=g)
    kw = dict(causal=c["causal"], value_weighted=c["vw"], recency_decay=c["decay"], observation_window=c["win"])
    out, mass = materialized(q, k, v, **kw)
    bout, bmass = brute.attention(q.tolist(), k.tolist(), v.tolist(), **kw)
    torch.testing.assert_close(out.double(), torch.tensor(bout, dtype=torch.float64), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(mass.double(), torch.tensor(bmass, dtype=torch.float64), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("c", BRUTE_CASES)
def test_chunked_float64_matches_brute_force(c):
    """chunked(dtype=float64) against the float64 loops, to float64 accuracy: the same
    formulas, only the precision differs."""
    g = torch.Generator().manual_seed(c["n"] * 37 + c["hq"])
    q = torch.randn(c["b"], c["hq"], c["n"], c["d"], generator=g, dtype=torch.float64)
    k = torch.randn(c["b"], c["hk"], c["n"], c["d"], generator=g, dtype=torch.float64)
    v = torch.randn(c["b"], c["hk"], c["n"], c["d"], generator=g, dtype=torch.float64)
    kw = dict(causal=c["causal"], value_weighted=c["vw"], recency_decay=c["decay"], observation_window=c["win"])
    out, mass = chunked(q, k, v, block=4, dtype=torch.float64, **kw)
    bout, bmass = brute.attention(q.tolist(), k.tolist(), v.tolist(), **kw)
    torch.testing.assert_close(out, torch.tensor(bout, dtype=torch.float64), rtol=1e-6, atol=1e-9)
    # the recency weights are the FP32 values of the reference (a relative 1e-7 apart from
    # the float64 loops' weights)
    torch.testing.assert_close(mass, torch.tensor(bmass, dtype=torch.float64), rtol=1e-6, atol=1e-9)


def test_chunked_float64_resolves_extreme_logits():
    """With x30 inputs the logits are ~1e3 and FP32 evaluation is off by up to ~1e-3
    relative in the probabilities; float64 agrees with the float64 loops to 1e-9."""
    g = torch.Generator().manual_seed(4)
    q = (torch.randn(1, 2, 12, 16, generator=g) * 30).to(torch.float16)
    k = (torch.randn(1, 1, 12, 16, generator=g) * 30).to(torch.float16)
    v = torch.randn(1, 1, 12, 16, generator=g).to(torch.float16)
    kw = dict(causal=False, value_weighted=False)
    _, mass64 = chunked(q, k, v, block=5, dtype=torch.float64, **kw)
    _, bmass = brute.attention(q.double().tolist(), k.double().tolist(), v.double().tolist(), **kw)
    torch.testing.assert_close(mass64, torch.tensor(bmass, dtype=torch.float64), rtol=1e-9, atol=1e-12)
    _, mass32 = chunked(q, k, v, block=5, **kw)
    torch.testing.assert_close(mass32.double(), mass64, rtol=5e-3, atol=1e-6)


# ---- textbook attention from the library (output only)

@pytest.mark.parametrize("causal", [True, False])
def test_materialized_output_matches_sdpa(causal):
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, 8, 70, 32, generator=g)
    k = torch.randn(1, 2, 70, 32, generator=g)
    v = torch.randn(1, 2, 70, 32, generator=g)
    out, _ = materialized(q, k, v, causal=causal)
    ref = F.scaled_dot_product_attention(q, k.repeat_interleave(4, 1), v.repeat_interleave(4, 1), is_causal=causal)
    torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-5)


# ---- chunked == materialized wherever the dense form fits

@pytest.mark.parametrize("kw", [
    dict(causal=True), dict(causal=False), dict(causal=True, recency_decay=0.1),
    dict(causal=True, observation_window=70, value_weighted=False),
    dict(causal=False, recency_decay=0.02, observation_window=33),
])
def test_chunked_matches_materialized(kw):
    g = torch.Generator().manual_seed(9)
    q = torch.randn(2, 6, 300, 48, generator=g).to(torch.bfloat16)
    k = torch.randn(2, 3, 300, 48, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 3, 300, 48, generator=g).to(torch.bfloat16)
    out, mass = materialized(q, k, v, **kw)
    cout, cmass = chunked(q, k, v, block=64, **kw)
    torch.testing.assert_close(cout, out, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(cmass, mass, rtol=1e-5, atol=1e-5)
    # restricting to one head keeps exactly that head's contribution
    _, hmass = chunked(q, k, v, block=64, heads=[(1, 4)], want_out=False, **kw)
    _, dense_h = materialized(q[1:2, 4:5], k[1:2, 2:3], v[1:2, 2:3], **kw)
    torch.testing.assert_close(hmass[1, 2], dense_h[0, 0], rtol=1e-5, atol=1e-6)


# ---- closed forms (tests/test_prefill.py:87-102,134-146)

@pytest.mark.parametrize("decay,window", [(0.0, 0), (0.01, 0), (0.0, 100), (0.1, 65)])
def test_closed_forms(decay, window):
    n, groups = 512, 2
    q = torch.zeros(1, groups, n, 16)
    k = torch.zeros(1, 1, n, 16)
    v = torch.randn(1, 1, n, 16, generator=torch.Generator().manual_seed(3))
    out, mass = materialized(q, k, v, recency_decay=decay, observation_window=window)
    torch.testing.assert_close(out.double(), analytic.zero_qk_output(v).expand(1, groups, n, 16), rtol=1e-5, atol=1e-6)
    expected = v.double().abs().sum(-1) * analytic.zero_qk_mass(n, groups, decay, window)
    torch.testing.assert_close(mass.double(), expected, rtol=1e-5, atol=1e-7)
    _, cmass = chunked(q, k, v, recency_decay=decay, observation_window=window, block=100)
    torch.testing.assert_close(cmass.double(), expected, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("decay,window", [(0.0, 0), (0.1, 0), (0.0, 64)])
def test_mass_conservation(decay, window):
    g = torch.Generator().manual_seed(11)
    n = 200
    q = torch.randn(1, 4, n, 16, generator=g)
    k = torch.randn(1, 2, n, 16, generator=g)
    v = torch.randn(1, 2, n, 16, generator=g)
    _, mass = materialized(q, k, v, value_weighted=False, recency_decay=decay, observation_window=window)
    pos = torch.arange(n, dtype=torch.float64)
    w = (decay * (pos - (n - 1))).exp()
    if window:
        w = w * (pos >= n - window)
    torch.testing.assert_close(mass.sum(-1).double(), (2 * w.sum()).expand(1, 2), rtol=1e-5, atol=1e-5)


# ---- planted mistakes: each must be caught by one of the checks above

def _small():
    g = torch.Generator().manual_seed(21)
    q = torch.randn(1, 4, 12, 8, generator=g)
    k = torch.randn(1, 2, 12, 8, generator=g)
    v = torch.randn(1, 2, 12, 8, generator=g)
    return q, k, v


def test_planted_gqa_mean_is_caught():
    q, k, v = _small()
    _, mass = materialized(q, k, v, value_weighted=False)
    wrong = mass / 2                      # averaging grouped heads instead of summing
    assert not torch.allclose(wrong.sum(-1), torch.full((1, 2), 2 * 12.0), rtol=1e-3)


def test_planted_exp2_weights_are_caught():
    q, k, v = _small()
    kw = dict(recency_decay=0.3, value_weighted=False)
    _, bmass = brute.attention(q.tolist(), k.tolist(), v.tolist(), **kw)
    # base-2 recency weights instead of natural exp
    _, m2 = materialized(q, k, v, recency_decay=0.3 / math.log(2), value_weighted=False)
    assert not torch.allclose(m2.double(), torch.tensor(bmass, dtype=torch.float64), rtol=1e-3)


def test_planted_mask_transpose_is_caught():
    q, k, v = _small()
    out, _ = materialized(q, k, v)
    # an anti-causal (transposed) mask attends to the future instead of the past
    lg = (q @ k.repeat_interleave(2, 1).transpose(-1, -2)) * 8 ** -0.5
    pos = torch.arange(12)
    p = lg.masked_fill(pos[None, :] < pos[:, None], float("-inf")).softmax(-1)
    wrong = p @ v.repeat_interleave(2, 1)
    bout, _ = brute.attention(q.tolist(), k.tolist(), v.tolist())
    assert torch.allclose(out.double(), torch.tensor(bout, dtype=torch.float64), rtol=1e-5, atol=1e-6)
    assert not torch.allclose(wrong.double(), torch.tensor(bout, dtype=torch.float64), rtol=1e-3)


# ---- selection oracle

def test_select_known_answers():
    ka = known()
    sc = ka["selection_contract"]
    idx, keep = osel.select_tokens(np.array(sc["scores"], dtype=np.float32).reshape(1, 1, -1), sc["budget"],
                                   recent=sc["recent"])
    assert idx.tolist() == [[sc["indices"]]]
    assert keep.sum() == sc["budget"]
    for bad in sc["invalid_budgets"]:
        with pytest.raises(ValueError):
            osel.select_tokens(np.zeros((1, 20), np.float32), bad)
    with pytest.raises(ValueError):
        osel.select_tokens(np.zeros((1, 20), np.float32), 2, recent=sc["invalid_recent_for_budget_2"])
    vn = ka["value_norm_selection"]
    norms = np.abs(np.array(vn["values"], np.float32))[None, :].repeat(vn["channels"], 0).sum(0)
    idx, _ = osel.select_tokens(norms, vn["budget"])
    assert idx.tolist() == vn["indices"]
    idx, _ = osel.select_tokens(norms, vn["budget"], recent=vn["budget"])
    assert idx.tolist() == vn["suffix_indices"]


def test_avg_pool_matches_torch_bitwise():
    for seed, m, k in [(0, 137, 5), (1, 1000, 3), (2, 9, 7), (3, 4, 9)]:
        x = torch.randn(3, m, generator=torch.Generator().manual_seed(seed))
        ref = F.avg_pool1d(x[:, None], k, stride=1, padding=k // 2).squeeze(1)
        got = osel.avg_pool(x.numpy(), k)
        assert np.array_equal(got, ref.numpy()), (seed, m, k)


@pytest.mark.parametrize("seed", range(6))
def test_select_matches_torch_topk_without_ties(seed):
    g = torch.Generator().manual_seed(seed)
    n = int(torch.randint(10, 400, (1,), generator=g))
    x = torch.randn(2, 3, n, generator=g)
    budget = int(torch.randint(1, n + 1, (1,), generator=g))
    recent = int(torch.randint(0, budget + 1, (1,), generator=g))
    pk = [1, 3, 5][seed % 3]
    idx, keep = osel.select_tokens(x.numpy(), budget, recent=recent, pool_kernel=pk)
    past = x[..., :n - recent]
    if pk > 1 and budget > recent:
        past = F.avg_pool1d(past.reshape(-1, 1, past.shape[-1]), pk, stride=1, padding=pk // 2).reshape_as(past)
    top = past.topk(budget - recent, dim=-1).indices
    tail = torch.arange(n - recent, n).expand(2, 3, recent)
    ref = torch.cat((top, tail), -1).sort(-1).values
    assert np.array_equal(idx, ref.numpy())
    refkeep = torch.zeros_like(x, dtype=torch.bool).scatter_(-1, ref, True)
    assert np.array_equal(keep, refkeep.numpy())


@pytest.mark.parametrize("seed", range(8))
def test_select_matches_brute_with_ties(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(5, 40))
    x = rng.integers(0, 4, size=n).astype(np.float32)     # many exact ties
    budget = int(rng.integers(1, n + 1))
    recent = int(rng.integers(0, budget + 1))
    idx, keep = osel.select_tokens(x, budget, recent=recent)
    bidx, bkeep = brute.select_row(x.tolist(), budget, recent)
    assert idx.tolist() == bidx and keep.tolist() == bkeep


def test_snap_select_equivalence():
    # tests/test_prefill.py:149-155: pooled top-k with reserved suffix == SnapKV selection
    case = known()["pool_pin_case"]
    torch.manual_seed(case["seed"])
    scores = torch.randn(*case["shape"]).numpy()
    idx, keep = osel.select_tokens(scores, case["budget"], reserved_recent=case["reserved_recent"],
                                   pool_kernel=case["pool_kernel"])
    eidx, ekeep = osel.snap_select(scores, case["budget"], case["reserved_recent"], case["pool_kernel"])
    assert np.array_equal(idx, eidx) and np.array_equal(keep, ekeep)
    _, tail = osel.select_tokens(scores, case["suffix_only_budget"], reserved_recent=case["suffix_only_budget"],
                                 pool_kernel=case["pool_kernel"])
    assert tail.sum() == 3 * case["suffix_only_budget"] and tail[..., -case["suffix_only_budget"]:].all()


def test_select_special_values():
    x = np.array([0.0, -0.0, np.nan, -np.inf, np.inf, 1.0, -0.0, 0.0], dtype=np.float32)
    idx, _ = osel.select_tokens(x, 3)
    assert idx.tolist() == [2, 4, 5]          # NaN ranks first, then +inf, then 1
    idx, _ = osel.select_tokens(x, 5)
    assert idx.tolist() == [0, 1, 2, 4, 5]    # -0.0 ties with +0.0: lower index first


def test_golden_fixture_reproduces():
    data = np.load(os.path.join(GOLDEN, "prefill_small.npz"), allow_pickle=False)
    names = sorted({k.split(".")[0] for k in data.files})
    assert len(names) == 3
    for name in names:
        meta = json.loads(str(data[f"{name}.meta"]))
        dt = getattr(torch, meta["dtype"])
        q, k, v = (torch.from_numpy(data[f"{name}.{t}"]).view(dt) for t in "qkv")
        out, imp = materialized(q, k, v, **meta["kwargs"])
        # CPU matmul kernels may differ by host; the fixture must agree to float32 rounding
        np.testing.assert_allclose(out.numpy(), data[f"{name}.out"], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(imp.numpy(), data[f"{name}.importance"], rtol=1e-5, atol=1e-6)
