"""Seeded randomized parity sweep of the workspace-free entry point fe_prefill (the single
fused attention + replay kernel: 12 waves on tile dims 96 and 128, 8 on 32 and 64; head dims
below their tile dim on the partial instantiations) against the dense FP32 oracle (oracle/attention.materialized, restating
reference.py:5-25), at the reference's tolerances (tests/test_prefill.py: bf16 .012/.006,
fp16 .002/.006). Shapes, GQA groups, ragged N, dtypes, masks, windows, decays, scales and
layouts are drawn from a seeded generator."""
import random

import pytest
import torch

from oracle.attention import materialized

from _helpers import seeded_randn, transposed_qkv
from test_schedules_gpu import _run

pytestmark = pytest.mark.gpu


def draw(seed):
    r = random.Random(5000 + seed)
    n = r.choice([1, 31, 64, 65, 127, 129, 300, 511, 700, 1025])
    return dict(b=r.choice([1, 1, 2]), hk=r.choice([1, 2, 4]), g=r.choice([1, 2, 4, 7]), n=n,
                d=r.choice([40, 64, 80, 96, 120, 128, 128]), dtype=r.choice([torch.float16, torch.bfloat16]),
                causal=r.random() < 0.8, decay=r.choice([0.0, 0.0, 0.05, 0.5, 50.0]),
                window=r.choice([0, 0, 1, 17, 64, n + 5]), weighted=r.random() < 0.7,
                transposed=r.random() < 0.5)


@pytest.mark.parametrize("seed", range(24))
def test_fused_entry_point_matches_oracle(seed):
    c = draw(seed)
    print("fused fuzz seed=%d %s" % (seed, c), flush=True)
    b, hq, hk, n, d = c["b"], c["g"] * c["hk"], c["hk"], c["n"], c["d"]
    if c["transposed"]:
        q, k, v = transposed_qkv(b, n, hq, hk, d, c["dtype"], 900 + seed)
    else:
        q = seeded_randn((b, hq, n, d), c["dtype"], 900 + seed)
        k = seeded_randn((b, hk, n, d), c["dtype"], 901 + seed)
        v = seeded_randn((b, hk, n, d), c["dtype"], 902 + seed)
    out, imp = _run(q, k, v, c["causal"], c["weighted"], c["decay"], c["window"], use_ws=False)
    ref_out, ref_imp = materialized(q.cpu(), k.cpu(), v.cpu(), causal=c["causal"], value_weighted=c["weighted"],
                                    recency_decay=c["decay"], observation_window=c["window"])
    atol = .012 if c["dtype"] == torch.bfloat16 else .002
    torch.testing.assert_close(out.float().cpu(), ref_out, atol=atol, rtol=.006)
    big = float(ref_imp.abs().max())
    torch.testing.assert_close(imp.cpu(), ref_imp, atol=3e-5 + 1e-6 * big, rtol=4e-4)
