"""Write the golden fixtures under tests/golden/.

known_answers.json: known-answer vectors held by the reference repository
(anishesg/flash-evict-prefill), transcribed here as data with their source lines:
  * normalisation counterexample, tests/test_prefill.py:62-74
  * two-query causal counterexample, RESEARCH_NOTES.md:47-52
  * selection contract, tests/test_prefill.py:77-84
  * value-norm and suffix ablation selections, tests/test_quality_adapter.py:18-24
  * pooling + pinning equivalence case, tests/test_prefill.py:149-155 (inputs are
    regenerated from the seed recorded there)

prefill_small.npz: seeded small prefill cases (inputs and the FP32 oracle's outputs,
oracle/attention.materialized), so GPU parity can be checked against fixed numbers.

Run from the repository root:  python tests/golden/make_golden.py
"""
import json
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle.attention import materialized  # noqa: E402

KNOWN = {
    "normalization_counterexample": {
        "source": "tests/test_prefill.py:62-74",
        "logits": [[0.0, 0.0], [0.0, math.log(9.0)]],
        "softmax_column_sums": [0.6, 1.4],
    },
    "causal_counterexample": {
        "source": "tests/test_prefill.py:70-74; RESEARCH_NOTES.md:47-52",
        "weights": [[9.0, 0.0], [100.0, 200.0]],
        "importance": [4.0 / 3.0, 2.0 / 3.0],
        "kept_top1": 0,
        "unnormalized_top1": 1,
    },
    "selection_contract": {
        "source": "tests/test_prefill.py:77-84",
        "scores": list(range(20)),
        "budget": 4,
        "recent": 2,
        "indices": [16, 17, 18, 19],
        "invalid_budgets": [0, 21, True, 2.5],
        "invalid_recent_for_budget_2": 3,
    },
    "value_norm_selection": {
        "source": "tests/test_quality_adapter.py:18-24",
        "values": [1.0, -9.0, 3.0, -7.0, 2.0],
        "channels": 2,
        "budget": 2,
        "indices": [1, 3],
        "suffix_indices": [3, 4],
    },
    "pool_pin_case": {
        "source": "tests/test_prefill.py:149-159",
        "seed": 1,
        "shape": [1, 3, 137],
        "budget": 48,
        "reserved_recent": 32,
        "pool_kernel": 5,
        "suffix_only_budget": 64,
    },
}

CASES = [
    # name, B, Hq, Hkv, N, D, dtype, kwargs
    ("fp16_causal_gqa2", 1, 4, 2, 64, 64, torch.float16, dict(causal=True)),
    ("bf16_noncausal_window", 1, 6, 2, 50, 32, torch.bfloat16,
     dict(causal=False, recency_decay=0.2, observation_window=17)),
    ("bf16_causal_h2o_decay", 2, 2, 1, 40, 128, torch.bfloat16,
     dict(causal=True, value_weighted=False, recency_decay=0.05)),
]


def main():
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(KNOWN, f, indent=1)
    arrays = {}
    for i, (name, b, hq, hk, n, d, dtype, kw) in enumerate(CASES):
        g = torch.Generator().manual_seed(4242 + i)
        q = torch.randn((b, hq, n, d), generator=g).to(dtype)
        k = torch.randn((b, hk, n, d), generator=g).to(dtype)
        v = torch.randn((b, hk, n, d), generator=g).to(dtype)
        out, imp = materialized(q, k, v, **kw)
        for tag, t in (("q", q), ("k", k), ("v", v)):
            arrays[f"{name}.{tag}"] = t.view(torch.int16).numpy()
        arrays[f"{name}.out"] = out.numpy()
        arrays[f"{name}.importance"] = imp.numpy()
        arrays[f"{name}.meta"] = np.array(json.dumps(
            {"dtype": str(dtype).replace("torch.", ""), "kwargs": kw}))
    np.savez_compressed(os.path.join(HERE, "prefill_small.npz"), **arrays)
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
