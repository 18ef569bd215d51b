"""The replay skips query rows whose recency weight is exactly zero in FP32
(fe_replay_rows). CPU-only: fe_replay_rows is host arithmetic, and the checks below pin
the rule against the reference's own weight formula rather than restating it.

Reference: flash_evict/prefill.py:66-67 weights row q by exp(DECAY*(q-(N-1))) in FP32 and
multiplies every probability of the row by it; reference.py:19 does the same in the
materialized path. A row whose weight is exactly 0.0 therefore adds exactly 0.0 to every
column, so leaving it out of the replay cannot change the importance.
"""
import math

import pytest
import torch

from flash_evict import _lib


def rows(n, window, decay):
    return _lib.lib().fe_replay_rows(n, window, float(decay))


@pytest.mark.parametrize("decay", [1e-3, 0.01, 0.1, 0.25, 1.0, 3.7, 105.0, 1e6])
def test_skipped_rows_have_zero_reference_weight(decay):
    r = rows(1 << 40, 1 << 40, decay)
    decay32 = float(torch.tensor(decay, dtype=torch.float32))   # the C ABI takes a float
    assert r == math.ceil(105.0 / decay32)
    # the reference's FP32 weight of the newest skipped row and a run of older ones
    n = r + 4096
    pos = torch.arange(n)
    weight = (torch.tensor(decay, dtype=torch.float32) * (pos.float() - (n - 1))).exp()
    skipped = weight[: n - r]
    assert torch.count_nonzero(skipped) == 0
    # the kernels' replay term is bounded by 2^(-decay*log2(e)*t) for t = N-1-q: zero too
    t = torch.arange(r, r + 4096, dtype=torch.float64)
    bound = torch.exp2((-(decay * math.log2(math.e)) * t).float())
    assert torch.count_nonzero(bound) == 0
    # every kept row but possibly the oldest few has a nonzero weight: the rule is tight
    kept = weight[n - r:]
    assert kept[-1] == 1.0
    assert torch.count_nonzero(kept) >= min(r, 10)


def test_rows_follow_window_and_no_decay():
    assert rows(32768, 32768, 0.0) == 32768
    assert rows(32768, 128, 0.0) == 128
    assert rows(32768, 32768, 0.1) == 1050          # the headline: 3.2% of the rows
    assert rows(32768, 128, 0.1) == 128             # a smaller window wins
    assert rows(1, 1, 0.1) == 1
    assert rows(4096, 4096, 1.0) == 105
    assert rows(10, 10, 1e9) == 1                   # the last row always has weight 1


def test_rows_reject_invalid_arguments():
    for args in [(0, 1, 0.0), (4, 0, 0.0), (4, 5, 0.0), (4, 4, -1.0), (4, 4, float("nan")),
                 (4, 4, float("inf"))]:
        assert rows(*args) == -1, args
