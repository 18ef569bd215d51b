"""CPU checks of the transformers integration's host logic: the evaluation policies'
index choice (reference tests/test_quality_adapter.py:17-24, known answers) and the budget
parsing of compress (kv_distill_adapter.py:31-33)."""
import torch

from flash_evict.hf import _budget, choose_indices


def test_ablation_selection_is_exact():
    k = torch.zeros(1, 2, 5, 2)
    v = torch.tensor([1., -9., 3., -7., 2.]).view(1, 1, 5, 1).expand(1, 2, 5, 2)
    norms = choose_indices(dict(backend="value_norm_only", budget=2), k, v)
    recent = choose_indices(dict(backend="uniform_recent", budget=2), k, v)
    assert norms.tolist() == [[[1, 3], [1, 3]]]
    assert recent.tolist() == [[[3, 4], [3, 4]]]
    assert choose_indices(dict(backend="full", budget=None), k, v) is None
    assert choose_indices(dict(backend="fused", budget=5), k, v) is None


def test_budget_parsing():
    assert _budget("0.1", 137) == 14
    assert _budget("48", 137) == 48
    assert _budget("full", 137) == 137
    assert _budget("500", 137) == 137
    assert _budget("0.001", 137) == 1
