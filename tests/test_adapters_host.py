"""CPU checks of the model adapters' host logic: the evaluation policies' index choice
(reference tests/test_quality_adapter.py:17-24, known answers), the budget parsing of
compress (kv_distill_adapter.py:31-33), the streaming controller's argument checks and
chunk_mlp (reference tests/test_streaming_adapter.py:62-76, here on the CPU in float32)."""
import pytest
import torch

from flash_evict.controller import parse_budget
from flash_evict.quality_adapter import PairedController, choose_indices, default_methods, group_key
from flash_evict.streaming_adapter import StreamingController, chunk_mlp


def test_ablation_selection_is_exact():
    k = torch.zeros(1, 2, 5, 2)
    v = torch.tensor([1., -9., 3., -7., 2.]).view(1, 1, 5, 1).expand(1, 2, 5, 2)
    norms = choose_indices(dict(backend="value_norm_only", budget=2), k, v)
    recent = choose_indices(dict(backend="uniform_recent", budget=2), k, v)
    assert norms.tolist() == [[[1, 3], [1, 3]]]
    assert recent.tolist() == [[[3, 4], [3, 4]]]
    assert choose_indices(dict(backend="full", budget=None), k, v) is None
    assert choose_indices(dict(backend="fused", budget=5), k, v) is None      # budget covers the prompt
    with pytest.raises(ValueError, match="Unknown policy backend"):
        choose_indices(dict(backend="h2o", budget=2), k, v)


def test_budget_parsing():
    assert parse_budget("0.1", 137) == 14
    assert parse_budget("48", 137) == 48
    assert parse_budget("full", 137) == 137
    assert parse_budget("500", 137) == 137
    assert parse_budget("0.001", 137) == 1


def _tiny_cpu_model(layers=2):
    import transformers
    cfg = transformers.Qwen2Config(vocab_size=257, hidden_size=128, intermediate_size=256, num_hidden_layers=layers,
                                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(3)
    return transformers.Qwen2ForCausalLM(cfg).eval()


def test_streaming_controller_rejects_bad_arguments():
    # streaming_adapter.py:19-20 (checked before the model is touched)
    for kwargs, msg in [(dict(backend="h2o"), "Unsupported backend"), (dict(budget=0), "Positive integer budget"),
                        (dict(budget=True), "Positive integer budget"), (dict(budget=2.0), "Positive integer budget")]:
        with pytest.raises(ValueError, match=msg):
            StreamingController(None, **kwargs)


def test_chunk_mlp_matches_and_restores():
    model = _tiny_cpu_model()
    ids = torch.randint(0, 257, (1, 75), generator=torch.Generator().manual_seed(1))
    with torch.inference_mode():
        expected = model.model(ids, use_cache=False).last_hidden_state
        restore = chunk_mlp(model, 31)
        actual = model.model(ids, use_cache=False).last_hidden_state
        torch.testing.assert_close(actual, expected, atol=1e-5, rtol=1e-5)
        restore()
        assert torch.equal(model.model(ids, use_cache=False).last_hidden_state, expected)
    restore = chunk_mlp(model, 8)
    with pytest.raises(RuntimeError, match="inference-only"):
        with torch.enable_grad():
            model.model(ids, use_cache=False)
    restore()
    for bad in (0, -3, True, 2.5):
        with pytest.raises(ValueError, match="positive integer"):
            chunk_mlp(model, bad)


def test_policy_groups_and_default_methods():
    # quality_adapter.py:19-37
    methods = default_methods()
    assert [m["name"] for m in methods][:3] == ["full", "snap_256", "d01_r0_256"]
    assert len(methods) == 1 + 2 * 4 + 2
    fused = [m for m in methods if m["backend"] == "fused"]
    assert {group_key(m) for m in fused} == {("fused", .1, 0, True), ("fused", .1, 128, True)}
    assert {group_key(m) for m in methods if m["backend"] != "fused"} == {("baseline",)}
    ctl = PairedController.__new__(PairedController)   # argument checks only; no model needed
    with pytest.raises(ValueError, match="shared prefill"):
        ctl.prepare([methods[0], fused[0]])


def test_activate_rejects_unequal_retained_lengths():
    ctl = PairedController.__new__(PairedController)
    ctl.bank = {"a": {0: {"k": torch.zeros(1, 2, 5, 4), "v": torch.zeros(1, 2, 5, 4)}},
                "b": {0: {"k": torch.zeros(1, 2, 6, 4), "v": torch.zeros(1, 2, 6, 4)}}}
    with pytest.raises(ValueError, match="same number of tokens"):
        ctl.activate(["a", "b"])
    ctl.activate(["a"], consume=False)
    assert ctl.mode == "decode" and ctl.states[0]["k"].shape == (1, 2, 5, 4) and "a" in ctl.bank
