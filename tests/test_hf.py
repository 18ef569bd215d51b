"""CPU checks of the transformers integration's host logic: the evaluation policies'
index choice (reference tests/test_quality_adapter.py:17-24, known answers), the budget
parsing of compress (kv_distill_adapter.py:31-33), the streaming controller's argument checks
and chunk_mlp (reference tests/test_streaming_adapter.py:62-76, here on the CPU)."""
import torch

from flash_evict.hf import PairedController, StreamingController, _budget, choose_indices, chunk_mlp, default_methods, group_key


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
        try:
            StreamingController(None, **kwargs)
        except ValueError as e:
            assert msg in str(e)
        else:
            raise AssertionError(kwargs)


def test_chunk_mlp_matches_and_restores():
    # streaming_adapter.py:30-51, on the CPU in float32
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
    try:
        with torch.enable_grad():
            model.model(ids, use_cache=False)
    except RuntimeError as e:
        assert "inference-only" in str(e)
    else:
        raise AssertionError("grad-enabled chunked MLP must raise")
    restore()
    for bad in (0, -3, True, 2.5):
        try:
            chunk_mlp(model, bad)
        except ValueError as e:
            assert "positive integer" in str(e)
        else:
            raise AssertionError(bad)


def test_policy_groups_and_default_methods():
    # quality_adapter.py:19-37
    methods = default_methods()
    assert [m["name"] for m in methods][:3] == ["full", "snap_256", "d01_r0_256"]
    assert len(methods) == 1 + 2 * 4 + 2
    fused = [m for m in methods if m["backend"] == "fused"]
    assert {group_key(m) for m in fused} == {("fused", .1, 0, True), ("fused", .1, 128, True)}
    assert {group_key(m) for m in methods if m["backend"] != "fused"} == {("baseline",)}
    ctl = PairedController.__new__(PairedController)   # argument checks only; no model needed
    try:
        ctl.prepare([methods[0], fused[0]])
    except ValueError as e:
        assert "shared prefill" in str(e)
    else:
        raise AssertionError("mixed groups must be rejected")
