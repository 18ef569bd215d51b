"""The model adapters on a tiny random-init Qwen2 (bf16), in the configuration and with the
assertions of the reference's adapter tests (tests/test_adapter.py,
tests/test_streaming_adapter.py and tests/test_quality_adapter.py of
anishesg/flash-evict-prefill), through the same API: FusedController / StreamingController /
PairedController, compress(method, prompt_length), finish_prefill, activate, decode_batch,
with decoding through the controller's growing cache (use_cache=False). The reference runs
these on kv_distill's Controller; here they run on the local stand-in
(flash_evict.controller). Added: H2O mass per layer, the inference transform, and the
DynamicCache hand-off.
"""
import pytest
import torch

from flash_evict.kv_distill_adapter import FusedController
from flash_evict.quality_adapter import PairedController, decode_batch
from flash_evict.streaming_adapter import StreamingController, chunk_mlp

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")


def tiny_model(layers=2):
    config = transformers.Qwen2Config(vocab_size=257, hidden_size=128, intermediate_size=256,
                                      num_hidden_layers=layers, num_attention_heads=4, num_key_value_heads=2,
                                      max_position_embeddings=512)
    config._attn_implementation = "sdpa"
    return transformers.Qwen2ForCausalLM(config).cuda().to(torch.bfloat16).eval()


# reference tests/test_adapter.py
@torch.inference_mode()
@pytest.mark.parametrize("scoring,recent", [({}, 0), ({"recency_decay": .1}, 5), ({"observation_window": 32}, 5)])
def test_qwen_prefill_compress_decode(scoring, recent):
    torch.manual_seed(19)
    model = tiny_model()
    ids = torch.randint(0, 257, (1, 137), device="cuda")
    pos = torch.arange(137, device="cuda")[None]
    native = model.model(ids, position_ids=pos, use_cache=False).last_hidden_state
    ctl = FusedController(model)
    ctl.scoring = scoring
    ctl.reserved_recent = recent
    ctl.prefill_backend = "fused"
    ctl.reset()
    ctl.position_end = 137
    fused = model.model(ids, position_ids=pos, use_cache=False).last_hidden_state
    torch.testing.assert_close(fused, native, atol=.025, rtol=.02)
    original = {i: state["k"].clone() for i, state in ctl.states.items()}
    ctl.compress("fused_0.1", 137)
    for i, state in ctl.states.items():
        assert state["k"].shape[2] == 14
        assert set(state) == {"k", "v"}
        assert state["k"].untyped_storage().nbytes() == state["k"].numel() * state["k"].element_size()
        if recent:
            assert torch.equal(state["k"][:, :, -recent:], original[i][:, :, -recent:])
        # every compacted key is a key at its original (already RoPE-rotated) position
        assert all(any(torch.equal(state["k"][0, h, j], original[i][0, h, p]) for p in range(137))
                   for h in range(2) for j in range(14))
    ctl.position_end = 138
    out = model.model(ids[:, -1:], position_ids=torch.tensor([[137]], device="cuda"), use_cache=False)
    assert torch.isfinite(out.last_hidden_state).all()
    assert all(s["k"].shape[2] == 15 for s in ctl.states.values())
    ctl.close()
    assert model.config._attn_implementation == "sdpa"


# reference tests/test_streaming_adapter.py:9-35
@torch.inference_mode()
@pytest.mark.parametrize("scoring", [{"recency_decay": .1}, {"observation_window": 128}])
def test_immediate_layer_compaction_matches_delayed_compaction(scoring):
    torch.manual_seed(190)
    model = tiny_model(3)
    ids = torch.randint(0, 257, (1, 137), device="cuda")
    pos = torch.arange(137, device="cuda")[None]
    ctl = FusedController(model)
    ctl.prefill_backend = "fused"
    ctl.scoring = scoring
    ctl.reserved_recent = 16
    ctl.reset()
    ctl.position_end = 137
    delayed = model.model(ids, position_ids=pos, use_cache=False).last_hidden_state
    ctl.compress("fused_48", 137)
    cache = {i: {k: v.clone() for k, v in state.items()} for i, state in ctl.states.items()}
    ctl.position_end = 138
    decode = model.model(ids[:, -1:], position_ids=pos[:, -1:] + 1, use_cache=False).last_hidden_state
    ctl.close()
    ctl = StreamingController(model, budget=48, scoring=scoring, reserved_recent=16)
    ctl.reset()
    ctl.position_end = 137
    immediate = model.model(ids, position_ids=pos, use_cache=False).last_hidden_state
    assert torch.equal(immediate, delayed)
    for i, state in ctl.states.items():
        assert set(state) == {"k", "v"}
        for key, tensor in state.items():
            assert torch.equal(tensor, cache[i][key])
    ctl.finish_prefill()
    ctl.position_end = 138
    actual = model.model(ids[:, -1:], position_ids=pos[:, -1:] + 1, use_cache=False).last_hidden_state
    assert torch.equal(actual, decode)
    ctl.close()


# reference tests/test_streaming_adapter.py:38-59
@torch.inference_mode()
@pytest.mark.parametrize("backend,method", [("full", "full"), ("snap", "snap_48")])
def test_streaming_baselines_match_evaluator(backend, method):
    torch.manual_seed(17)
    model = tiny_model()
    ids = torch.randint(0, 257, (1, 137), device="cuda")
    pos = torch.arange(137, device="cuda")[None]
    ctl = FusedController(model)
    ctl.reset()
    ctl.position_end = 137
    expected = model.model(ids, position_ids=pos, use_cache=False).last_hidden_state
    ctl.compress(method, 137)
    cache = {i: {k: v.clone() for k, v in state.items()} for i, state in ctl.states.items()}
    ctl.close()
    ctl = StreamingController(model, backend=backend, budget=48)
    ctl.reset()
    ctl.position_end = 137
    actual = model.model(ids, position_ids=pos, use_cache=False).last_hidden_state
    torch.testing.assert_close(actual, expected, atol=.025, rtol=.02)
    for i, state in ctl.states.items():
        assert set(state) == {"k", "v"}
        assert state["k"].shape[2] == (137 if backend == "full" else 48)
        for key, tensor in state.items():
            torch.testing.assert_close(tensor, cache[i][key], atol=.005, rtol=.005)
    ctl.close()


# reference tests/test_streaming_adapter.py:62-76
@torch.inference_mode()
def test_chunked_mlp_and_restore():
    model = tiny_model()
    ids = torch.randint(0, 257, (1, 137), device="cuda")
    expected = model.model(ids, use_cache=False).last_hidden_state
    restore = chunk_mlp(model, 31)
    actual = model.model(ids, use_cache=False).last_hidden_state
    torch.testing.assert_close(actual, expected, atol=.025, rtol=.02)
    restore()
    assert torch.equal(model.model(ids, use_cache=False).last_hidden_state, expected)


# reference tests/test_quality_adapter.py:27-52
@torch.inference_mode()
@pytest.mark.parametrize("backend", ["full", "snap", "fused"])
def test_shared_prefill_matches_independent_policy(backend):
    torch.manual_seed(73)
    model = tiny_model()
    ids = torch.randint(0, 257, (1, 137), device="cuda")
    pos = torch.arange(137, device="cuda")[None]
    scoring = dict(recency_decay=.1, observation_window=128, value_weighted=True)
    methods = [dict(name="%s_%d" % (backend, budget), backend=backend, budget=budget, **scoring, reserved_recent=16)
               for budget in (32, 48)]
    paired = PairedController(model)
    paired.prepare(methods, 137)
    actual = model.model(ids, position_ids=pos, use_cache=False).last_hidden_state
    bank = paired.bank
    paired.close()
    for method in methods:
        ctl = StreamingController(model, backend=backend, budget=method["budget"], scoring=scoring,
                                  reserved_recent=16)
        ctl.reset()
        ctl.position_end = 137
        expected = model.model(ids, position_ids=pos, use_cache=False).last_hidden_state
        torch.testing.assert_close(actual, expected, atol=.001, rtol=.001)
        for layer, state in ctl.states.items():
            for key in ("k", "v"):
                torch.testing.assert_close(bank[method["name"]][layer][key], state[key], atol=.001, rtol=.001)
        ctl.close()


# reference tests/test_quality_adapter.py:55-76
@torch.inference_mode()
def test_batched_decode_matches_independent_caches():
    torch.manual_seed(91)
    model = tiny_model()
    ids = torch.randint(0, 257, (1, 137), device="cuda")
    ctl = PairedController(model)
    methods = [dict(name=name, backend=name, budget=48) for name in ("uniform_recent", "value_norm_only", "snap")]
    ctl.prepare(methods, 136)
    model.model(ids[:, :-1], position_ids=torch.arange(136, device="cuda")[None], use_cache=False)
    bank = {name: {i: {k: v.clone() for k, v in state.items()} for i, state in states.items()}
            for name, states in ctl.bank.items()}
    names = [m["name"] for m in methods]
    ctl.activate(names)
    batched = decode_batch(model, ctl, int(ids[0, -1]), 137, 8, set())
    assert len(batched) == 3 and all(len(g) == 8 for g in batched)
    for name, actual in zip(names, batched):
        ctl.bank = {name: bank[name]}
        ctl.activate([name])
        expected = decode_batch(model, ctl, int(ids[0, -1]), 137, 8, set())[0]
        assert actual == expected
    ctl.close()


# ---- additions of this build

@torch.inference_mode()
def test_h2o_mass_per_layer():
    torch.manual_seed(5)
    model = tiny_model()
    ids = torch.randint(0, 257, (1, 100), device="cuda")
    ctl = FusedController(model)
    ctl.prefill_backend = "fused"
    ctl.scoring = {"value_weighted": False}
    model.model(ids, use_cache=False)
    for state in ctl.states.values():
        # every query row is a distribution: the mass of a KV head sums to G * N
        torch.testing.assert_close(state["importance"].sum(-1), torch.full((1, 2), 2.0 * 100, device="cuda"),
                                   rtol=1e-4, atol=1e-3)
    ctl.close()


@torch.inference_mode()
def test_inference_transform_applies_before_scoring():
    torch.manual_seed(23)
    model = tiny_model()
    ids = torch.randint(0, 257, (1, 100), device="cuda")
    ctl = FusedController(model)
    ctl.prefill_backend = "fused"
    model.model(ids, use_cache=False)
    plain = {i: s["importance"].clone() for i, s in ctl.states.items()}
    v0 = ctl.states[0]["v"].clone()
    ctl.reset()
    ctl.inference_transform = lambda layer, k, v: (k, v * 2 if layer == 0 else v)
    model.model(ids, use_cache=False)
    # layer 0 sees V doubled (exact in bf16): P is unchanged and the value L1 norms double, so
    # its importance doubles (up to FP32 atomic order)
    assert torch.equal(ctl.states[0]["v"], v0 * 2)
    torch.testing.assert_close(ctl.states[0]["importance"], plain[0] * 2, rtol=1e-5, atol=1e-6)
    ctl.close()


@torch.inference_mode()
@pytest.mark.parametrize("method", ["full", "fused_full"])
def test_keeping_everything_decodes_like_the_uncompressed_model(method):
    """With nothing evicted, decoding through the controller's cache and through a
    DynamicCache handed to transformers both match the model's own cached decode."""
    torch.manual_seed(7)
    model = tiny_model(3)
    ids = torch.randint(0, 257, (1, 90), device="cuda")
    nxt = torch.randint(0, 257, (1, 1), device="cuda")
    pre = model(ids, use_cache=True)
    ref = model(nxt, past_key_values=pre.past_key_values, use_cache=True).logits
    ctl = FusedController(model)
    ctl.prefill_backend = "fused" if method.startswith("fused") else "baseline"
    model(ids, use_cache=False)
    ctl.compress(method, 90)
    cache = ctl.dynamic_cache()
    got = model(nxt, position_ids=torch.tensor([[90]], device="cuda"), use_cache=False).logits
    torch.testing.assert_close(got, ref, atol=.02, rtol=.02)
    ctl.close()
    via_cache = model(nxt, past_key_values=cache, use_cache=True, position_ids=torch.tensor([[90]], device="cuda"),
                      cache_position=torch.tensor([90], device="cuda")).logits
    torch.testing.assert_close(via_cache, ref, atol=.02, rtol=.02)


@torch.inference_mode()
def test_unavailable_baseline_method_is_an_error():
    model = tiny_model()
    ctl = FusedController(model)
    model.model(torch.randint(0, 257, (1, 40), device="cuda"), use_cache=False)
    with pytest.raises(ValueError, match="not available"):
        ctl.compress("h2o_16", 40)
    ctl.close()
