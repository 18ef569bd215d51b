"""The transformers integration on a tiny random-init Qwen2 (bf16, the reference adapter
tests' configuration, tests/test_adapter.py and tests/test_streaming_adapter.py): the
fused-prefill model matches the SDPA model (the reference's tolerance, atol .025 rtol .02),
importance is recorded per layer (H2O mass sums to G*N per KV head), compaction keeps the
budget with the reserved suffix and only original (RoPE-rotated) keys, and decoding from
the compacted cache works; with the full budget it reproduces uncompressed decoding. The
streaming controller (per-layer compaction during the forward) keeps exactly what delayed
compaction keeps (reference tests/test_streaming_adapter.py)."""
import pytest
import torch

from flash_evict.hf import EvictionController, PairedController, StreamingController, chunk_mlp, decode_batch

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")


def tiny_model(layers=2):
    cfg = transformers.Qwen2Config(vocab_size=257, hidden_size=128, intermediate_size=256, num_hidden_layers=layers,
                                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512)
    cfg._attn_implementation = "sdpa"
    return transformers.Qwen2ForCausalLM(cfg).cuda().to(torch.bfloat16).eval()


@torch.inference_mode()
@pytest.mark.parametrize("scoring,recent", [({}, 0), ({"recency_decay": .1}, 5), ({"observation_window": 32}, 5)])
def test_qwen_prefill_compress_decode(scoring, recent):
    torch.manual_seed(19)
    model = tiny_model()
    ids = torch.randint(0, 257, (1, 137), device="cuda")
    pos = torch.arange(137, device="cuda")[None]
    native = model.model(ids, position_ids=pos, use_cache=False).last_hidden_state
    ctl = EvictionController(model, scoring=scoring, reserved_recent=recent)
    fused = model.model(ids, position_ids=pos, use_cache=True)
    torch.testing.assert_close(fused.last_hidden_state, native, atol=.025, rtol=.02)
    original = {i: s["k"].clone() for i, s in ctl.states.items()}
    assert sorted(ctl.states) == [0, 1] and all(s["importance"].shape == (1, 2, 137) for s in ctl.states.values())
    cache = ctl.compress("fused_0.1")
    for i, state in ctl.states.items():
        assert state["k"].shape[2] == 14 and set(state) == {"k", "v"}
        # a compact tensor of its own, not a view into the prompt cache
        assert state["k"].untyped_storage().nbytes() == state["k"].numel() * state["k"].element_size()
        if recent:
            assert torch.equal(state["k"][:, :, -recent:], original[i][:, :, -recent:])
        # every compacted key is a key at its original (already RoPE-rotated) position
        assert all(any(torch.equal(state["k"][0, h, j], original[i][0, h, p]) for p in range(137))
                   for h in range(2) for j in range(14))
    out = model.model(ids[:, -1:], position_ids=torch.tensor([[137]], device="cuda"), past_key_values=cache,
                      use_cache=True, cache_position=torch.tensor([14], device="cuda"))
    assert torch.isfinite(out.last_hidden_state).all()
    assert cache.get_seq_length() == 15
    ctl.close()
    assert model.config._attn_implementation == "sdpa"


@torch.inference_mode()
def test_h2o_mass_per_layer():
    torch.manual_seed(5)
    model = tiny_model()
    ids = torch.randint(0, 257, (1, 100), device="cuda")
    ctl = EvictionController(model, scoring={"value_weighted": False})
    model.model(ids, use_cache=False)
    for state in ctl.states.values():
        # every query row is a distribution: the mass of a KV head sums to G * N
        torch.testing.assert_close(state["importance"].sum(-1), torch.full((1, 2), 2.0 * 100, device="cuda"),
                                   rtol=1e-4, atol=1e-3)
    ctl.close()


@torch.inference_mode()
@pytest.mark.parametrize("backend", ["fused", "snap", "full"])
def test_full_budget_decode_matches_uncompressed(backend):
    torch.manual_seed(7)
    model = tiny_model(3)
    ids = torch.randint(0, 257, (1, 90), device="cuda")
    nxt = torch.randint(0, 257, (1, 1), device="cuda")
    ctl = EvictionController(model, backend=backend, reserved_recent=8)
    pre = model(ids, use_cache=True)
    ref = model(nxt, past_key_values=pre.past_key_values, use_cache=True).logits
    ctl.reset()
    model(ids, use_cache=True)
    cache = ctl.compress(90)
    got = model(nxt, past_key_values=cache, use_cache=True, position_ids=torch.tensor([[90]], device="cuda"),
                cache_position=torch.tensor([90], device="cuda")).logits
    assert torch.equal(got, ref)
    ctl.close()


@torch.inference_mode()
def test_snap_backend_budget():
    torch.manual_seed(11)
    model = tiny_model()
    ids = torch.randint(0, 257, (1, 137), device="cuda")
    ctl = EvictionController(model, backend="snap")
    model.model(ids, use_cache=False)
    ctl.compress(48)
    for state in ctl.states.values():
        assert state["k"].shape[2] == 48
    ctl.close()


def _decode_one(model, ids, cache, n_prompt, kept):
    return model.model(ids[:, -1:], position_ids=torch.tensor([[n_prompt]], device="cuda"), past_key_values=cache,
                       use_cache=True, cache_position=torch.tensor([kept], device="cuda")).last_hidden_state


# reference tests/test_streaming_adapter.py:9-35: compacting each layer during the forward
# equals compacting all layers after it, and decoding from either cache agrees
@torch.inference_mode()
@pytest.mark.parametrize("scoring", [{"recency_decay": .1}, {"observation_window": 128}])
def test_immediate_layer_compaction_matches_delayed_compaction(scoring):
    torch.manual_seed(190)
    model = tiny_model(3)
    ids = torch.randint(0, 257, (1, 137), device="cuda")
    pos = torch.arange(137, device="cuda")[None]
    ctl = EvictionController(model, scoring=scoring, reserved_recent=16)
    delayed = model.model(ids, position_ids=pos, use_cache=False).last_hidden_state
    cache = ctl.compress(48)
    states = {i: {k: t.clone() for k, t in s.items()} for i, s in ctl.states.items()}
    decode = _decode_one(model, ids, cache, 137, 48)
    ctl.close()
    ctl = StreamingController(model, budget=48, scoring=scoring, reserved_recent=16)
    immediate = model.model(ids, position_ids=pos, use_cache=False).last_hidden_state
    assert torch.equal(immediate, delayed)
    for i, state in ctl.states.items():
        assert set(state) == {"k", "v"}
        for key, tensor in state.items():
            assert torch.equal(tensor, states[i][key])
    actual = _decode_one(model, ids, ctl.finish_prefill(), 137, 48)
    assert torch.equal(actual, decode)
    ctl.close()
    assert model.config._attn_implementation == "sdpa"


# reference tests/test_streaming_adapter.py:38-59
@torch.inference_mode()
@pytest.mark.parametrize("backend", ["full", "snap"])
def test_streaming_baselines_match_delayed(backend):
    torch.manual_seed(17)
    model = tiny_model()
    ids = torch.randint(0, 257, (1, 137), device="cuda")
    native = model.model(ids, use_cache=False).last_hidden_state
    ctl = EvictionController(model, backend=backend)
    expected = model.model(ids, use_cache=False).last_hidden_state
    ctl.compress(48 if backend == "snap" else 137)
    states = {i: {k: t.clone() for k, t in s.items()} for i, s in ctl.states.items()}
    ctl.close()
    ctl = StreamingController(model, backend=backend, budget=48)
    actual = model.model(ids, use_cache=False).last_hidden_state
    torch.testing.assert_close(actual, native, atol=.025, rtol=.02)
    assert torch.equal(actual, expected)
    for i, state in ctl.states.items():
        assert set(state) == {"k", "v"}
        assert state["k"].shape[2] == (48 if backend == "snap" else 137)
        for key, tensor in state.items():
            assert torch.equal(tensor, states[i][key])
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


# reference tests/test_quality_adapter.py:27-52: one shared prefill gives every policy the
# cache the streaming controller gives it alone
@torch.inference_mode()
@pytest.mark.parametrize("backend", ["full", "snap", "fused"])
def test_shared_prefill_matches_independent_policy(backend):
    torch.manual_seed(73)
    model = tiny_model()
    ids = torch.randint(0, 257, (1, 137), device="cuda")
    pos = torch.arange(137, device="cuda")[None]
    scoring = dict(recency_decay=.1, observation_window=128, value_weighted=True)
    methods = [dict(name="%s_%d" % (backend, b), backend=backend, budget=b, **scoring, reserved_recent=16)
               for b in (32, 48)]
    paired = PairedController(model)
    paired.prepare(methods, 137)
    actual = model.model(ids, position_ids=pos, use_cache=False).last_hidden_state
    bank = paired.bank
    paired.close()
    for method in methods:
        ctl = StreamingController(model, backend=backend, budget=method["budget"], scoring=scoring,
                                  reserved_recent=16)
        expected = model.model(ids, position_ids=pos, use_cache=False).last_hidden_state
        assert torch.equal(actual, expected)
        for layer, state in ctl.states.items():
            for key in ("k", "v"):
                assert torch.equal(bank[method["name"]][layer][key], state[key])
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
    bank = {name: {i: {k: t.clone() for k, t in state.items()} for i, state in states.items()}
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


@torch.inference_mode()
def test_inference_transform_applies_before_scoring():
    torch.manual_seed(23)
    model = tiny_model()
    ids = torch.randint(0, 257, (1, 100), device="cuda")
    ctl = EvictionController(model)
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
