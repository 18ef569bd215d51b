"""The transformers integration on a tiny random-init Qwen2 (bf16, the reference adapter
tests' configuration, tests/test_adapter.py and tests/test_streaming_adapter.py): the
fused-prefill model matches the SDPA model (the reference's tolerance, atol .025 rtol .02),
importance is recorded per layer (H2O mass sums to G*N per KV head), compaction keeps the
budget with the reserved suffix and only original (RoPE-rotated) keys, and decoding from
the compacted cache works; with the full budget it reproduces uncompressed decoding."""
import pytest
import torch

from flash_evict.hf import EvictionController

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
