"""Hugging Face transformers integration: fused prefill with importance inside a model, then
KV-cache compaction by the kept indices.

This stands in for the reference's kv_distill adapters (flash_evict/kv_distill_adapter.py:16-67,
streaming_adapter.py:16-87, quality_adapter.py:38-52 of anishesg/flash-evict-prefill). Those
patch the attention forwards of an older transformers release and drive kv_distill's
Controller, a research package the reference does not vendor. Here the same flow uses the
pluggable attention of current transformers (`AttentionInterface`): during a prefill
forward every attention layer runs `prefill` (gfx950 kernels) and records its importance;
`compress` then selects and gathers each layer's K/V (`select_tokens`, `gather_tokens`) into a
new `DynamicCache`, and decoding continues from that cache at the original positions (the
kept keys keep their RoPE rotation), as the reference's fused controller does after
prefill. Decode steps (one query against the cache) use torch's SDPA, as the reference
hands decoding to the upstream attention.

`StreamingController` compacts each layer's K/V as soon as that layer's prefill attention
has run (reference streaming_adapter.py:16-87), so the full caches of all layers are never
held together; `chunk_mlp` bounds the feed-forward activations of long prompts
(streaming_adapter.py:30-51). `PairedController` shares one prefill forward between several
policies and decodes their caches as one batch (quality_adapter.py:55-136).
"""
import math

import torch

from .baselines import flash_attention, snap_scores, snap_select
from .cache import gather_tokens
from .prefill import prefill, select_tokens

# registered attention implementation name (transformers treats names containing "flash" as
# flash-attention kernels from its hub, so the name avoids that word)
ATTN_NAME = "evict_prefill"
_registered = False


def _sdpa(module, query, key, value, attention_mask, **kwargs):
    from transformers.integrations.sdpa_attention import sdpa_attention_forward
    return sdpa_attention_forward(module, query, key, value, attention_mask, **kwargs)


def _attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """The registered attention function: prefill (query length = key length) runs the fused
    kernels and records the layer's state; anything else goes to SDPA."""
    ctl = getattr(module, "_flash_evict_controller", None)
    if ctl is None or ctl.mode != "prefill" or query.shape[2] != key.shape[2]:
        return _sdpa(module, query, key, value, attention_mask, scaling=scaling, dropout=dropout, **kwargs)
    if query.shape[0] != 1:
        raise ValueError("flash_evict prefill expects one unpadded prompt at a time")
    layer = module.layer_idx
    if ctl.inference_transform is not None:   # kv_distill_adapter.py:62-63
        key, value = ctl.inference_transform(layer, key, value)
    if ctl.backend == "fused":
        out, importance = prefill(query, key, value, scale=scaling, **ctl.scoring)
        ctl._store(layer, {"k": key, "v": value, "importance": importance})
    elif ctl.backend == "snap":
        out = flash_attention(query, key, value)
        ctl._store(layer, {"k": key, "v": value, "snap": snap_scores(query, key, ctl.snap_window)})
    else:   # "full"
        out = flash_attention(query, key, value)
        ctl._store(layer, {"k": key, "v": value})
    return out.transpose(1, 2), None


def _register():
    global _registered
    if not _registered:
        from transformers import AttentionInterface
        from transformers.masking_utils import AttentionMaskInterface, sdpa_mask
        AttentionInterface.register(ATTN_NAME, _attention)
        AttentionMaskInterface.register(ATTN_NAME, sdpa_mask)
        _registered = True


def _budget(method_suffix, prompt_length):
    """Budget of a method suffix as the reference's compress parses it
    (kv_distill_adapter.py:31-33): 'full', a fraction ('0.1') or a count ('48')."""
    if method_suffix == "full":
        budget = prompt_length
    elif "." in method_suffix:
        budget = math.ceil(prompt_length * float(method_suffix))
    else:
        budget = int(method_suffix)
    return max(1, min(budget, prompt_length))


class EvictionController:
    """Runs a model's prefill through the fused kernels and compacts its KV cache.

    backend: "fused" (importance from the fused replay), "snap" (SnapKV scores of the last
    `snap_window` queries, torch SDPA attention) or "full" (no scoring; compaction keeps
    everything). `scoring` holds prefill keyword arguments (recency_decay,
    observation_window, value_weighted). Use `mode = "prefill"` (the default after
    construction) for the prompt forward, then `compress`. `inference_transform`, when set,
    is called as f(layer_idx, k, v) -> (k, v) on each layer's prompt K/V before attention and
    scoring (the reference's Controller hook, kv_distill_adapter.py:62-63).
    """

    def __init__(self, model, *, backend="fused", scoring=None, reserved_recent=0, pool_kernel=1, snap_window=32):
        if backend not in ("fused", "snap", "full"):
            raise ValueError("Unsupported backend")
        _register()
        self.model = model
        self.backend = backend
        self.scoring = dict(scoring or {})
        self.reserved_recent = reserved_recent
        self.pool_kernel = pool_kernel
        self.snap_window = snap_window
        self.states = {}
        self.mode = "prefill"
        self.inference_transform = None
        self._previous = model.config._attn_implementation
        self._modules = [m for m in model.modules() if hasattr(m, "layer_idx") and hasattr(m, "q_proj")]
        for m in self._modules:
            m._flash_evict_controller = self
        model.set_attn_implementation(ATTN_NAME)

    def reset(self):
        self.states = {}
        self.mode = "prefill"

    def _store(self, layer, state):
        """Keep one layer's prefill state (K, V and its scores) until `compress`."""
        self.states[layer] = state

    def _indices(self, state, budget):
        """Ascending kept indices [B, Hkv, budget] of one layer's state, or None to keep all."""
        n = state["k"].shape[2]
        b = max(1, min(budget, n))
        if self.backend == "fused":
            return select_tokens(state["importance"], b, recent=min(self.reserved_recent, b),
                                 pool_kernel=self.pool_kernel)[0]
        if self.backend == "snap":
            return snap_select(state["snap"], b, self.snap_window)[0]
        return None

    def kept_indices(self, budget):
        """Per layer, the ascending kept indices [B, Hkv, budget] of the method."""
        kept = {}
        for layer, state in self.states.items():
            idx = self._indices(state, budget)
            if idx is None:
                n = state["k"].shape[2]
                idx = torch.arange(n, device=state["k"].device).expand(*state["k"].shape[:2], n)
            kept[layer] = idx
        return kept

    def _cache(self):
        from transformers import DynamicCache
        cache = DynamicCache()
        for layer in sorted(self.states):
            cache.update(self.states[layer]["k"], self.states[layer]["v"], layer)
        return cache

    def compress(self, budget):
        """Compact every layer's K/V to `budget` tokens (an int, or a method suffix such as
        'fused_0.1' / '0.1' / '48' / 'full' as the reference's compress accepts) and return
        the compacted `DynamicCache`. Switches to decode mode."""
        if not self.states:
            raise RuntimeError("compress needs a prefill forward first")
        n = next(iter(self.states.values()))["k"].shape[2]
        if isinstance(budget, str):
            budget = _budget(budget.split("_")[-1], n)
        kept = self.kept_indices(budget)
        for layer in sorted(self.states):
            state = self.states[layer]
            self.states[layer] = {"k": gather_tokens(state["k"], kept[layer]), "v": gather_tokens(state["v"], kept[layer])}
        self.mode = "decode"
        return self._cache()

    def close(self):
        """Restore the model's previous attention implementation."""
        for m in self._modules:
            if getattr(m, "_flash_evict_controller", None) is self:
                del m._flash_evict_controller
        self.model.set_attn_implementation(self._previous)


class StreamingController(EvictionController):
    """Compacts each layer's K/V during the prefill forward, right after that layer's
    attention (reference streaming_adapter.py:16-27,55-87): the attention output of every
    layer stays exact for the next layer, only the stored K/V shrink to `budget` tokens, so
    the full prompt caches of all layers are never held at once. Run the prompt forward
    with use_cache=False, then `finish_prefill()` returns the compacted `DynamicCache` for
    decoding. The kept tokens are those `EvictionController.compress(budget)` keeps.
    """

    def __init__(self, model, *, backend="fused", budget=1024, scoring=None, reserved_recent=64, pool_kernel=1,
                 snap_window=32):
        if backend not in ("fused", "snap", "full"):
            raise ValueError("Unsupported backend")
        if isinstance(budget, bool) or not isinstance(budget, int) or budget < 1:
            raise ValueError("Positive integer budget required")
        self.cache_budget = budget
        super().__init__(model, backend=backend, scoring=scoring, reserved_recent=reserved_recent,
                         pool_kernel=pool_kernel, snap_window=snap_window)

    def _store(self, layer, state):
        idx = self._indices(state, self.cache_budget)
        if idx is None:
            self.states[layer] = {"k": state["k"], "v": state["v"]}
        else:
            self.states[layer] = {"k": gather_tokens(state["k"], idx), "v": gather_tokens(state["v"], idx)}

    def finish_prefill(self):
        """The compacted `DynamicCache` of every layer; switches to decode mode."""
        if not self.states:
            raise RuntimeError("finish_prefill needs a prefill forward first")
        self.mode = "decode"
        return self._cache()

    def compress(self, budget):
        raise RuntimeError("StreamingController compacts during the prefill forward; call finish_prefill()")


def chunk_mlp(model, chunk_size):
    """Run every decoder layer's MLP over at most `chunk_size` positions at a time, bounding
    the feed-forward activation memory of long prompts (reference streaming_adapter.py:30-51).
    Inference only. Returns a function that restores the original MLP forwards."""
    if isinstance(chunk_size, bool) or not isinstance(chunk_size, int) or chunk_size < 1:
        raise ValueError("chunk_size must be a positive integer")
    saved = []

    def chunked(forward):
        def run(hidden):
            if torch.is_grad_enabled():
                raise RuntimeError("Chunked MLP is inference-only")
            n = hidden.shape[1]
            if n <= chunk_size:
                return forward(hidden)
            parts = [forward(hidden[:, i:i + chunk_size]) for i in range(0, n, chunk_size)]
            return torch.cat(parts, dim=1)
        return run

    for layer in model.model.layers:
        saved.append((layer.mlp, layer.mlp.forward))
        layer.mlp.forward = chunked(layer.mlp.forward)

    def restore():
        for mlp, forward in saved:
            mlp.forward = forward
    return restore


def default_methods():
    """The evaluation's policy list (reference quality_adapter.py:19-31): the full cache, SnapKV
    and three fused policies at budgets 256 and 1024, and two 256-token ablations."""
    methods = [dict(name="full", backend="full", budget=None)]
    for budget in (256, 1024):
        methods.append(dict(name="snap_%d" % budget, backend="snap", budget=budget))
        for label, window, recent in (("d01_r0", 0, 0), ("d0.1_w128_r0", 128, 0), ("d0.1_w128_r64", 128, 64)):
            methods.append(dict(name="%s_%d" % (label, budget), backend="fused", budget=budget, recency_decay=.1,
                                observation_window=window, value_weighted=True, reserved_recent=recent))
    methods += [dict(name="%s_256" % backend, backend=backend, budget=256)
                for backend in ("value_norm_only", "uniform_recent")]
    return methods


def group_key(method):
    """Policies that can share one prefill forward have equal keys (quality_adapter.py:34-37):
    every baseline uses the same attention output; fused policies need equal scoring."""
    if method["backend"] != "fused":
        return ("baseline",)
    return ("fused", method["recency_decay"], method["observation_window"], method["value_weighted"])


class PairedController(EvictionController):
    """Several eviction policies share one prefill forward, then decode their own compacted
    caches as one batch (reference quality_adapter.py:55-81,84-112).

    `prepare(methods)` takes policies of one `group_key`. During the prompt forward (run with
    use_cache=False) every layer computes its attention once, then stores each policy's
    compacted K/V in `bank[name][layer]` (`choose_indices`). `activate(names)` concatenates the
    named caches along the batch (equal retained lengths) into a `DynamicCache`, kept as
    `self.cache`, for `decode_batch`.
    """

    def __init__(self, model):
        super().__init__(model, backend="full")
        self.bank = {}
        self.active_methods = []
        self.cache = None

    def prepare(self, methods, length=None):
        methods = list(methods)
        if not methods or len({group_key(m) for m in methods}) != 1:
            raise ValueError("A shared prefill requires identical attention output and score settings")
        self.reset()
        self.active_methods = methods
        self.bank = {m["name"]: {} for m in methods}
        first = methods[0]
        if first["backend"] == "fused":
            self.backend = "fused"
            self.scoring = {key: first[key] for key in ("recency_decay", "observation_window", "value_weighted")}
        else:
            self.backend = "snap" if any(m["backend"] == "snap" for m in methods) else "full"
            self.scoring = {}

    def _store(self, layer, state):
        k, v = state["k"], state["v"]
        for method in self.active_methods:
            idx = choose_indices(method, k, v, state.get("importance"), state.get("snap"))
            self.bank[method["name"]][layer] = {"k": k if idx is None else gather_tokens(k, idx),
                                                "v": v if idx is None else gather_tokens(v, idx)}

    def activate(self, names, *, consume=True):
        """Batch the named policies' caches (the same retained length) for decoding."""
        sources = [self.bank[name] for name in names]
        self.states = {layer: {key: torch.cat([src[layer][key] for src in sources], 0) if len(sources) > 1
                               else sources[0][layer][key] for key in ("k", "v")} for layer in sources[0]}
        self.mode = "decode"
        if consume:
            for name in names:
                del self.bank[name]
        self.cache = self._cache()
        return self.cache


@torch.inference_mode()
def decode_batch(model, ctl, last_token, prompt_length, max_new_tokens, stop_ids, *, suppress_first_stop=False):
    """Greedy decoding of every cache of `ctl.activate(...)` from the prompt's last token at
    position prompt_length-1 (reference quality_adapter.py:115-136); returns the generated
    ids per batch row, each ending at its first stop id."""
    cache = ctl.cache
    batch = next(iter(ctl.states.values()))["k"].shape[0]
    kept = cache.get_seq_length()
    device = next(model.parameters()).device
    token = torch.full((batch, 1), last_token, dtype=torch.long, device=device)
    generated = [[] for _ in range(batch)]
    finished = [False] * batch
    for step in range(max_new_tokens):
        pos = torch.full((batch, 1), prompt_length - 1 + step, dtype=torch.long, device=device)
        hidden = model.model(token, position_ids=pos, past_key_values=cache, use_cache=True,
                             cache_position=torch.tensor([kept + step], device=device)).last_hidden_state
        logits = model.lm_head(hidden[:, -1])
        if suppress_first_stop and step == 0:
            logits[:, list(stop_ids)] = -torch.inf
        token = logits.argmax(-1, keepdim=True)
        for i, token_id in enumerate(token[:, 0].tolist()):
            if not finished[i]:
                generated[i].append(token_id)
                finished[i] = token_id in stop_ids
        if all(finished):
            break
    return generated


def choose_indices(method, k, v, importance=None, snap=None):
    """Kept indices of one evaluation policy (reference quality_adapter.py:38-52): None for
    the full cache, a suffix for 'uniform_recent', the largest value L1 norms for
    'value_norm_only', SnapKV for 'snap', and the fused importance otherwise."""
    n = k.shape[2]
    budget = min(n, method["budget"] or n)
    if method["backend"] == "full" or budget == n:
        return None
    if method["backend"] == "uniform_recent":
        return torch.arange(n - budget, n, device=k.device).expand(*k.shape[:2], budget)
    if method["backend"] == "value_norm_only":
        return select_tokens(v.float().abs().sum(-1), budget)[0]
    if method["backend"] == "snap":
        return snap_select(snap, budget, window=32, kernel=5)[0]
    return select_tokens(importance, budget, reserved_recent=min(budget, method["reserved_recent"]))[0]
