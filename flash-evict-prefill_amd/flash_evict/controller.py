"""Per-model KV controller: a local stand-in for `kv_distill.attention.Controller`.

The reference's model adapters (flash_evict/kv_distill_adapter.py:16, streaming_adapter.py:16,
quality_adapter.py:55 in anishesg/flash-evict-prefill) subclass the Controller of kv_distill, an
external evaluation package the reference does not vendor. This module gives the same
contract on the installed transformers, so those adapters' callers and tests run unchanged:

  * `Controller(model)` routes every attention layer of `model` through the controller
    (transformers' AttentionInterface; the reference patches the forwards of an older
    transformers release). `close()` restores the model's attention implementation.
  * mode "prefill": one unpadded prompt (batch 1, no external cache, `use_cache=False`).
    Each layer's output comes from `_prefill_layer`, and the layer's K/V (RoPE already
    applied, so a kept key keeps its original position) are held in `states[layer]` as
    {"k", "v", ...}. `inference_transform`, when set, maps (layer, k, v) -> (k, v) first.
  * `compress(method, prompt_length)`: the baseline methods "full" (keep every prompt
    token) and "snap_<budget>" (SnapKV over the last 32 prompt queries, pooling 5:
    flash_evict.baselines); then mode "decode". A budget is a count ("48"), a fraction of
    the prompt ("0.1") or "full".
  * mode "decode": each forward (`use_cache=False`) appends its tokens' K/V to `states`
    and attends over the whole stored cache, so the cache grows after compression.
  * `reset()` clears the states and returns to prefill; `method` and `position_end` are
    kept as the reference's callers set them (RoPE positions here come from position_ids).
  * `dynamic_cache()` hands the stored K/V to transformers as a `DynamicCache` (for
    `generate`), an addition of this build.
"""
import math

import torch
from torch.nn.attention import SDPBackend, sdpa_kernel

from .baselines import flash_attention, snap_scores, snap_select
from .cache import gather_tokens

# Name of the registered attention implementation (transformers treats names containing
# "flash" as hub flash-attention kernels, so the name avoids that word).
ATTN_NAME = "evict_prefill"
SNAP_WINDOW = 32
_registered = []


def _route(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """The registered attention function: layers owned by a controller go to it."""
    ctl = getattr(module, "_flash_evict_controller", None)
    if ctl is None:
        from transformers.integrations.sdpa_attention import sdpa_attention_forward
        return sdpa_attention_forward(module, query, key, value, attention_mask, scaling=scaling, dropout=dropout,
                                      **kwargs)
    return ctl._attend(module, query, key, value, scaling)


def _register():
    if not _registered:
        from transformers import AttentionInterface
        from transformers.masking_utils import AttentionMaskInterface, sdpa_mask
        AttentionInterface.register(ATTN_NAME, _route)
        AttentionMaskInterface.register(ATTN_NAME, sdpa_mask)
        _registered.append(ATTN_NAME)


def parse_budget(spec, prompt_length):
    """Token budget of a method suffix: "full", a fraction of the prompt ("0.1", rounded up)
    or a count ("48"), clamped to [1, prompt_length] (kv_distill_adapter.py:31-33)."""
    if spec == "full":
        count = prompt_length
    elif "." in spec:
        count = math.ceil(float(spec) * prompt_length)
    else:
        count = int(spec)
    return min(max(count, 1), prompt_length)


def compact(state, indices):
    """Replace a layer's K/V by the rows `indices` [B, Hkv, kept] (own storage, not views)."""
    state["k"] = gather_tokens(state["k"], indices)
    state["v"] = gather_tokens(state["v"], indices)


def _visible_mask(t, total, device):
    """Boolean [1, 1, t, total]: query i of the newest t positions sees keys up to its own."""
    rows = torch.arange(t, device=device)[:, None] + (total - t)
    return (torch.arange(total, device=device)[None, :] <= rows)[None, None]


class Controller:
    def __init__(self, model):
        _register()
        self.model = model
        self.states = {}
        self.mode = "prefill"
        self.method = None
        self.position_end = None
        self.inference_transform = None
        self._layers = [m for m in model.modules() if hasattr(m, "layer_idx") and hasattr(m, "q_proj")]
        for m in self._layers:
            m._flash_evict_controller = self
        self._previous_impl = model.config._attn_implementation
        model.set_attn_implementation(ATTN_NAME)

    # -- lifecycle
    def reset(self):
        self.states = {}
        self.mode = "prefill"
        self.method = None

    def close(self):
        for m in self._layers:
            if getattr(m, "_flash_evict_controller", None) is self:
                del m._flash_evict_controller
        self.model.set_attn_implementation(self._previous_impl)

    # -- attention
    def _attend(self, module, query, key, value, scaling):
        layer = module.layer_idx
        if self.mode == "prefill":
            if query.shape[0] != 1:
                raise ValueError("Prefill expects one unpadded prompt at a time")
            if key.shape[2] != query.shape[2]:
                raise ValueError("Prefill expects an empty external cache (use_cache=False)")
            if self.inference_transform is not None:
                key, value = self.inference_transform(layer, key, value)
            return self._prefill_layer(layer, query, key, value, scaling).transpose(1, 2), None
        return self._decode_layer(layer, query, key, value, scaling), None

    def _prefill_layer(self, layer, q, k, v, scaling):
        """Baseline prefill: the exact attention of flash_evict.baselines, with the layer's
        SnapKV scores kept for a later "snap_<budget>" compression."""
        self.states[layer] = {"k": k, "v": v, "snap": snap_scores(q, k, SNAP_WINDOW)}
        return flash_attention(q, k, v)

    def _decode_layer(self, layer, q, k, v, scaling):
        state = self.states[layer]
        state["k"] = torch.cat((state["k"], k), 2)
        state["v"] = torch.cat((state["v"], v), 2)
        keys, vals = state["k"], state["v"]
        t, total = q.shape[2], keys.shape[2]
        g = q.shape[1] // keys.shape[1]
        if g > 1:
            keys, vals = keys.repeat_interleave(g, 1), vals.repeat_interleave(g, 1)
        mask = _visible_mask(t, total, q.device) if t > 1 else None
        # fused SDPA kernels only: the unfused math path forms batched products with a
        # transposed right operand, which this stack does not run reliably in bf16
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            out = torch.nn.functional.scaled_dot_product_attention(q, keys.contiguous(), vals.contiguous(),
                                                                   attn_mask=mask, scale=scaling)
        return out.transpose(1, 2)

    # -- compression
    def compress(self, method, prompt_length):
        """Baseline methods: "full" or "snap_<budget>"."""
        if method == "full":
            select = None
        elif method.startswith("snap_"):
            budget = parse_budget(method[len("snap_"):], prompt_length)

            def select(state):
                return snap_select(state["snap"], budget, SNAP_WINDOW)[0]
        else:
            raise ValueError("method %r is not available: the baseline methods are 'full' and 'snap_<budget>'; "
                             "the other kv_distill evaluator methods are not part of this build" % (method,))
        for state in self.states.values():
            if select is not None:
                compact(state, select(state))
            for extra in [key for key in state if key not in ("k", "v")]:
                del state[extra]
        self.method = method
        self.mode = "decode"

    def dynamic_cache(self):
        """The stored K/V of every layer as a transformers DynamicCache."""
        from transformers import DynamicCache
        cache = DynamicCache()
        for layer in sorted(self.states):
            cache.update(self.states[layer]["k"], self.states[layer]["v"], layer)
        return cache
