"""Fused-prefill controller for Hugging Face decoder models (reference
flash_evict/kv_distill_adapter.py:16-67 in anishesg/flash-evict-prefill).

`FusedController(model)` is the reference's class on the local Controller stand-in
(flash_evict.controller). Attributes a caller sets before the prompt forward:
  prefill_backend  "baseline" (exact attention, baseline methods) or "fused" (the
                   library's fused attention + replay importance per layer)
  scoring          prefill keyword arguments: recency_decay, observation_window,
                   value_weighted
  reserved_recent  prompt suffix always kept by "fused_*" compression
  pool_kernel      SnapKV-style pooling of the importance before top-k
`compress("fused_<budget>", prompt_length)` keeps, per layer and KV head, the `budget`
tokens select_tokens picks from that layer's importance and gathers their K/V; any other
method goes to the baseline Controller. Decoding then grows the compacted cache.
"""
from .controller import Controller, compact, parse_budget
from .prefill import prefill, select_tokens

__all__ = ["FusedController"]


class FusedController(Controller):
    def __init__(self, model):
        super().__init__(model)
        self.prefill_backend = "baseline"
        self.scoring = {}
        self.reserved_recent = 0
        self.pool_kernel = 1

    def _prefill_layer(self, layer, q, k, v, scaling):
        if self.prefill_backend != "fused":
            return super()._prefill_layer(layer, q, k, v, scaling)
        out, importance = prefill(q, k, v, scale=scaling, **self.scoring)
        self.states[layer] = {"k": k, "v": v, "importance": importance}
        return out

    def _fused_keep(self, state, budget):
        """Kept indices [B, Hkv, budget] of one layer; consumes its importance."""
        keep, _ = select_tokens(state.pop("importance"), budget, recent=min(self.reserved_recent, budget),
                                pool_kernel=self.pool_kernel)
        return keep

    def compress(self, method, prompt_length):
        prefix = "fused_"
        if not method.startswith(prefix):
            return super().compress(method, prompt_length)
        budget = parse_budget(method[len(prefix):], prompt_length)
        for state in self.states.values():
            compact(state, self._fused_keep(state, budget))
        self.method = method
        self.mode = "decode"
