"""Per-layer compaction during the prefill forward (reference
flash_evict/streaming_adapter.py:16-87 in anishesg/flash-evict-prefill).

`StreamingController(model, backend=..., budget=..., scoring=..., reserved_recent=...,
pool_kernel=...)` is a FusedController that compacts each layer's K/V to `budget` tokens as
soon as that layer's attention has run. The attention output every layer passes on stays
exact; only the stored K/V shrink, so the full prompt caches of all layers are never held at
once. Backends: "fused" (the library's importance, the tokens `compress("fused_<budget>")`
keeps), "snap" (SnapKV over the last 32 queries) and "full" (nothing dropped).
`finish_prefill()` switches to decoding, which grows the compacted cache.

`chunk_mlp(model, chunk_size)` bounds the feed-forward activations of long prompts
(streaming_adapter.py:30-51).
"""
import torch

from .baselines import flash_attention, snap_scores, snap_select
from .controller import SNAP_WINDOW, compact
from .kv_distill_adapter import FusedController

__all__ = ["StreamingController", "chunk_mlp"]

BACKENDS = ("fused", "snap", "full")


class StreamingController(FusedController):
    def __init__(self, model, *, backend="fused", budget=1024, scoring=None, reserved_recent=64, pool_kernel=1):
        # argument checks come first, before the model is touched
        if backend not in BACKENDS:
            raise ValueError("Unsupported backend")
        if isinstance(budget, bool) or not isinstance(budget, int) or budget < 1:
            raise ValueError("Positive integer budget required")
        super().__init__(model)
        self.prefill_backend = backend
        self.cache_budget = budget
        self.scoring = dict(scoring or {})
        self.reserved_recent = reserved_recent
        self.pool_kernel = pool_kernel

    def _prefill_layer(self, layer, q, k, v, scaling):
        budget = min(k.shape[2], self.cache_budget)
        if self.prefill_backend == "fused":
            out = super()._prefill_layer(layer, q, k, v, scaling)
            state = self.states[layer]
            compact(state, self._fused_keep(state, budget))
            return out
        out = flash_attention(q, k, v)
        state = self.states[layer] = {"k": k, "v": v}
        if self.prefill_backend == "snap":
            compact(state, snap_select(snap_scores(q, k, SNAP_WINDOW), budget, SNAP_WINDOW)[0])
        return out

    def finish_prefill(self):
        """End of the prompt forward: decode from (and grow) the compacted cache."""
        self.mode = "decode"
        self.method = "full"


def chunk_mlp(model, chunk_size):
    """Run every decoder layer's MLP over at most `chunk_size` positions at a time, bounding
    the feed-forward activation memory of long prompts. Inference only. Returns a function
    that restores the original MLP forwards."""
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
            return torch.cat([forward(hidden[:, i:i + chunk_size]) for i in range(0, n, chunk_size)], dim=1)
        return run

    for layer in model.model.layers:
        saved.append((layer.mlp, layer.mlp.forward))
        layer.mlp.forward = chunked(layer.mlp.forward)

    def restore():
        for mlp, forward in saved:
            mlp.forward = forward
    return restore
