"""KV compaction gather oracle in numpy (test infrastructure only).

Restates kv_distill.cache.gather_tokens as the reference calls it
(flash_evict/kv_distill_adapter.py:38-39, streaming_adapter.py:86,
quality_adapter.py:109-110 of anishesg/flash-evict-prefill). kv_distill is a local
research package (`/home/qcb/kv-distill` in the reference README) with no published
version; the contract comes from the call sites: cache [B, H, N, D], int64 indices
[B, H, K], result [B, H, K, D] with out[b,h,j,:] = cache[b,h,indices[b,h,j],:].
This build defines an index outside [0, N) to give a zero row.
"""
import numpy as np


def gather_tokens(cache, indices):
    """out[b, h, j, :] = cache[b, h, indices[b, h, j], :]; zero rows for bad indices."""
    cache = np.asarray(cache)
    idx = np.asarray(indices, dtype=np.int64)
    b, h, n, d = cache.shape
    assert idx.shape[:2] == (b, h)
    ok = (idx >= 0) & (idx < n)
    safe = np.where(ok, idx, 0)
    out = np.take_along_axis(cache, safe[..., None], axis=2)
    return np.where(ok[..., None], out, np.zeros((), dtype=cache.dtype))
