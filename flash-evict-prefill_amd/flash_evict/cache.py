"""KV cache compaction: `gather_tokens`, the consumer of the kept indices.

The reference adapters call `kv_distill.cache.gather_tokens(cache, indices)` on each
layer's K and V after selection (flash_evict/kv_distill_adapter.py:38-39,
streaming_adapter.py:86, quality_adapter.py:109-110). kv_distill is a local research
package the reference does not vendor; its contract follows from those call sites:
`cache` is [B, H, N, D] (often a transposed view), `indices` is [B, H, K] int64 (the
`select_tokens` output or an expanded `arange`), and the result is the contiguous
[B, H, K, D] tensor `cache.gather(2, indices[..., None].expand(..., D))`.

The copy runs in the library's gfx950 gather kernel (fe_gather_rows); CPU tensors are
not supported (the hot path has no CPU fallback).
"""
import torch

from . import _lib


def gather_tokens(cache, indices):
    """Return cache[b, h, indices[b, h, j], :] as a new contiguous [B, H, K, D] tensor.

    Indices outside [0, N) give zero rows (torch.gather would assert on the device).
    """
    if cache.ndim != 4 or indices.ndim != 3:
        raise ValueError("gather_tokens expects a [B, H, N, D] cache and [B, H, K] indices")
    b, h, n, d = cache.shape
    if tuple(indices.shape[:2]) != (b, h):
        raise ValueError("indices must share the cache's batch and head dimensions")
    if indices.dtype != torch.int64:
        raise ValueError("indices must be int64")
    if not cache.is_cuda or indices.device != cache.device:
        raise ValueError("gather_tokens needs CUDA (HIP) tensors on one device")
    if any(s < 0 for s in cache.stride()) or any(s < 0 for s in indices.stride()):
        raise ValueError("negative strides are not supported")
    k = indices.shape[2]
    out = torch.empty((b, h, k, d), dtype=cache.dtype, device=cache.device)
    if out.numel() == 0:
        return out
    L = _lib.lib()
    with torch.cuda.device(cache.device):
        stream = torch.cuda.current_stream(cache.device).cuda_stream
        rc = L.fe_gather_rows(cache.data_ptr(), indices.data_ptr(), out.data_ptr(), b, h, n, d, k,
                              _lib.strides(cache), _lib.strides(indices), cache.element_size(), stream)
    _lib.check(rc, "fe_gather_rows")
    return out
