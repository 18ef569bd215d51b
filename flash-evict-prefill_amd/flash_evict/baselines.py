"""SnapKV baseline path on MI355X (reference flash_evict/baselines.py:1-47).

`flash_attention` is the comparison attention the reference pairs with SnapKV: torch's
fused scaled-dot-product attention (its flash kernel on ROCm), causal with grouped KV
heads. `snap_scores` runs the library's gfx950 kernels (fe_snap_scores) and `snap_select`
the library's pool + radix top-k kernels (fe_select): SnapKV selection is select_tokens
with the observation window as the reserved suffix (reference tests/test_prefill.py:149-155).
"""
import math

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from . import _lib
from .prefill import _DTYPES, _select


def flash_attention(q, k, v):
    """Causal GQA attention through torch's flash SDPA kernel alone (baselines.py:7-9).

    Only SDPBackend.FLASH_ATTENTION is admitted, as in the reference, so the comparison
    kernel is pinned: a shape that backend rejects raises torch's error instead of running
    on another backend.
    """
    with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
        return F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)


def snap_scores(q, k, window=32):
    """SnapKV scores [B, Hkv, N] (FP32) of the last `window` queries (baselines.py:15-27).

    Logits are the native-dtype products q.k (FP32 accumulation rounded to the input
    dtype) times D^-0.5; softmax in FP32 with the causal mask; summed over the window
    queries and averaged over the query heads of each KV head.
    """
    if q.ndim != 4 or k.ndim != 4 or q.shape[0] != k.shape[0] or tuple(q.shape[2:]) != tuple(k.shape[2:]):
        raise ValueError("snap_scores expects q [B, Hq, N, D] and k [B, Hkv, N, D]")
    b, hq, n, d = q.shape
    hk = k.shape[1]
    if min(b, hq, hk, n, d) < 1 or hq % hk or d > 256:
        raise ValueError("Query heads must be divisible by KV heads; head dimension must be <= 256")
    if k.dtype != q.dtype or k.device != q.device or not q.is_cuda or q.dtype not in _DTYPES:
        raise ValueError("CUDA fp16 or bf16 inputs required")
    if isinstance(window, bool) or not isinstance(window, int) or window < 1:
        raise ValueError("window must be a positive integer")
    scores = torch.empty((b, hk, n), dtype=torch.float32, device=q.device)
    L = _lib.lib()
    ws_bytes = L.fe_snap_scores_workspace_bytes(b, hq, hk, n, window)
    with torch.cuda.device(q.device):
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
        stream = torch.cuda.current_stream(q.device).cuda_stream
        rc = L.fe_snap_scores(q.data_ptr(), k.data_ptr(), scores.data_ptr(), b, hq, hk, n, d,
                              _lib.strides(q), _lib.strides(k), _DTYPES[q.dtype], window,
                              ws.data_ptr(), ws_bytes, stream)
    _lib.check(rc, "fe_snap_scores")
    return scores


def snap_select(scores, budget, window=32, kernel=5):
    """Kept indices (ascending int64) and keep mask of SnapKV (baselines.py:30-40).

    n <= budget keeps everything; otherwise the last min(window, n, budget-1) tokens are
    pinned and the rest of the budget is the top of the kernel-pooled earlier scores.
    Ties keep the lower index.
    """
    n = scores.shape[-1]
    if n <= budget:
        idx = torch.arange(n, device=scores.device).expand(*scores.shape[:-1], n)
        return idx, torch.ones(scores.shape, dtype=torch.bool, device=scores.device)
    if not isinstance(kernel, int) or kernel < 1 or kernel % 2 != 1:
        raise ValueError("kernel must be a positive odd integer")
    if not isinstance(budget, int) or budget < 1:
        raise ValueError("budget must be a positive integer")
    recent = min(window, n, budget - 1)
    pool = kernel if budget > recent else 1
    return _select(scores, budget, recent, pool, invert=False)


def flash_snap(q, k, v, budget, window=32):
    """Attention output, SnapKV scores, kept indices and eviction mask (baselines.py:43-47)."""
    out = flash_attention(q, k, v)
    scores = snap_scores(q, k, window)
    idx, keep = snap_select(scores, budget, window)
    return out, scores, idx, ~keep
