"""flash_evict prefill API on MI355X: `prefill`, `select_tokens`, `evict`.

Signatures, defaults, return contracts and ValueError conditions are those of the
reference module flash_evict/prefill.py (anishesg/flash-evict-prefill):
  prefill        prefill.py:102-137
  _validate      prefill.py:86-99
  select_tokens  prefill.py:140-170
  evict          prefill.py:173-180
The compute runs in hand-written gfx950 HIP kernels reached through the C ABI of
libflash_evict_hip.so (see include/flash_evict.h); nothing here computes on the host
except `select_tokens` on CPU tensors, which runs the library's native host routine.
"""
import math

import torch

from . import _lib

_DTYPES = {torch.float16: _lib.FE_DTYPE_F16, torch.bfloat16: _lib.FE_DTYPE_BF16}


def _validate(q, k, v):
    """Reject inputs the kernel does not define (reference prefill.py:86-99)."""
    if any(t.ndim != 4 for t in (q, k, v)):
        raise ValueError("Q/K/V must have shape [batch, heads, tokens, channels]")
    b, h, n, d = q.shape
    if (min(b, h, n, d, k.shape[1]) < 1 or k.shape != v.shape or k.shape[0] != b
            or tuple(k.shape[2:]) != (n, d)):
        raise ValueError("Expected nonempty self-attention Q/K/V with equal sequence and channel dimensions")
    if h % k.shape[1] or d > 256:
        raise ValueError("Query heads must be divisible by KV heads; head dimension must be <= 256")
    if any(t.device != q.device or t.dtype != q.dtype for t in (k, v)):
        raise ValueError("Q/K/V must have the same device and dtype")
    if not q.is_cuda or q.dtype not in _DTYPES:
        raise ValueError("CUDA fp16 or bf16 inputs required")
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        raise ValueError("Inference only: no backward implementation")


def _is_int(x):
    return isinstance(x, int) and not isinstance(x, bool)


def prefill(q, k, v, *, causal=True, value_weighted=True, score=True,
            scale=None, block_q=32, block_k=64, recency_decay=0., observation_window=0):
    """Return (attention output, FP32 importance [B, Hkv, N]).

    Importance sums over queries and the query heads sharing a KV head:
      I[b,h,k] = ||V[b,h,k]||_1 * sum_(g,q) w[q] softmax(Q K^T)[b,h,g,q,k],
    w[q] = exp(recency_decay * (q - (N-1))) restricted to the last observation_window
    queries (0 means all). The attention output does not depend on the scoring options
    (bitwise). With value_weighted=False the importance is H2O attention mass; with
    score=False importance is None. FP32 atomic reduction order can cause run-to-run
    differences of a few ulps. block_q/block_k are validated as in the reference but
    the gfx950 kernel uses its own tiling (32-query row tiles, 64-key KV tiles).
    """
    _validate(q, k, v)
    recency_decay = float(recency_decay)
    if not math.isfinite(recency_decay) or recency_decay < 0:
        raise ValueError("recency_decay must be finite and nonnegative")
    if not _is_int(observation_window) or observation_window < 0:
        raise ValueError("observation_window must be a nonnegative integer; 0 means all queries")
    if block_q not in (16, 32, 64) or block_k not in (32, 64, 128):
        raise ValueError("Unsupported tile dimensions")
    scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
    if not math.isfinite(scale):
        raise ValueError("scale must be finite")
    b, h, n, d = q.shape
    hk = k.shape[1]
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    importance = torch.empty((b, hk, n), dtype=torch.float32, device=q.device) if score else None
    window = min(n, observation_window or n)
    L = _lib.lib()
    with torch.cuda.device(q.device):
        stream = torch.cuda.current_stream(q.device).cuda_stream
        # workspace: replay biases (one float per query row), the work-item counters, and
        # room to repack K/V the fast kernels cannot read in place
        ws_bytes = L.fe_prefill_workspace_bytes_kv(b, h, hk, n, d, int(bool(score)), k.data_ptr(), _lib.strides(k),
                                                   v.data_ptr(), _lib.strides(v))
        ws = torch.empty(ws_bytes // 4, dtype=torch.float32, device=q.device) if ws_bytes else None
        rc = L.fe_prefill_ws(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                             importance.data_ptr() if score else None,
                             b, h, hk, n, d, _lib.strides(q), _lib.strides(k), _lib.strides(v),
                             _DTYPES[q.dtype], scale, int(bool(causal)), int(bool(value_weighted)),
                             int(bool(score)), recency_decay, window,
                             ws.data_ptr() if ws is not None else None, ws_bytes, stream)
    _lib.check(rc, "fe_prefill_ws")
    return out, importance


def _select(importance, budget, recent, pool_kernel, invert):
    n = importance.shape[-1]
    lead = tuple(importance.shape[:-1])
    rows = math.prod(lead)
    x = importance.reshape(rows, n) if rows else importance.reshape(0, n)
    if x.dtype != torch.float32:
        x = x.float()
    if x.stride(-1) != 1 or (rows > 1 and x.stride(0) < n):
        x = x.contiguous()
    row_stride = x.stride(0) if rows > 1 else n
    indices = torch.empty((rows, budget), dtype=torch.int64, device=importance.device)
    mask = torch.empty((rows, n), dtype=torch.bool, device=importance.device)
    L = _lib.lib()
    if rows:
        if x.is_cuda:
            ws_bytes = L.fe_select_workspace_bytes(rows, n, budget, recent, pool_kernel)
            with torch.cuda.device(x.device):
                ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
                stream = torch.cuda.current_stream(x.device).cuda_stream
                rc = L.fe_select(x.data_ptr(), rows, n, row_stride, budget, recent, pool_kernel,
                                 indices.data_ptr(), mask.data_ptr(), int(invert),
                                 ws.data_ptr(), ws_bytes, stream)
            _lib.check(rc, "fe_select")
        elif x.device.type == "cpu":
            rc = L.fe_select_host(x.data_ptr(), rows, n, row_stride, budget, recent, pool_kernel,
                                  indices.data_ptr(), mask.data_ptr(), int(invert))
            _lib.check(rc, "fe_select_host")
        else:
            raise ValueError("select_tokens supports CUDA (HIP) and CPU tensors")
    return indices.reshape(*lead, budget), mask.reshape(*lead, n)


def _check_selection(n, budget, recent, reserved_recent, pool_kernel):
    """Argument rules of the reference select_tokens (prefill.py:150-159)."""
    if reserved_recent is not None:
        if recent != 0 and recent != reserved_recent:
            raise ValueError("recent and reserved_recent disagree")
        recent = reserved_recent
    if not _is_int(budget) or not 1 <= budget <= n:
        raise ValueError("budget must be an integer in [1, sequence length]")
    if not _is_int(recent) or not 0 <= recent <= budget:
        raise ValueError("recent must be an integer in [0, budget]")
    if not _is_int(pool_kernel) or pool_kernel < 1 or pool_kernel % 2 != 1:
        raise ValueError("pool_kernel must be a positive odd integer")
    return recent


def select_tokens(importance, budget, *, recent=0, reserved_recent=None, pool_kernel=1):
    """Return chronologically sorted kept indices (int64) and a bool KEEP mask.

    recent (alias reserved_recent) reserves the last `recent` tokens inside the total
    budget; the other budget-recent tokens are the top scores of the earlier tokens,
    optionally smoothed by SnapKV average pooling (pool_kernel > 1, zero padding counted).
    Ties keep the lower index (the reference leaves tie order unspecified).
    """
    n = importance.shape[-1]
    recent = _check_selection(n, budget, recent, reserved_recent, pool_kernel)
    return _select(importance, budget, recent, pool_kernel, invert=False)


def evict(q, k, v, budget, *, recent=0, reserved_recent=None, pool_kernel=1, **kwargs):
    """Return output, importance, kept indices, and bool eviction mask (True=evict)."""
    if kwargs.get("score") is False:
        raise ValueError("evict requires importance scoring")
    output, importance = prefill(q, k, v, **kwargs)
    n = importance.shape[-1]
    recent = _check_selection(n, budget, recent, reserved_recent, pool_kernel)
    indices, evicted = _select(importance, budget, recent, pool_kernel, invert=True)
    return output, importance, indices, evicted
