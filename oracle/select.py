"""Token-selection oracle in numpy (test infrastructure only).

Restates select_tokens, flash_evict/prefill.py:140-170, and snap_select,
flash_evict/baselines.py:28-40 (anishesg/flash-evict-prefill). The reference's ties
follow torch.topk (unspecified, prefill.py:144); this restatement fixes them the way the
build does: among equal scores the lower index wins; -0.0 equals +0.0; NaN ranks above
every number.
"""
import numpy as np


def avg_pool(x, kernel):
    """avg_pool1d(x, kernel, stride=1, padding=kernel//2), count_include_pad=True.

    Each output is the left-to-right float32 sum of the window (zeros outside the row)
    divided by `kernel`, the order torch's avg_pool kernels use.
    """
    x = np.asarray(x, dtype=np.float32)
    m = x.shape[-1]
    pad = kernel // 2
    xp = np.zeros(x.shape[:-1] + (m + 2 * pad,), dtype=np.float32)
    xp[..., pad:pad + m] = x
    acc = np.zeros(x.shape, dtype=np.float32)
    for j in range(kernel):
        acc = (acc + xp[..., j:j + m]).astype(np.float32)
    return (acc / np.float32(kernel)).astype(np.float32)


def topk_lowest_index(row, k):
    """Indices of the k largest entries of a 1-D array; ties keep the lower index."""
    row = np.asarray(row)
    idx = np.arange(row.shape[0])
    nan = np.isnan(row)
    val = np.where(nan, 0.0, row).astype(np.float64)
    # lexsort: last key is primary. NaN first, then value descending, then index ascending.
    order = np.lexsort((idx, -val, ~nan))
    return order[:k]


def _is_int(x):
    return isinstance(x, (int, np.integer)) and not isinstance(x, (bool, np.bool_))


def select_tokens(importance, budget, *, recent=0, reserved_recent=None, pool_kernel=1):
    """Return (indices int64 [..., budget] ascending, keep bool [..., n])."""
    scores = np.asarray(importance, dtype=np.float32)
    n = scores.shape[-1]
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
    lead = scores.shape[:-1]
    flat = scores.reshape(-1, n)
    past = flat[:, :n - recent]
    if pool_kernel > 1 and budget > recent:
        past = avg_pool(past, pool_kernel)
    idx = np.empty((flat.shape[0], budget), dtype=np.int64)
    keep = np.zeros(flat.shape, dtype=bool)
    for r in range(flat.shape[0]):
        top = topk_lowest_index(past[r], budget - recent)
        sel = np.sort(np.concatenate([top, np.arange(n - recent, n)]).astype(np.int64))
        idx[r] = sel
        keep[r, sel] = True
    return idx.reshape(lead + (budget,)), keep.reshape(lead + (n,))


def snap_select(scores, budget, window=32, kernel=5):
    """SnapKV selection of flash_evict/baselines.py:28-40 (pooled top-k + pinned window)."""
    scores = np.asarray(scores, dtype=np.float32)
    n = scores.shape[-1]
    lead = scores.shape[:-1]
    flat = scores.reshape(-1, n)
    if n <= budget:
        idx = np.broadcast_to(np.arange(n, dtype=np.int64), flat.shape[:-1] + (n,)).copy()
    else:
        window = min(window, n, budget - 1)
        pooled = avg_pool(flat[:, :n - window], kernel)
        idx = np.empty((flat.shape[0], budget), dtype=np.int64)
        for r in range(flat.shape[0]):
            top = topk_lowest_index(pooled[r], budget - window)
            idx[r] = np.sort(np.concatenate([top, np.arange(n - window, n)]))
    keep = np.zeros(flat.shape, dtype=bool)
    for r in range(flat.shape[0]):
        keep[r, idx[r]] = True
    return idx.reshape(lead + (idx.shape[-1],)), keep.reshape(lead + (n,))
