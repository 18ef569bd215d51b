"""FP32 attention + replay-importance oracle (test infrastructure only).

Restates flash_evict/reference.py:5-25 of anishesg/flash-evict-prefill:
  out[b,h,q]  = softmax_k(scale * q.k, causal) @ v           (GQA: kv head = h // G)
  mass[b,j,k] = sum_{h in group j} sum_q w_q softmax(...)[b,h,q,k]
  w_q         = exp(decay*(q-(N-1))) * [q >= N - window]       (window 0 = all queries)
  mass       *= ||v[b,j,k]||_1 when value_weighted
Everything is computed in float32 from the (bf16/fp16) input values, as the reference
oracle does with `.float()`. Works on any torch device; tests run it on the CPU.
"""
import torch


def _weights(n, recency_decay, observation_window, device):
    pos = torch.arange(n, device=device)
    w = (recency_decay * (pos.float() - (n - 1))).exp()
    if observation_window:
        w = w * (pos >= n - observation_window)
    return w


def materialized(q, k, v, *, causal=True, value_weighted=True, scale=None,
                 recency_decay=0., observation_window=0):
    """Dense FP32 ground truth (reference.py:5-25). O(N^2) memory: small N only."""
    b, hq, n, d = q.shape
    hk = k.shape[1]
    g = hq // hk
    kr = k.float().repeat_interleave(g, 1)
    vr = v.float().repeat_interleave(g, 1)
    logits = torch.matmul(q.float(), kr.transpose(-1, -2).contiguous())
    logits = logits * (d ** -0.5 if scale is None else scale)
    if causal:
        pos = torch.arange(n, device=q.device)
        logits = logits.masked_fill(pos[None, :] > pos[:, None], float("-inf"))
    p = logits.softmax(-1)
    out = torch.matmul(p, vr)
    w = _weights(n, recency_decay, observation_window, q.device)
    mass = (p * w[:, None]).sum(-2).reshape(b, hk, g, n).sum(2)
    if value_weighted:
        mass = mass * v.float().abs().sum(-1)
    return out, mass


def chunked(q, k, v, *, causal=True, value_weighted=True, scale=None,
            recency_decay=0., observation_window=0, block=1024, heads=None, want_out=True,
            query_rows=None, dtype=torch.float32):
    """Exact FP32 oracle streamed over (head, query block); never forms the N x N matrix.

    `heads` optionally restricts the computation to a list of (b, query head) pairs (the
    importance then only holds their contributions). `query_rows`, a list of (q0, q1)
    ranges, restricts the output rows computed (only those rows of `out` are filled; the
    importance is then only meaningful when every weighted row is included).
    `dtype=torch.float64` evaluates the same formulas in double precision (the recency
    weights stay the FP32 values the reference uses): a truth the FP32 rounding of the
    logits does not blur, for inputs whose logits are so large that any FP32 evaluation,
    the reference's included, is uncertain in the last bits.
    Returns (out or None, mass).
    """
    b, hq, n, d = q.shape
    hk = k.shape[1]
    g = hq // hk
    sc = d ** -0.5 if scale is None else scale
    w = _weights(n, recency_decay, observation_window, q.device).to(dtype)
    win_lo = n - min(n, observation_window or n)
    out = torch.zeros((b, hq, n, d), dtype=dtype, device=q.device) if want_out else None
    mass = torch.zeros((b, hk, n), dtype=dtype, device=q.device)
    pairs = heads if heads is not None else [(bi, hi) for bi in range(b) for hi in range(hq)]
    for bi, hi in pairs:
        j = hi // g
        kf = k[bi, j].to(dtype)
        vf = v[bi, j].to(dtype)
        col = torch.zeros(n, dtype=dtype, device=q.device)
        if query_rows is None:
            spans = [(q0, min(n, q0 + block)) for q0 in range(0, n, block)]
        else:
            spans = [(a, min(hi_, a + block)) for lo_, hi_ in query_rows for a in range(lo_, hi_, block)]
        for q0, q1 in spans:
            if not want_out and q1 <= win_lo:
                continue
            kend = q1 if causal else n
            qf = q[bi, hi, q0:q1].to(dtype)
            logits = torch.matmul(qf, kf[:kend].t().contiguous()) * sc
            if causal:
                rows = torch.arange(q0, q1, device=q.device)
                keys = torch.arange(kend, device=q.device)
                logits = logits.masked_fill(keys[None, :] > rows[:, None], float("-inf"))
            p = logits.softmax(-1)
            if want_out:
                out[bi, hi, q0:q1] = torch.matmul(p, vf[:kend])
            if q1 > win_lo:
                col[:kend] += (p * w[q0:q1, None]).sum(0)
        mass[bi, j] += col
    if value_weighted:
        mass = mass * v.to(dtype).abs().sum(-1)
    return out, mass
