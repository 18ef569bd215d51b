"""Closed forms of the prefill path for Q = K = 0 (test infrastructure only).

With all logits equal and causal masking, softmax(QK^T)[q, k] = 1/(q+1) for k <= q, so
(anishesg/flash-evict-prefill tests/test_prefill.py:87-102,134-146):
  out[q]      = mean(v[0..q])                                  (running value mean)
  mass[k]     = G * sum_{q >= k} w_q / (q+1)                   (reverse harmonic sum)
  importance  = mass * ||v_k||_1 when value weighted
Computed in float64 from the given value rows.
"""
import torch


def zero_qk_output(v):
    """v: [B, Hkv, N, D] -> running mean over tokens, float64 [B, Hkv, N, D]."""
    n = v.shape[2]
    pos = torch.arange(1, n + 1, dtype=torch.float64, device=v.device)
    return v.double().cumsum(2) / pos[None, None, :, None]


def zero_qk_mass(n, groups, recency_decay=0.0, observation_window=0, device="cpu"):
    """Unweighted importance per key, float64 [N]."""
    pos = torch.arange(n, dtype=torch.float64, device=device)
    w = (recency_decay * (pos - (n - 1))).exp()
    if observation_window:
        w = w * (pos >= n - observation_window)
    return (w / (pos + 1)).flip(0).cumsum(0).flip(0) * groups
