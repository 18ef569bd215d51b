"""SnapKV observation-window score oracle (test infrastructure only).

Restates `snap_scores`, flash_evict/baselines.py:15-27 of anishesg/flash-evict-prefill:
  W = min(window, N); logits of the last W queries of every query head against all keys
  of its KV head, computed in the input dtype (the reference's native-dtype matmul);
  float(logits) * D^-0.5; causal mask key > query position; FP32 softmax; sum over the W
  rows; mean over the G query heads of a KV head.
The native-dtype product is modelled as the FP32 dot product of the input values rounded
once to the input dtype (what a GEMM with FP32 accumulation returns); the scale is the
FP32 value of D^-0.5, as torch applies a Python float to a float32 tensor.
Works on any torch device; tests run it on the CPU.
"""
import torch


def snap_scores(q, k, window=32):
    b, hq, n, d = q.shape
    hk = k.shape[1]
    g = hq // hk
    w = min(window, n)
    kr = k.float().repeat_interleave(g, 1)
    logits = torch.matmul(q[:, :, n - w:].float(), kr.transpose(-1, -2).contiguous())
    logits = logits.to(q.dtype).float() * torch.tensor(d ** -0.5, dtype=torch.float32)
    qpos = torch.arange(n - w, n, device=q.device)
    kpos = torch.arange(n, device=q.device)
    logits = logits.masked_fill(kpos[None, :] > qpos[:, None], float("-inf"))
    p = logits.softmax(-1)
    return p.sum(2).reshape(b, hk, g, n).mean(2)


def snap_scores_brute(q, k, window=32):
    """Float64 loops over the same definition (tiny inputs only)."""
    import math
    b, hq, n, d = q.shape
    hk = k.shape[1]
    g = hq // hk
    w = min(window, n)
    sc = float(torch.tensor(d ** -0.5, dtype=torch.float32))
    out = [[[0.0] * n for _ in range(hk)] for _ in range(b)]
    qf, kf = q.double(), k.double()
    for bi in range(b):
        for h in range(hq):
            j = h // g
            for t in range(n - w, n):
                row = []
                for key in range(t + 1):
                    dot = float(torch.tensor(float((qf[bi, h, t] * kf[bi, j, key]).sum()),
                                             dtype=torch.float32).to(q.dtype).float())
                    row.append(dot * sc)
                mx = max(row)
                e = [math.exp(x - mx) for x in row]
                s = sum(e)
                for key in range(t + 1):
                    out[bi][j][key] += e[key] / s / g
    return torch.tensor(out, dtype=torch.float64)
