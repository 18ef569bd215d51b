"""Pure-Python loop restatements for tiny inputs (test infrastructure only).

Independent of torch/numpy vectorisation: used to pin oracle.attention and
oracle.select against the definitions of flash_evict/reference.py:5-25 and
flash_evict/prefill.py:140-170 (anishesg/flash-evict-prefill), computed in float64.
Inputs are nested Python lists; sizes must stay tiny (N <= ~24).
"""
import math


def attention(q, k, v, *, causal=True, value_weighted=True, scale=None,
              recency_decay=0.0, observation_window=0):
    """q: [B][Hq][N][D], k/v: [B][Hkv][N][D] lists of floats. Returns (out, mass)."""
    B, Hq, N, D = len(q), len(q[0]), len(q[0][0]), len(q[0][0][0])
    Hk = len(k[0])
    G = Hq // Hk
    sc = D ** -0.5 if scale is None else scale
    W = min(N, observation_window or N)
    out = [[[[0.0] * D for _ in range(N)] for _ in range(Hq)] for _ in range(B)]
    mass = [[[0.0] * N for _ in range(Hk)] for _ in range(B)]
    for b in range(B):
        for h in range(Hq):
            j = h // G
            for i in range(N):
                keys = range(i + 1) if causal else range(N)
                logit = {t: sc * sum(q[b][h][i][c] * k[b][j][t][c] for c in range(D)) for t in keys}
                mx = max(logit.values())
                e = {t: math.exp(x - mx) for t, x in logit.items()}
                z = sum(e.values())
                for c in range(D):
                    out[b][h][i][c] = sum(e[t] / z * v[b][j][t][c] for t in keys)
                w = math.exp(recency_decay * (i - (N - 1))) if i >= N - W else 0.0
                for t in keys:
                    mass[b][j][t] += w * e[t] / z
    if value_weighted:
        for b in range(B):
            for j in range(Hk):
                for t in range(N):
                    mass[b][j][t] *= sum(abs(x) for x in v[b][j][t])
    return out, mass


def select_row(scores, budget, recent=0, pool_kernel=1):
    """One row of select_tokens by explicit loops; ties keep the lower index."""
    n = len(scores)
    m = n - recent
    past = [float(x) for x in scores[:m]]
    if pool_kernel > 1 and budget > recent:
        half = pool_kernel // 2
        past = [sum(past[j] for j in range(i - half, i + half + 1) if 0 <= j < m) / pool_kernel
                for i in range(m)]
    chosen = []
    remaining = list(range(m))
    for _ in range(budget - recent):
        best = remaining[0]
        for i in remaining[1:]:
            if past[i] > past[best]:
                best = i
        chosen.append(best)
        remaining.remove(best)
    idx = sorted(chosen + list(range(m, n)))
    keep = [i in set(idx) for i in range(n)]
    return idx, keep
