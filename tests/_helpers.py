"""Shared helpers for the tests: seeded inputs and selection comparison."""
import torch


def seeded_randn(shape, dtype, seed, scale=1.0, device="cuda"):
    """N(0,1)*scale drawn on the CPU from a seeded generator, then moved to `device`.

    Drawing on the CPU makes the inputs bit-identical on every machine, so the CPU oracle
    and the GPU kernel see the same values.
    """
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g, dtype=torch.float32) * scale
    return x.to(dtype).to(device)


def transposed_qkv(b, n, hq, hk, d, dtype, seed, scale=1.0, device="cuda"):
    """q/k/v as transposed [B,N,H,D] -> [B,H,N,D] views (the adapters' layout)."""
    q = seeded_randn((b, n, hq, d), dtype, seed, scale, device).transpose(1, 2)
    k = seeded_randn((b, n, hk, d), dtype, seed + 1, scale, device).transpose(1, 2)
    v = seeded_randn((b, n, hk, d), dtype, seed + 2, 1.0, device).transpose(1, 2)
    return q, k, v


def assert_same_selection(keep, ref_keep, ref_scores, budget, recent=0, atol=0.0, rtol=0.0):
    """Kept sets must be identical, except for tokens whose reference scores lie within
    (atol + rtol*|s|) of the row's selection threshold (a near-tie the tolerance of the
    scores cannot order)."""
    keep = keep.cpu().reshape(-1, keep.shape[-1])
    ref_keep = ref_keep.cpu().reshape(-1, ref_keep.shape[-1])
    s = ref_scores.detach().float().cpu().reshape(-1, ref_scores.shape[-1])
    n = s.shape[-1]
    assert keep.shape == ref_keep.shape
    assert torch.equal(keep.sum(-1), ref_keep.sum(-1))
    for r in range(keep.shape[0]):
        diff = (keep[r] != ref_keep[r]).nonzero().flatten()
        if diff.numel() == 0:
            continue
        past = s[r, :n - recent]
        kk = budget - recent
        thr = past.topk(kk).values[-1]
        near = (past[diff] - thr).abs() <= atol + rtol * thr.abs()
        assert bool(near.all()), ("selection differs beyond near-ties", r, diff.tolist(),
                                  past[diff].tolist(), float(thr))
