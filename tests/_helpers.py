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


def assert_importance_close(imp, ref, rtol=1e-3, floor=1e-30):
    """Element-wise importance bound: |imp - ref| <= rtol * |ref| + floor for every key.

    Unlike a bound normalised by the row maximum, this binds on every key, including the
    many whose importance lies orders of magnitude below the largest. Returns the largest
    relative error over the elements above the floor (for the log)."""
    imp = imp.detach().double()
    ref = ref.detach().to(imp.device).double()
    assert imp.shape == ref.shape, (imp.shape, ref.shape)
    err = (imp - ref).abs()
    bound = rtol * ref.abs() + floor
    bad = err > bound
    big = ref.abs() > floor
    worst = float((err[big] / ref.abs()[big]).max()) if bool(big.any()) else 0.0
    print("importance: max element-wise rel err %.3e over %d of %d elements above the floor %g"
          % (worst, int(big.sum()), big.numel(), floor), flush=True)
    if bool(bad.any()):
        i = int(bad.flatten().nonzero()[0])
        raise AssertionError("importance differs beyond %g*|ref| + %g at %d of %d elements; first at flat index %d: "
                             "kernel %r, oracle %r" % (rtol, floor, int(bad.sum()), bad.numel(), i,
                                                       float(imp.flatten()[i]), float(ref.flatten()[i])))
    return worst


def split_runs_two_row_tiles(d):
    """Whether the split schedule (fe_prefill_ws) may run the two-row-tile attention kernel at
    head dim d in the default build: tile dims 96 and 128 (d a multiple of 8 in 72..128), for
    launches of more than 1.5 rounds of its work items (smaller ones run the one-row-tile
    small-grid kernel). Where it does, its reference max comes from a row's first 32 keys, the
    fused kernel's from 64, so callers compare the schedules within a bound instead of bitwise."""
    return d % 8 == 0 and 72 <= d <= 128


def assert_schedules_agree(o_split, o_fused, i_split, i_fused, v, hq, hk):
    """Outputs and importance of the split and fused schedules on the same inputs.

    Same attention kernel (bitwise-equal outputs): the importance differs only by the order of
    FP32 atomic additions. Different attention kernels: the probabilities P = exp2(s*scale - m)
    are rounded to the input dtype at other reference maxima m, so with rounding errors e1_k,
    e2_k (|e| <= u, the unit roundoff: 2^-8 for bf16, 2^-11 for fp16) and d_k = e1_k - e2_k the outputs differ to
    first order by sum_k w_k d_k (v_k - o), at most 2u (max_k |v_k| + |o|), plus one rounding
    of each stored output: |o_split - o_fused| <= 2u max|v| + 4u |o| per query head. The replay
    bias m + log2 l is then the same quantity summed in another order, so the importance agrees
    to FP32 summation error (1e-4 element-wise, plus the atomic-order floor)."""
    floor = 3e-6 * float(i_fused.abs().max())
    if torch.equal(o_split, o_fused):
        assert float((i_split - i_fused).abs().max()) <= floor
        return
    u = 2.0 ** -8 if o_split.dtype == torch.bfloat16 else 2.0 ** -11
    vmax = v.float().abs().amax(dim=(2, 3)).repeat_interleave(hq // hk, dim=1)[:, :, None, None]
    diff = (o_split.float() - o_fused.float()).abs()
    bound = 2 * u * vmax + 4 * u * o_fused.float().abs()
    print("schedules: max |o_split - o_fused| = %.3e, max rel importance diff = %.3e"
          % (diff.max().item(), ((i_split - i_fused).abs() / (i_fused.abs() + 1e-30)).max().item()), flush=True)
    assert bool((diff <= bound).all()), float((diff - bound).max())
    assert bool(((i_split - i_fused).abs() <= 1e-4 * i_fused.abs() + floor).all())


def out_err_all_rows(out, q, k, v, block=2048, **kw):
    """Max-abs error of the attention output against the FP32 oracle over every row of every
    query head, computed one head at a time (oracle.attention.chunked on out's device)."""
    from oracle.attention import chunked
    b, hq = out.shape[:2]
    worst = 0.0
    for bi in range(b):
        for h in range(hq):
            ref_out, _ = chunked(q, k, v, heads=[(bi, h)], block=block, value_weighted=False, **kw)
            worst = max(worst, float((out[bi, h].float() - ref_out[bi, h]).abs().max()))
            del ref_out
    return worst
