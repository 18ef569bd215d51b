"""GPU tests of the attention kernel's reference max and its output normalisation.

The kernel keeps a row's reference max m at the exact max of the row's first keys (the first
64-key tile in the fused kernel, the first 32 keys in the split schedule's two-row-tile kernel
at head dims 72-128) and moves it only when a step's probabilities relative to m could overflow
(a lane's sum above 2^32 for bf16, 2^15 for fp16). It divides the output by the sum of the probabilities
exactly as rounded for the P@V product. The reference's kernel (flash_evict/prefill.py:37-60)
follows the running max exactly instead, so the key that dominates a row enters P@V as 1.0.
These tests plant such a key after the first tile, and at key 40 (inside the first 64-key
tile, after the first 32 keys):

  * a jump of ~2^20 (below the guard): the dominant key's probability is far from 1 and is
    rounded to bf16. With the rounded-sum normalisation the output of every dominated row
    equals that key's value row bit for bit; dividing by the unrounded sum instead would
    leave the probability's rounding error (up to 2^-8 relative) in the output, which
    changes some of these bf16 outputs by an ulp;
  * a jump of ~2^56 (above the guard): the tile takes a new exact max and is recomputed;
    the same bitwise property holds;
  * fp16, whose guard is 2^15, across both regimes: output and importance against the
    float64 oracle;
  * head dim 120 (the two-row-tile kernel below its tile dim, lanes past channel 120 reading
    zeros) with an observation window of 100 rows, so that the waves holding earlier rows take
    the tile loop without the FP32 sum, in bf16 and fp16 across both regimes;
  * values scaled by 2^60: every rounding in the kernel is relative, so the output and the
    importance scale by exactly 2^60 (the bound on |V| under which the accumulators stay
    finite is in fe_common.h).

Importance is checked element-wise against the oracle in every case.
"""
import math

import pytest
import torch

from flash_evict import prefill
from oracle.attention import chunked
from _helpers import assert_importance_close
from test_schedules_gpu import _run

pytestmark = pytest.mark.gpu

LOG2E = 1.4426950408889634


def _planted(n, hq, hk, d, dtype, kp, jump_log2, seed):
    """Queries along one direction u (a slightly different length per row); keys with small
    logits except key kp, whose logit is ~jump_log2 (log2 units) above them for every query;
    values of the planted key in [1, 8) in magnitude, so a dominated row's bf16/fp16 output
    is that row of V exactly."""
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(d, generator=g)
    u = u / u.norm() * math.sqrt(d)                              # |u|^2 = d
    rows = 1.0 + 0.05 * torch.arange(n, dtype=torch.float32) / n  # per-row length: varied rounding
    q = (u[None, None, :] * rows[None, :, None]).expand(hq, n, d).clone()
    k = 0.5 * torch.randn((hk, n, d), generator=g)
    beta = jump_log2 / (math.sqrt(d) * LOG2E)                   # logit(kp) = beta * sqrt(d) per unit row
    k[:, kp] = beta * u
    v = torch.randn((hk, n, d), generator=g)
    mag = 1.0 + 6.0 * torch.rand((hk, d), generator=g)
    sign = torch.where(torch.rand((hk, d), generator=g) < 0.5, -1.0, 1.0)
    v[:, kp] = sign * mag
    return (q[None].to(dtype).cuda(), k[None].to(dtype).cuda(), v[None].to(dtype).cuda())


@pytest.mark.parametrize("kp", [300, 40])
@pytest.mark.parametrize("jump_log2", [24.0, 60.0])
@pytest.mark.parametrize("use_ws", [True, False])
def test_dominant_key_after_first_tile_bf16(jump_log2, use_ws, kp):
    n, hq, hk, d = 1024, 2, 1, 128
    print("planted dominant key bf16: n=%d kp=%d jump 2^%g use_ws=%s" % (n, kp, jump_log2, use_ws), flush=True)
    q, k, v = _planted(n, hq, hk, d, torch.bfloat16, kp, jump_log2, seed=11)
    out, imp = _run(q, k, v, True, True, 0.0, 0, use_ws=use_ws)
    assert torch.isfinite(out).all() and torch.isfinite(imp).all()
    # every row that sees key kp returns its value row exactly
    dom = out[0, :, kp:, :]
    want = v[0, 0, kp][None, None, :].expand_as(dom)
    bad = (dom != want).sum().item()
    assert bad == 0, "%d of %d outputs of dominated rows differ from the dominant value" % (bad, dom.numel())
    ref_out, ref_imp = chunked(q, k, v, block=512, dtype=torch.float64)
    assert (out.float() - ref_out).abs().max().item() <= 2e-2
    assert_importance_close(imp, ref_imp, rtol=1e-3, floor=1e-30)


@pytest.mark.parametrize("d,kp", [(64, 700), (128, 700), (128, 40)])
@pytest.mark.parametrize("jump_log2", [10.0, 30.0])
def test_dominant_key_after_first_tile_fp16(jump_log2, d, kp):
    n, hq, hk = 1024, 4, 2
    print("planted dominant key fp16: n=%d d=%d kp=%d jump 2^%g" % (n, d, kp, jump_log2), flush=True)
    q, k, v = _planted(n, hq, hk, d, torch.float16, kp, jump_log2, seed=12)
    out, imp = prefill(q, k, v)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all() and torch.isfinite(imp).all()
    ref_out, ref_imp = chunked(q, k, v, block=512, dtype=torch.float64)
    assert (out.float() - ref_out).abs().max().item() <= 5e-3
    assert_importance_close(imp, ref_imp, rtol=1e-3, floor=1e-30)


@pytest.mark.parametrize("dtype,jump_log2", [(torch.bfloat16, 24.0), (torch.bfloat16, 60.0),
                                             (torch.float16, 10.0), (torch.float16, 30.0)])
def test_dominant_key_partial_head_dim_short_window(dtype, jump_log2):
    n, hq, hk, d, kp, window = 1024, 4, 2, 120, 300, 100
    print("planted dominant key %s: n=%d d=%d kp=%d jump 2^%g window %d" % (dtype, n, d, kp, jump_log2, window),
          flush=True)
    q, k, v = _planted(n, hq, hk, d, dtype, kp, jump_log2, seed=13)
    out, imp = prefill(q, k, v, observation_window=window)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all() and torch.isfinite(imp).all()
    ref_out, ref_imp = chunked(q, k, v, block=512, dtype=torch.float64, observation_window=window)
    bar = 2e-2 if dtype == torch.bfloat16 else 5e-3
    assert (out.float() - ref_out).abs().max().item() <= bar
    assert_importance_close(imp, ref_imp, rtol=1e-3, floor=1e-30)
    if dtype == torch.bfloat16:
        # every row that sees key kp returns its KV head's value row of kp exactly
        want = v[0, torch.arange(hq) // (hq // hk), kp]           # [hq, d]
        dom = out[0, :, kp:, :]
        assert bool((dom == want[:, None, :].expand_as(dom)).all())


@pytest.mark.parametrize("use_ws", [True, False])
def test_large_values_scale_exactly(use_ws):
    n, hq, hk, d, kp = 1024, 2, 1, 128, 300
    q, k, v = _planted(n, hq, hk, d, torch.bfloat16, kp, 24.0, seed=14)
    s = 2.0 ** 60
    out1, imp1 = _run(q, k, v, True, True, 0.0, 0, use_ws=use_ws)
    out2, imp2 = _run(q, k, v * s, True, True, 0.0, 0, use_ws=use_ws)
    assert torch.isfinite(out2).all() and torch.isfinite(imp2).all()
    assert torch.equal(out2, out1 * s)
    # the importance is the value-weighted mass: exactly 2^60 times, up to FP32 atomic order
    assert float((imp2 / s - imp1).abs().max()) <= 3e-6 * float(imp1.abs().max())
