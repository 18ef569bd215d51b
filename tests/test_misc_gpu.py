"""GPU checks beyond the reference tests: argument validation on device tensors, the generic
kernel's layouts and scales, golden fixtures, determinism, and resource introspection."""
import json
import os

import numpy as np
import pytest
import torch

import flash_evict
from flash_evict import _lib, prefill
from oracle.attention import materialized
from _helpers import seeded_randn

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _qkv(b=1, hq=4, hk=2, n=96, d=64, dtype=torch.bfloat16, seed=3):
    return (seeded_randn((b, hq, n, d), dtype, seed), seeded_randn((b, hk, n, d), dtype, seed + 1),
            seeded_randn((b, hk, n, d), dtype, seed + 2))


def test_argument_validation_on_device():
    # flash_evict/prefill.py:117-126 of the reference
    q, k, v = _qkv()
    for kw in (dict(recency_decay=-1.0), dict(recency_decay=float("inf")), dict(observation_window=-1),
               dict(observation_window=True), dict(observation_window=2.0), dict(block_q=48),
               dict(block_k=16), dict(scale=float("nan"))):
        with pytest.raises(ValueError):
            prefill(q, k, v, **kw)
    qg = q.clone().requires_grad_(True)
    with pytest.raises(ValueError, match="Inference only"):
        prefill(qg, k, v)
    with torch.no_grad():
        prefill(qg, k, v)
    with pytest.raises(ValueError, match="same device and dtype"):
        prefill(q, k.half(), v)
    with pytest.raises(ValueError, match="fp16 or bf16"):
        prefill(q.float(), k.float(), v.float())
    for bq in (16, 32, 64):
        for bk in (32, 64, 128):
            out, _ = prefill(q, k, v, block_q=bq, block_k=bk)   # accepted tile hints, same result
            assert torch.equal(out, prefill(q, k, v)[0])


@pytest.mark.parametrize("d", [16, 32, 80, 100, 136, 200, 256])
def test_head_dims_across_kernels(d):
    # multiples of 8 run the fast kernels (16, 136 and 200 below their tile dims, 80 on the
    # two-row-tile attention kernel); 100 takes the generic kernel
    print(f"head dim {d}", flush=True)
    q, k, v = _qkv(hq=4, hk=1, n=150, d=d, dtype=torch.float16, seed=d)
    out, imp = prefill(q, k, v, recency_decay=0.05)
    ref_out, ref_imp = materialized(q.cpu(), k.cpu(), v.cpu(), recency_decay=0.05)
    torch.testing.assert_close(out.float().cpu(), ref_out, atol=2e-3, rtol=6e-3)
    torch.testing.assert_close(imp.cpu(), ref_imp, atol=3e-5, rtol=4e-4)


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("scale", [-0.1, 0.0, 0.5, 3.0])
def test_scales(scale, d):
    # a negative scale runs on the fast kernels (|scale| on -Q), zero on the generic one
    q, k, v = _qkv(n=130, d=d, seed=11)
    for causal in (True, False):
        out, imp = prefill(q, k, v, scale=scale, causal=causal)
        ref_out, ref_imp = materialized(q.cpu(), k.cpu(), v.cpu(), scale=scale, causal=causal)
        torch.testing.assert_close(out.float().cpu(), ref_out, atol=1.2e-2, rtol=6e-3)
        torch.testing.assert_close(imp.cpu(), ref_imp, atol=3e-5, rtol=4e-4)


def test_unusual_layouts():
    # channel stride != 1 (D not innermost) and unaligned views take the generic loaders
    g = torch.Generator().manual_seed(4)
    base = torch.randn(1, 64, 70, 4, generator=g).to(torch.bfloat16).cuda()    # [B, D, N, H]
    q = base.permute(0, 3, 2, 1)                                                  # [B, H, N, D], d-stride 280
    kb = torch.randn(1, 2, 70, 65, generator=g).to(torch.bfloat16).cuda()
    k, v = kb[..., 1:], kb.flip(-1)[..., 1:]                                      # offset / negative-free views
    assert q.stride(-1) != 1 and k.data_ptr() % 16 != 0
    out, imp = prefill(q, k, v)
    ref_out, ref_imp = materialized(q.cpu(), k.cpu(), v.cpu())
    torch.testing.assert_close(out.float().cpu(), ref_out, atol=1.2e-2, rtol=6e-3)
    torch.testing.assert_close(imp.cpu(), ref_imp, atol=3e-5, rtol=4e-4)
    # broadcast K/V along tokens (stride 0) must not use the buffer-addressed fast path
    k0 = torch.randn(1, 2, 1, 64, generator=g).to(torch.bfloat16).cuda().expand(1, 2, 70, 64)
    assert k0.data_ptr() % 16 == 0 and k0.stride(2) == 0
    out, imp = prefill(q.contiguous(), k0, k0)
    ref_out, ref_imp = materialized(q.cpu(), k0.cpu(), k0.cpu())
    torch.testing.assert_close(out.float().cpu(), ref_out, atol=1.2e-2, rtol=6e-3)
    torch.testing.assert_close(imp.cpu(), ref_imp, atol=3e-5, rtol=4e-4)


def _misaligned(x):
    """The same values, 2 bytes off 16-byte alignment (contiguous otherwise)."""
    flat = torch.zeros(x.numel() + 1, dtype=x.dtype, device=x.device)
    flat[1:] = x.reshape(-1)
    return flat[1:].view(x.shape)


def _channel_strided(x):
    """The same values with channel stride 2."""
    wide = torch.zeros(x.shape[:-1] + (2 * x.shape[-1],), dtype=x.dtype, device=x.device)
    wide[..., ::2] = x
    return wide[..., ::2]


@pytest.mark.parametrize("d", [64, 128, 192])
def test_repacked_kv_equals_contiguous_call(d):
    """K/V the tile DMA cannot read in place (2 bytes off alignment; channel stride 2): prefill()
    sizes its workspace with fe_prefill_workspace_bytes_kv, the library copies K and V into it
    and runs the fast kernels, so the output equals the call on the contiguous tensors bit for
    bit and the importance equals it up to FP32 atomic order."""
    print("repacked K/V d=%d" % d, flush=True)
    q, k, v = _qkv(hq=4, hk=2, n=300, d=d, seed=31)
    for causal in (True, False):
        ref_out, ref_imp = prefill(q, k, v, causal=causal, recency_decay=0.02)
        for kk, vv in ((_misaligned(k), _channel_strided(v)), (_channel_strided(k), _misaligned(v))):
            assert kk.data_ptr() % 16 != 0 or kk.stride(-1) != 1
            out, imp = prefill(q, kk, vv, causal=causal, recency_decay=0.02)
            assert torch.equal(out, ref_out)
            assert float((imp - ref_imp).abs().max()) <= 2e-6 * float(ref_imp.abs().max())


@pytest.mark.parametrize("d", [100, 37])
def test_head_dims_not_multiple_of_8_on_the_fast_path(d):
    """A head dim that is not a multiple of 8: K and V are repacked to D rounded up to 8 channels
    (zeros past D), Q is read element-wise up to D and the output stores D channels (one by one
    when D is not a multiple of 4). Against the FP32 oracle, with and without a causal mask and
    through the workspace-free entry point (the generic kernel) as well."""
    print("head dim %d" % d, flush=True)
    q, k, v = _qkv(hq=4, hk=2, n=200, d=d, seed=33)
    for causal in (True, False):
        ref_out, ref_imp = materialized(q.cpu(), k.cpu(), v.cpu(), causal=causal, recency_decay=0.02)
        out, imp = prefill(q, k, v, causal=causal, recency_decay=0.02)
        torch.testing.assert_close(out.float().cpu(), ref_out, atol=1.2e-2, rtol=6e-3)
        torch.testing.assert_close(imp.cpu(), ref_imp, atol=3e-5, rtol=4e-4)
        assert torch.isfinite(out).all()
    # the generic kernel (no workspace: nowhere to repack)
    L = _lib.lib()
    out = torch.empty_like(q)
    imp = torch.empty((1, 2, 200), dtype=torch.float32, device=q.device)
    _lib.check(L.fe_prefill(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), imp.data_ptr(), 1, 4, 2, 200, d,
                            _lib.strides(q), _lib.strides(k), _lib.strides(v), 1, d ** -0.5, 1, 1, 1, 0.02, 200,
                            torch.cuda.current_stream().cuda_stream), "fe_prefill")
    torch.cuda.synchronize()
    ref_out, ref_imp = materialized(q.cpu(), k.cpu(), v.cpu(), causal=True, recency_decay=0.02)
    torch.testing.assert_close(out.float().cpu(), ref_out, atol=1.2e-2, rtol=6e-3)
    torch.testing.assert_close(imp.cpu(), ref_imp, atol=3e-5, rtol=4e-4)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_zero_scale_fast_and_generic(d):
    """scale = 0: the fast kernels run it with Q zeroed at load (every logit exactly 0: uniform
    attention over the visible keys), the workspace-free entry point with the generic kernel.
    Both against the FP32 oracle."""
    print("zero scale d=%d" % d, flush=True)
    q, k, v = _qkv(hq=4, hk=2, n=150, d=d, seed=35)
    ref_out, ref_imp = materialized(q.cpu(), k.cpu(), v.cpu(), scale=0.0)
    out, imp = prefill(q, k, v, scale=0.0)
    torch.testing.assert_close(out.float().cpu(), ref_out, atol=1.2e-2, rtol=6e-3)
    torch.testing.assert_close(imp.cpu(), ref_imp, atol=3e-5, rtol=4e-4)
    L = _lib.lib()
    out2 = torch.empty_like(q)
    imp2 = torch.empty((1, 2, 150), dtype=torch.float32, device=q.device)
    _lib.check(L.fe_prefill(q.data_ptr(), k.data_ptr(), v.data_ptr(), out2.data_ptr(), imp2.data_ptr(), 1, 4, 2, 150,
                            d, _lib.strides(q), _lib.strides(k), _lib.strides(v), 1, 0.0, 1, 1, 1, 0.0, 150,
                            torch.cuda.current_stream().cuda_stream), "fe_prefill")
    torch.cuda.synchronize()
    torch.testing.assert_close(out2.float().cpu(), ref_out, atol=1.2e-2, rtol=6e-3)
    torch.testing.assert_close(imp2.cpu(), ref_imp, atol=3e-5, rtol=4e-4)


@pytest.mark.parametrize("d", [64, 128])
def test_strided_q_on_the_fast_path(d):
    # Q with channel stride 2, or 2 bytes off 16-byte alignment, and aligned K/V: the fast
    # kernels read such a Q element-wise, so the result equals the contiguous call bit for bit
    q, k, v = _qkv(hq=4, hk=2, n=200, d=d, seed=21)
    wide = torch.zeros((1, 4, 200, 2 * d), dtype=q.dtype, device=q.device)
    wide[..., ::2] = q
    flat = torch.zeros(q.numel() + 1, dtype=q.dtype, device=q.device)
    flat[1:] = q.reshape(-1)
    for causal in (True, False):
        ref_out, ref_imp = prefill(q, k, v, causal=causal, recency_decay=0.02)
        for qq in (wide[..., ::2], flat[1:].view(q.shape)):
            assert qq.stride(-1) != 1 or qq.data_ptr() % 16 != 0
            out, imp = prefill(qq, k, v, causal=causal, recency_decay=0.02)
            assert torch.equal(out, ref_out)
            # same kernels; only the order of the FP32 atomic additions can differ
            assert float((imp - ref_imp).abs().max()) <= 2e-6 * float(ref_imp.abs().max())
        o_out, o_imp = materialized(q.cpu(), k.cpu(), v.cpu(), causal=causal, recency_decay=0.02)
        torch.testing.assert_close(ref_out.float().cpu(), o_out, atol=1.2e-2, rtol=6e-3)
        torch.testing.assert_close(ref_imp.cpu(), o_imp, atol=3e-5, rtol=4e-4)


def test_golden_fixtures():
    data = np.load(os.path.join(GOLDEN, "prefill_small.npz"), allow_pickle=False)
    for name in sorted({f.split(".")[0] for f in data.files}):
        meta = json.loads(str(data[f"{name}.meta"]))
        dt = getattr(torch, meta["dtype"])
        q, k, v = (torch.from_numpy(data[f"{name}.{t}"]).view(dt).cuda() for t in "qkv")
        out, imp = prefill(q, k, v, **meta["kwargs"])
        atol = 1.2e-2 if dt == torch.bfloat16 else 2e-3
        torch.testing.assert_close(out.float().cpu(), torch.from_numpy(data[f"{name}.out"]), atol=atol, rtol=6e-3)
        torch.testing.assert_close(imp.cpu(), torch.from_numpy(data[f"{name}.importance"]), atol=3e-5, rtol=4e-4)


@pytest.mark.parametrize("d,window", [(128, 0), (128, 200), (64, 77)])
def test_output_independent_of_scoring_and_deterministic(d, window):
    q, k, v = _qkv(b=2, hq=8, hk=2, n=1500, d=d, seed=d + window)
    out1, imp1 = prefill(q, k, v, recency_decay=0.1, observation_window=window)
    out2, imp2 = prefill(q, k, v, recency_decay=0.1, observation_window=window)
    plain, none = prefill(q, k, v, score=False)
    h2o = prefill(q, k, v, value_weighted=False)[0]
    assert none is None
    assert torch.equal(out1, out2) and torch.equal(out1, plain) and torch.equal(out1, h2o)
    torch.testing.assert_close(imp1, imp2, rtol=1e-6, atol=0)    # atomics may reorder FP32 sums


def test_kernel_resources():
    res = flash_evict.kernel_resources()
    names = {r["kernel"] for r in res}
    assert "fused_fast<bf16,128>" in names and {"select_lds", "select_sample", "avg_pool"} <= names
    # the selection kernels hold a whole row's keys (LDS schedule) or the sample and the
    # candidate pairs (sampled schedule) in static LDS, within the 160 KiB of a CU
    sel = {r["kernel"]: r for r in res if r["kernel"].startswith("select_")}
    assert 16384 * 4 <= sel["select_lds"]["lds_static_bytes"] <= 160 * 1024
    assert 4096 * 4 + 2 * 12288 * 4 <= sel["select_sample"]["lds_static_bytes"] <= 160 * 1024
    assert all(r["scratch_bytes_per_thread"] == 0 for r in sel.values())
    fast = [r for r in res if r["kernel"] == "fused_fast<bf16,128>"][0]
    # K/V double buffers of two 64-key tiles (8 x 64 rows x 256 B) plus the column-sum
    # exchange of the twelve waves, all static LDS; three waves per SIMD
    assert 0 < fast["registers_per_thread"] <= 168 and fast["lds_static_bytes"] == 8 * 64 * 256 + 2 * 12 * 64 * 4
    assert fast["max_threads_per_block"] >= 768
    # the attention-only kernel of the split schedule: 12 waves, three per SIMD
    attn = [r for r in res if r["kernel"] == "attn_fast<bf16,128>"][0]
    assert 0 < attn["registers_per_thread"] <= 168 and 8 * 64 * 256 <= attn["lds_static_bytes"] <= 8 * 64 * 256 + 64
    assert attn["max_threads_per_block"] >= 768
