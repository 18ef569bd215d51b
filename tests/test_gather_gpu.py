"""GPU KV compaction gather (fe_gather_rows) against the oracle: bit-exact byte copies on
the layouts the reference's adapters produce, plus edge cases (out-of-range indices, K=0,
K=N, odd row sizes, non-unit channel strides, 1- and 8-byte elements) and the headline
compaction at full size."""
import ctypes

import numpy as np
import pytest
import torch

from flash_evict import evict, gather_tokens
from flash_evict import _lib
from oracle import gather as og

from _helpers import transposed_qkv

pytestmark = pytest.mark.gpu


def _bits(t):
    """Integer view of the same bytes (numpy has no bfloat16; the comparison is bitwise)."""
    return {2: torch.int16, 4: torch.int32, 8: torch.int64}.get(t.element_size(), torch.uint8) \
        if t.is_floating_point() else t.dtype


def _check(x, idx):
    got = gather_tokens(x, idx)
    torch.cuda.synchronize()
    assert got.is_contiguous() and got.dtype == x.dtype
    assert got.shape == (x.shape[0], x.shape[1], idx.shape[2], x.shape[3])
    ref = og.gather_tokens(x.view(_bits(x)).cpu().numpy(), idx.cpu().numpy())
    assert np.array_equal(got.view(_bits(got)).cpu().numpy(), ref)


def _xview(b, h, n, d, dtype, layout, seed):
    g = torch.Generator().manual_seed(seed)
    if dtype in (torch.uint8, torch.int64):
        base = torch.randint(0, 250, (b, n, h, 2 * d), generator=g).to(dtype)
    else:
        base = torch.randn((b, n, h, 2 * d), generator=g).to(dtype)
    base = base.cuda()
    if layout == "contiguous":
        return base[..., :d].transpose(1, 2).contiguous()
    if layout == "transposed":          # the adapters' k/v: [B,N,H,D] viewed as [B,H,N,D]
        return base[..., :d].transpose(1, 2)
    if layout == "channel_stride2":
        return base[..., ::2].transpose(1, 2)
    raise AssertionError(layout)


CASES = [
    # b, h, n, d, k, dtype, layout
    (1, 8, 4096, 128, 409, torch.bfloat16, "transposed"),
    (2, 4, 1000, 64, 100, torch.float16, "contiguous"),
    (1, 2, 333, 40, 77, torch.bfloat16, "contiguous"),        # 80-byte rows: 16-byte chunks
    (1, 3, 257, 36, 50, torch.bfloat16, "transposed"),        # 72-byte rows: element kernel
    (2, 2, 129, 32, 129, torch.float32, "transposed"),        # K = N
    (1, 1, 64, 8, 1, torch.float16, "channel_stride2"),
    (1, 4, 500, 16, 31, torch.uint8, "contiguous"),
    (2, 3, 90, 12, 17, torch.int64, "transposed"),
]


@pytest.mark.parametrize("b,h,n,d,k,dtype,layout", CASES)
def test_random_indices(b, h, n, d, k, dtype, layout):
    print(f"gather b={b} h={h} n={n} d={d} k={k} {dtype} {layout}", flush=True)
    x = _xview(b, h, n, d, dtype, layout, n + d)
    g = torch.Generator().manual_seed(k)
    idx = torch.randint(0, n, (b, h, k), generator=g).cuda()
    _check(x, idx)


def test_uniform_recent_expanded_indices():
    """quality_adapter.py:41-43: arange(n-budget, n).expand(B, H, budget) (zero strides)."""
    x = _xview(1, 4, 2048, 128, torch.bfloat16, "transposed", 5)
    idx = torch.arange(2048 - 256, 2048, device="cuda").expand(1, 4, 256)
    assert idx.stride()[:2] == (0, 0)
    _check(x, idx)
    assert torch.equal(gather_tokens(x, idx), x[:, :, -256:])


def test_out_of_range_indices_give_zero_rows():
    x = _xview(1, 2, 50, 64, torch.bfloat16, "contiguous", 6)
    idx = torch.tensor([[[0, 49, -1, 50, 7], [1000, 3, -5, 2, 2]]], device="cuda")
    _check(x, idx)
    got = gather_tokens(x, idx)
    assert got[0, 0, 2].abs().sum() == 0 and got[0, 1, 0].abs().sum() == 0


def test_empty_selection():
    x = _xview(1, 2, 10, 64, torch.bfloat16, "contiguous", 7)
    got = gather_tokens(x, torch.zeros((1, 2, 0), dtype=torch.int64, device="cuda"))
    assert got.shape == (1, 2, 0, 64)


def test_c_abi_argument_errors():
    L = _lib.lib()
    st = (ctypes.c_int64 * 4)(1, 1, 1, 1)
    ist = (ctypes.c_int64 * 3)(1, 1, 1)
    assert L.fe_gather_rows(None, None, None, 1, 1, 4, 4, 2, st, ist, 3, None) == -1
    assert L.fe_gather_rows(None, None, None, 1, 1, 4, 4, 2, st, ist, 2, None) == -1   # null data
    assert L.fe_gather_rows(None, None, None, 1, 1, 4, 4, 0, st, ist, 2, None) == 0    # nothing to do


def test_headline_compaction_full_size():
    """Full-size compaction after evict() at the headline shape: K and V of 8 KV heads by
    the 1024 kept indices, bit-exact against the oracle; the kept rows are the rows the
    keep mask marks."""
    q, k, v = transposed_qkv(1, 32768, 32, 8, 128, torch.bfloat16, 20260910)
    _, _, idx, evicted = evict(q, k, v, 1024, reserved_recent=64, recency_decay=0.1)
    for x in (k, v):
        _check(x, idx)
    kk = gather_tokens(k, idx)
    keep = ~evicted
    ref = torch.stack([k[0, h][keep[0, h]] for h in range(8)])[None]
    assert torch.equal(kk, ref)
