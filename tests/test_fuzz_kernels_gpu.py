"""Seeded randomized sweeps of the KV compaction gather and the SnapKV scores against their
oracles (oracle/gather.py, oracle/snap.py): random shapes, element sizes, layouts, index sets
(sorted, unsorted, repeated) and observation windows. The gather must be bit-exact; the
scores meet the tolerance stated in tests/test_snap_gpu.py."""
import random

import numpy as np
import pytest
import torch

from flash_evict import gather_tokens
from flash_evict.baselines import snap_scores
from oracle import gather as og
from oracle import snap as osnap

from test_gather_gpu import _bits, _xview
from test_snap_gpu import _check_scores, _qk

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed", range(24))
def test_random_gather(seed):
    r = random.Random(seed)
    b, h, n = r.choice([1, 2]), r.choice([1, 2, 3, 8]), r.choice([1, 7, 64, 65, 300, 1025])
    d = r.choice([4, 8, 12, 16, 40, 64, 128, 256])
    dtype = r.choice([torch.bfloat16, torch.float16, torch.float32, torch.uint8, torch.int64])
    layout = r.choice(["contiguous", "transposed", "channel_stride2"])
    k = r.randint(0, n)
    kind = r.choice(["sorted", "unsorted", "repeated"])
    print("gather seed=%d b=%d h=%d n=%d d=%d k=%d %s %s %s" % (seed, b, h, n, d, k, dtype, layout, kind), flush=True)
    x = _xview(b, h, n, d, dtype, layout, 77 + seed)
    g = torch.Generator().manual_seed(seed)
    if kind == "repeated":
        idx = torch.randint(0, n, (b, h, k), generator=g)
    else:
        idx = torch.stack([torch.stack([torch.randperm(n, generator=g)[:k] for _ in range(h)]) for _ in range(b)])
        if kind == "sorted":
            idx = idx.sort(-1).values
    idx = idx.cuda()
    got = gather_tokens(x, idx)
    torch.cuda.synchronize()
    assert got.shape == (b, h, k, d) and got.is_contiguous()
    ref = og.gather_tokens(x.view(_bits(x)).cpu().numpy(), idx.cpu().numpy())
    assert np.array_equal(got.view(_bits(got)).cpu().numpy(), ref)


@pytest.mark.parametrize("seed", range(16))
def test_random_snap_scores(seed):
    r = random.Random(1000 + seed)
    hk, g = r.choice([1, 2, 4]), r.choice([1, 2, 4, 7])
    n = r.choice([1, 33, 64, 200, 513, 1500])
    d = r.choice([16, 32, 64, 80, 128, 256])
    w = r.choice([1, 8, 32, 64, 128, n + 3])
    dtype = r.choice([torch.bfloat16, torch.float16])
    layout = r.choice(["contiguous", "transposed", "channel_stride2"])
    print("snap seed=%d hk=%d g=%d n=%d d=%d w=%d %s %s" % (seed, hk, g, n, d, w, dtype, layout), flush=True)
    q, k = _qk(r.choice([1, 2]), g * hk, hk, n, d, dtype, 300 + seed, layout)
    got = snap_scores(q, k, w)
    ref = osnap.snap_scores(q.cpu(), k.cpu(), w)
    _check_scores(got, ref, min(w, n))
