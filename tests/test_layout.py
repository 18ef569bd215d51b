"""Host-side check of the fast kernels' LDS tile layout (fe_attn_fast.hip `dma_tile_cm`,
`k_frags`, `v_frag`, and the replay kernel's K reads): K and V tiles are stored
channel-group-major. The DMA must write every LDS byte of a tile once, each fragment read
must return the key and channels the MFMA expects, and each read phase must touch distinct
bank slots (64 banks x 4 B = 256 B per cycle; 16 lanes per phase for 16-byte reads, 32 for
8-byte transposing reads)."""
import pytest


def cm_tile(dp, gb):
    """LDS byte -> (key, byte of the key's row) after dma_tile_cm<DPW, gb> has moved one
    64-key tile with contiguous rows (rowb = 2 dp): wave wv, block r, lane l."""
    rowb, dpw = 2 * dp, (64 * (dp // 8)) // 256
    kpb = 1024 // gb
    bpg = 64 // kpb
    lds = {}
    for wv in range(4):
        k0 = (wv % bpg) * kpb
        for r in range(dpw):
            assert 64 * r + gb <= rowb                     # soffset + group width within a row
            base = k0 * rowb + (wv // bpg) * gb + 64 * r
            for lane in range(64):
                if gb == 32:
                    doff = (lane >> 1) * rowb + (((lane & 1) ^ ((lane >> 4) & 1)) << 4)
                else:
                    doff = (lane >> 2) * rowb + ((lane & 3) << 4)
                key, byte = divmod(base + doff, rowb)
                assert byte + 16 <= rowb
                dst = wv * 1024 + r * 4096 + lane * 16
                for x in range(16):
                    assert dst + x not in lds
                    lds[dst + x] = (key, byte + x)
    assert sorted(lds) == list(range(64 * rowb))
    return lds


@pytest.mark.parametrize("dp", [32, 64, 96, 128, 160, 192, 224, 256])
def test_cm_k_fragments(dp):
    lds = cm_tile(dp, 32)
    for s in range(2):
        for c in range(dp // 16):
            phases = {}
            for lane in range(64):
                l32, hh = lane & 31, lane >> 5
                a = c * 2048 + s * 1024 + l32 * 32 + ((hh ^ ((l32 >> 3) & 1)) << 4)
                assert [lds[a + x] for x in range(16)] == [(32 * s + l32, (2 * c + hh) * 16 + x) for x in range(16)]
                phases.setdefault(lane // 16, []).extend((a // 4 + i) % 64 for i in range(4))
            assert all(len(set(b)) == 64 for b in phases.values())


@pytest.mark.parametrize("dp", [32, 64, 96, 128, 160, 192, 224, 256])
def test_cm_v_transposing_reads(dp):
    lds = cm_tile(dp, 64)
    for dt in range(dp // 32):
        for c4 in range(4):
            for half in range(2):
                phases = {}
                for lane in range(64):
                    r, g, hh = lane & 15, lane >> 4, lane >> 5
                    a = dt * 4096 + c4 * 1024 + half * 512 + (4 * hh + (r >> 2)) * 64 + 32 * (g & 1) + 8 * (r & 3)
                    key = 16 * c4 + 8 * half + 4 * hh + (r >> 2)
                    d = 32 * dt + 16 * (g & 1) + 4 * (r & 3)
                    assert [lds[a + x] for x in range(8)] == [(key, 2 * d + x) for x in range(8)]
                    phases.setdefault(lane // 32, []).extend((a // 4 + i) % 64 for i in range(2))
                assert all(len(set(b)) == 64 for b in phases.values())


@pytest.mark.parametrize("dp,d", [(32, 8), (32, 24), (64, 40), (64, 48), (96, 72), (96, 80), (128, 104), (128, 120),
                                  (160, 136), (192, 184), (224, 200), (256, 232), (256, 248)])
@pytest.mark.parametrize("gb", [32, 64])
def test_cm_partial_head_dim(dp, d, gb):
    # dma_tile_cm<DPW, GB, PARTIAL>: a lane's first channel, (group of block r) * GB/2 + dch, is
    # the channel its 16-byte read starts at; lanes at or past D read zeros (offset past the
    # record count), and every lane that reads stays inside the row's D channels
    rowb_dense = 2 * dp
    dpw = (64 * (dp // 8)) // 256
    kpb = 1024 // gb
    bpg = 64 // kpb
    zeros = set()
    for wv in range(4):
        for r in range(dpw):
            for lane in range(64):
                if gb == 32:
                    doff = (lane >> 1) * rowb_dense + (((lane & 1) ^ ((lane >> 4) & 1)) << 4)
                    dch = ((lane & 1) ^ ((lane >> 4) & 1)) << 3
                else:
                    doff = (lane >> 2) * rowb_dense + ((lane & 3) << 4)
                    dch = (lane & 3) << 3
                byte = (wv // bpg) * gb + 64 * r + doff % rowb_dense
                ch = (wv // bpg + (4 // bpg) * r) * (gb // 2) + dch
                assert ch == byte // 2
                if ch < d:
                    assert byte + 16 <= 2 * d
                else:
                    zeros.add((wv, r, lane))
    # the zero lanes are exactly the chunks of channels d .. dp-1 of every key
    assert len(zeros) * 8 == 64 * (dp - d)
