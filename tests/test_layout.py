"""Host-side check of the fast kernel's LDS layout rules (fe_attn_fast.hip `swz`, `k_frag`,
`v_frag`): the chunk swizzle is a bijection per row, and the two read patterns the kernel
issues touch distinct bank slots (64 banks x 4 B = 256 B per cycle)."""
import pytest


def swz(dp, k):
    if dp == 128:
        return ((k & 3) << 2) | ((k >> 2) & 3)
    return (((k >> 1) & 1) << 2) | ((k >> 2) & 3)


@pytest.mark.parametrize("dp", [64, 128])
def test_swizzle_is_bijective(dp):
    cpr = dp // 8
    for k in range(64):
        assert sorted(c ^ swz(dp, k) for c in range(cpr)) == list(range(cpr))


@pytest.mark.parametrize("dp", [64, 128])
def test_k_fragment_reads_conflict_free(dp):
    # 16 lanes of one phase: keys k0..k0+15, one logical chunk, 16 B each
    rowb, cpr = dp * 2, dp // 8
    for k0 in range(0, 64, 16):
        for lc in range(cpr):
            slots = [((k * rowb + ((lc ^ swz(dp, k)) << 4)) % 256) // 16 for k in range(k0, k0 + 16)]
            assert len(set(slots)) == 16


@pytest.mark.parametrize("dp", [64, 128])
def test_v_transposing_reads_conflict_free(dp):
    # half-wave of ds_read_b64_tr_b16: lanes r in 0..15 of groups g in {0,1}, 8 B each
    rowb = dp * 2
    for kc0 in range(0, 64, 16):
        for h in (0, 1):
            for dt in range(dp // 32):
                slots = set()
                for g in (0, 1):
                    for r in range(16):
                        k = kc0 + 4 * h + (r >> 2)
                        d = 32 * dt + 16 * g + 4 * (r & 3)
                        addr = k * rowb + (((d >> 3) ^ swz(dp, k)) << 4) + ((d >> 2) & 1) * 8
                        slots.add((addr % 256) // 8)
                assert len(slots) == 32
