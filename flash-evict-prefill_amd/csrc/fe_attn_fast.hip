// Fast path of the fused prefill kernel for gfx950: D in {64, 128}, positive softmax scale,
// 16-byte K/V rows. Same mathematics as the generic kernel in fe_attn.hip (reference
// flash_evict/prefill.py:14-83); the differences are in data movement and scheduling:
//
//   * K and V tiles (64 keys) go HBM -> LDS with buffer_load ... lds (16 B per lane), no
//     staging registers and no VALU work; rows past N read as zero through the buffer
//     range check. LDS rows are stored unpadded with the 16-byte chunk index XOR-swizzled
//     by the key, so fragment reads are bank-conflict free.
//   * The A operand of O^T = V^T P^T (eight keys of one channel per lane) comes straight
//     from the row-major V tile with two ds_read_b64_tr_b16 transposing reads; the key
//     order of the read matches the S^T accumulator row order that becomes P^T.
//   * Two LDS buffers per operand with K one tile ahead of V: iteration t issues the MFMAs
//     of QK(t+1) before the softmax VALU work of tile t (and, in the replay, before the
//     exp/column sums of tile t), so matrix and vector work of one wave can overlap; one
//     barrier per 64-key tile.
//   * O is rescaled only when some row's running max actually rises (wave vote).
//   * Masked logits are set to -inf in place, so masking costs one compare/select per
//     element on diagonal and ragged tiles only.
#include <math.h>
#include <string>

#include "fe_attn.h"
#include "fe_internal.h"

namespace fe {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Raise the wave's issue priority around MFMA blocks so that, of the two waves sharing a
// SIMD, the one with matrix work ready issues it first while the other fills the MFMA
// shadow with its softmax VALU work.
#ifndef FE_SETPRIO
#define FE_SETPRIO 1
#endif
// FE_PIPELINE=1 selects the software-pipelined schedule (QK of the next tile issued before
// the softmax of the current one); 0 the per-tile schedule.
#ifndef FE_PIPELINE
#define FE_PIPELINE 0
#endif
#if FE_SETPRIO
#define FE_PRIO_HI() __builtin_amdgcn_s_setprio(1)
#define FE_PRIO_LO() __builtin_amdgcn_s_setprio(0)
#else
#define FE_PRIO_HI() ((void)0)
#define FE_PRIO_LO() ((void)0)
#endif
typedef short s16x4 __attribute__((ext_vector_type(4)));


template <int DP>
struct FastTile {
  static constexpr int BN = 64;                  // keys per tile
  static constexpr int CPR = DP / 8;             // 16-byte chunks per row
  static constexpr int ROWB = DP * 2;            // bytes per row
  static constexpr int TILE = BN * ROWB;         // bytes per K or V tile
  static constexpr int DMA_PER_WAVE = (BN * CPR) / 256;
  static constexpr int NDC = DP / 16;            // MFMA k-chunks of QK^T
  static constexpr int NDT = DP / 32;            // 32-channel tiles of O^T
  static constexpr size_t RED_OFF = 4 * (size_t)TILE;
  static constexpr size_t LDS = RED_OFF + 2 * 4 * BN * 4;
};

// XOR applied to the 16-byte chunk index of row `key`. Two read patterns must be bank-
// conflict free (64 banks x 4 B = 256 B per cycle):
//   K fragments: 16 consecutive keys, one logical chunk per access phase;
//   V transposing reads: 4 consecutive keys x 4 consecutive chunks (aligned group of 4).
// Moving the key's two low bits into the chunk's high bits serves both: the 16 keys map to
// 16 distinct chunks, and the 4 keys of a transposing read land in 4 different chunk
// groups. For 128-byte rows (D = 64) two rows share a bank cycle, so key bit 0 selects the
// half and bits 1..3 are spread the same way.
template <int DP>
__device__ __forceinline__ int swz(int key) {
  return DP == 128 ? (((key & 3) << 2) | ((key >> 2) & 3)) : ((((key >> 1) & 1) << 2) | ((key >> 2) & 3));
}

// Issue the DMA of one 64-key tile: wave wv moves blocks wv, wv+4, ... of 1 KB; lane l of a
// block fills LDS chunk (block*64 + l) with the global chunk that the swizzle puts there.
template <int DP>
__device__ __forceinline__ void dma_tile(__amdgpu_buffer_rsrc_t rs, unsigned char* tile, int kb, u32 rowb_g,
                                         int wv, int lane) {
  typedef FastTile<DP> T;
#pragma unroll
  for (int r = 0; r < T::DMA_PER_WAVE; ++r) {
    const int blk = r * 4 + wv;
    const int c = blk * 64 + lane;
    const int key = c / T::CPR, pc = c % T::CPR;
    const int lc = pc ^ swz<DP>(key);
    const u32 voff = (u32)(kb + key) * rowb_g + (u32)lc * 16u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(tile + blk * 1024), 16, voff, 0, 0, 0);
  }
}

template <int DP>
__device__ __forceinline__ u32x4 k_frag(const unsigned char* tile, int key, int lc) {
  return *(const u32x4*)(tile + key * FastTile<DP>::ROWB + ((lc ^ swz<DP>(key)) << 4));
}

// Eight keys of channel (32*dt + lane%32) in P^T slot order for 16-key chunk `kc0`:
// slots 0-3 = keys kc0 + 4h + 0..3, slots 4-7 = keys kc0 + 8 + 4h + 0..3 (h = lane/32).
template <int DP>
__device__ __forceinline__ u32x4 v_frag(const unsigned char* tile, int kc0, int dt, int lane) {
  const int r = lane & 15, g = lane >> 4, h = lane >> 5;
  const int d = 32 * dt + 16 * (g & 1) + 4 * (r & 3);
  const int lc = d >> 3, hb = (d >> 2) & 1;
  const int k1 = kc0 + 4 * h + (r >> 2), k2 = k1 + 8;
  const unsigned char* p1 = tile + k1 * FastTile<DP>::ROWB + ((lc ^ swz<DP>(k1)) << 4) + (hb << 3);
  const unsigned char* p2 = tile + k2 * FastTile<DP>::ROWB + ((lc ^ swz<DP>(k2)) << 4) + (hb << 3);
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(lds_ptr_t)p1);
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(lds_ptr_t)p2);
  const u32x2 ua = __builtin_bit_cast(u32x2, a), ub = __builtin_bit_cast(u32x2, b);
  return (u32x4){ua[0], ua[1], ub[0], ub[1]};
}

template <typename E, int DP, int TPW>
__global__ __launch_bounds__(256, (TPW == 1 ? 2 : 1)) void fused_fast_kernel(const AttnArgs a) {
  typedef FastTile<DP> T;
  constexpr int BN = T::BN, NDC = T::NDC, NDT = T::NDT;
  constexpr float NEG_INF = -__builtin_huge_valf();
  constexpr float POS_INF = __builtin_huge_valf();

  extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];
  unsigned char* kt0 = smem;                     // K tiles [2]
  unsigned char* vt0 = smem + 2 * T::TILE;       // V tiles [2]
  float* red = (float*)(smem + T::RED_OFF);      // [2][4][BN]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6, l32 = lane & 31, hh = lane >> 5;
  const int N = a.N;

  const int bh = (int)(blockIdx.x % (unsigned)a.BH);
  const int wg = a.wg_bh - 1 - (int)(blockIdx.x / (unsigned)a.BH);
  const int b = bh / a.Hkv, hkv = bh - b * a.Hkv;
  const int t_begin = wg * 4 * TPW;
  const int t_end = min(a.tiles_bh, t_begin + 4 * TPW);
  const int wg_q_hi = min(N, ((t_end - 1) / a.G + 1) * 32);
  const int kv_end = a.causal ? wg_q_hi : N;
  const int ntiles = (kv_end + BN - 1) / BN;

  int q0[TPW], head[TPW], qlim[TPW];
  bool tv[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int t = t_begin + wv * TPW + j;
    tv[j] = t < t_end;
    const int tt = tv[j] ? t : t_begin;
    q0[j] = (tt / a.G) * 32;
    head[j] = hkv * a.G + (tt - (tt / a.G) * a.G);
    // last key this lane's query row may see; -1 for a padding tile
    qlim[j] = !tv[j] ? -1 : (a.causal ? min(q0[j] + l32, N - 1) : N - 1);
  }

  u32x4 qf[TPW][NDC];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int qr = q0[j] + l32;
    const bool ok = tv[j] && qr < N;
    const u16* qp = a.q + b * a.qs[0] + head[j] * a.qs[1] + (long long)(ok ? qr : 0) * a.qs[2];
#pragma unroll
    for (int c = 0; c < NDC; ++c)
      qf[j][c] = ok ? *(const u32x4*)(qp + 16 * c + 8 * hh) : (u32x4){0u, 0u, 0u, 0u};
  }

  const u32 krow = (u32)(a.ks[2] * 2), vrow = (u32)(a.vs[2] * 2);
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.k + b * a.ks[0] + hkv * a.ks[1]), (short)0, (int)((u32)N * krow), 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.v + b * a.vs[0] + hkv * a.vs[1]), (short)0, (int)((u32)N * vrow), 0x00020000);

  f32x16 o[TPW][NDT];
  float m_run[TPW], l_run[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    m_run[j] = NEG_INF;
    l_run[j] = 0.f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[j][dt] = (f32x16){};
  }

  // ---------------- traversal 1
  // Largest key any row of this wave attends to, and the smallest per-row limit of each
  // row tile (lane 0's): tiles past wave_hi are skipped, tiles past lo_lim[j] are masked.
  int lo_lim[TPW];
  int wave_hi = -1;
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    lo_lim[j] = !tv[j] ? -1 : (a.causal ? min(q0[j], N - 1) : N - 1);
    if (tv[j]) wave_hi = max(wave_hi, a.causal ? min(q0[j] + 31, N - 1) : N - 1);
  }

  // S^T = K Q^T for the 64 keys of one tile (two 32-key accumulators per row tile): per
  // 32-key half, the eight K fragments are requested, then the MFMA chain issues at raised
  // priority.
  auto qk_tile = [&](const unsigned char* kt, f32x16 (&sacc)[TPW][2]) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      u32x4 kf[NDC];
#pragma unroll
      for (int c = 0; c < NDC; ++c) kf[c] = k_frag<DP>(kt, 32 * s + l32, 2 * c + hh);
      FE_PRIO_HI();
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        sacc[j][s] = E::mfma(kf[0], qf[j][0], (f32x16){});
#pragma unroll
        for (int c = 1; c < NDC; ++c) sacc[j][s] = E::mfma(kf[c], qf[j][c], sacc[j][s]);
      }
      FE_PRIO_LO();
    }
  };

  // Mask, running max over the 64 keys of one tile, rescale of O and l when needed.
  // Returns nothing; leaves -m_run (0 for a row with no key yet) in nm.
  auto tile_stats = [&](int kb, f32x16 (&sacc)[TPW][2], float (&nm)[TPW]) {
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      if (kb + BN - 1 > lo_lim[j]) {
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = kb + 32 * s + 8 * (i >> 2) + 4 * hh + (i & 3);
            sacc[j][s][i] = key <= qlim[j] ? sacc[j][s][i] : NEG_INF;
          }
      }
      // max over the 32 keys of this lane: four independent max chains, then a tree
      float m4[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        m4[t] = fmaxf(sacc[j][0][4 * t], sacc[j][1][4 * t]);
#pragma unroll
        for (int i = 1; i < 4; ++i) m4[t] = fmaxf(m4[t], fmaxf(sacc[j][0][4 * t + i], sacc[j][1][4 * t + i]));
      }
      float mr = fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]));
      mr = half_swap_max(mr);
      // Exact running max: the dominant probability of a row stays exactly 1 before it is
      // rounded to the input dtype (a stale max would cost up to 2^-9 relative error on the
      // term that dominates a peaked row). O and l are only touched when some row's max rose.
      const float mt = mr * a.scale_log2;
      if (__any(mt > m_run[j])) {
        const float mn = fmaxf(m_run[j], mt);
        const float corr = mn > m_run[j] ? fast_exp2(m_run[j] - mn) : 1.f;
        l_run[j] *= corr;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) o[j][dt] *= corr;
        m_run[j] = mn;
      }
      nm[j] = m_run[j] == NEG_INF ? 0.f : -m_run[j];
    }
  };

  // P = exp2(S*scale - m) rounded to the input dtype (packed as the B operand of P@V)
  auto tile_exp = [&](f32x16 (&sacc)[TPW][2], const float (&nm)[TPW], u32x4 (&pb)[TPW][4]) {
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      float ps4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float p[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          p[i] = fast_exp2(fmaf(sacc[j][s][i], a.scale_log2, nm[j]));
          ps4[i & 3] += p[i];
        }
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2)
          pb[j][2 * s + c2] = (u32x4){E::pack2(p[8 * c2 + 0], p[8 * c2 + 1]), E::pack2(p[8 * c2 + 2], p[8 * c2 + 3]),
                                      E::pack2(p[8 * c2 + 4], p[8 * c2 + 5]), E::pack2(p[8 * c2 + 6], p[8 * c2 + 7])};
      }
      l_run[j] += (ps4[0] + ps4[1]) + (ps4[2] + ps4[3]);
    }
  };

  // O^T += V^T P^T over the four 16-key chunks of one tile, one 32-channel tile of O^T
  // at a time (four V fragments requested, then four MFMAs at raised priority)
  auto pv_tile = [&](const unsigned char* vt, const u32x4 (&pb)[TPW][4]) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      u32x4 vf[4];
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) vf[c4] = v_frag<DP>(vt, 16 * c4, dt, lane);
      FE_PRIO_HI();
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4)
#pragma unroll
        for (int j = 0; j < TPW; ++j) o[j][dt] = E::mfma(vf[c4], pb[j][c4], o[j][dt]);
      FE_PRIO_LO();
    }
  };

#if FE_PIPELINE
  // Pipeline: K runs one tile ahead of V in the two-buffer rings. Iteration t waits for
  // K(t+1) and V(t), starts the DMA of K(t+2) and V(t+1) into the buffers iteration t-1
  // finished with, settles the statistics of tile t, then issues QK(t+1) interleaved
  // (one LDS read, one MFMA, several VALU ops at a time) with the exponentials of tile t,
  // and finally P@V of tile t.
  f32x16 sA[TPW][2], sB[TPW][2];
  dma_tile<DP>(krs, kt0, 0, krow, wv, lane);
  dma_tile<DP>(vrs, vt0, 0, vrow, wv, lane);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (ntiles > 1) dma_tile<DP>(krs, kt0 + T::TILE, BN, krow, wv, lane);
  if (wave_hi >= 0) qk_tile(kt0, sA);

  auto t1_step = [&](int it, f32x16 (&cur)[TPW][2], f32x16 (&nxt)[TPW][2]) {
    const int kb = it * BN;
    const int buf = it & 1;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (it + 2 < ntiles) dma_tile<DP>(krs, kt0 + buf * T::TILE, kb + 2 * BN, krow, wv, lane);
    if (it + 1 < ntiles) dma_tile<DP>(vrs, vt0 + (buf ^ 1) * T::TILE, kb + BN, vrow, wv, lane);
    if (kb > wave_hi) return;
    float nm[TPW];
    tile_stats(kb, cur, nm);
    // Branch-free region: QK(t+1) (the last tile reads a stale buffer whose result is
    // never used) interleaved with the exponentials of tile t.
    u32x4 pb[TPW][4];
    qk_tile(kt0 + (buf ^ 1) * T::TILE, nxt);
    tile_exp(cur, nm, pb);
#pragma unroll
    for (int g = 0; g < 2 * NDC * TPW; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // six VALU
    }
    pv_tile(vt0 + buf * T::TILE, pb);
  };
  for (int it = 0; it < ntiles; it += 2) {
    t1_step(it, sA, sB);
    if (it + 1 < ntiles) t1_step(it + 1, sB, sA);
  }
#else
  // Per tile: wait for K(t) and V(t), start the DMA of tile t+1 into the other buffers,
  // QK(t), statistics, exponentials, P@V(t). The two waves sharing a SIMD overlap each
  // other's MFMA and VALU phases; s_setprio favours the one with matrix work ready.
  dma_tile<DP>(krs, kt0, 0, krow, wv, lane);
  dma_tile<DP>(vrs, vt0, 0, vrow, wv, lane);
  for (int it = 0; it < ntiles; ++it) {
    const int kb = it * BN;
    const int buf = it & 1;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (it + 1 < ntiles) {
      dma_tile<DP>(krs, kt0 + (buf ^ 1) * T::TILE, kb + BN, krow, wv, lane);
      dma_tile<DP>(vrs, vt0 + (buf ^ 1) * T::TILE, kb + BN, vrow, wv, lane);
    }
    if (kb > wave_hi) continue;
    f32x16 sacc[TPW][2];
    qk_tile(kt0 + buf * T::TILE, sacc);
    float nm[TPW];
    tile_stats(kb, sacc, nm);
    u32x4 pb[TPW][4];
    tile_exp(sacc, nm, pb);
    pv_tile(vt0 + buf * T::TILE, pb);
  }
#endif

  // ---------------- finish rows
  float l_tot[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    l_tot[j] = half_swap_sum(l_run[j]);
    const int qi = q0[j] + l32;
    if (!tv[j] || qi >= N) continue;
    const float inv = 1.f / l_tot[j];
    u16* op = a.out + ((long long)(b * a.Hq + head[j]) * N + qi) * DP;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d0 = 32 * dt + 8 * g4 + 4 * hh;
        const u32 w0 = E::pack2(o[j][dt][4 * g4 + 0] * inv, o[j][dt][4 * g4 + 1] * inv);
        const u32 w1 = E::pack2(o[j][dt][4 * g4 + 2] * inv, o[j][dt][4 * g4 + 3] * inv);
        *(u32x2*)(op + d0) = (u32x2){w0, w1};
      }
    }
  }

  // ---------------- traversal 2: replay
  if (!a.score || wg_q_hi - 1 < a.win_lo) return;

  float bias[TPW][16];
  bool rin[TPW];
  int wave_hi_r = -1;
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int qi = q0[j] + l32;
    const bool live = tv[j] && qi < N && qi >= a.win_lo;
    const float br = live ? (m_run[j] + fast_log2(l_tot[j]) - a.decay_log2 * (float)(qi - (N - 1))) : POS_INF;
#pragma unroll
    for (int i = 0; i < 16; ++i) bias[j][i] = __shfl(br, 8 * (i >> 2) + 4 * hh + (i & 3));
    rin[j] = tv[j] && q0[j] + 31 >= a.win_lo;
    if (rin[j]) wave_hi_r = max(wave_hi_r, a.causal ? min(q0[j] + 31, N - 1) : N - 1);
  }

  float* imp_row = a.imp + (long long)bh * N;

  // S = Q K^T (lanes hold keys) for the 64 keys of one tile
  auto qk_replay = [&](const unsigned char* kt, f32x16 (&sacc)[TPW][2]) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      u32x4 kf[NDC];
#pragma unroll
      for (int c = 0; c < NDC; ++c) kf[c] = k_frag<DP>(kt, 32 * s + l32, 2 * c + hh);
      FE_PRIO_HI();
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        sacc[j][s] = E::mfma(qf[j][0], kf[0], (f32x16){});
#pragma unroll
        for (int c = 1; c < NDC; ++c) sacc[j][s] = E::mfma(qf[j][c], kf[c], sacc[j][s]);
      }
      FE_PRIO_LO();
    }
  };

  // Column sums of one tile's S (in `cur`) -> cs[2]; diagonal tiles are masked first.
  auto replay_sums = [&](int kb, f32x16 (&cur)[TPW][2], float (&cs)[2]) {
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float c4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 16; ++i) c4[i & 3] += fast_exp2(fmaf(cur[j][s][i], a.scale_log2, -bias[j][i]));
        cs[s] += (c4[0] + c4[1]) + (c4[2] + c4[3]);
      }
    }
  };
  auto replay_mask = [&](int kb, f32x16 (&cur)[TPW][2]) {
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
      if (a.causal && kb + BN - 1 > q0[j]) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const int key = kb + 32 * s + l32;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int qr = q0[j] + 8 * (i >> 2) + 4 * hh + (i & 3);
            cur[j][s][i] = key > qr ? NEG_INF : cur[j][s][i];
          }
        }
      }
    }
  };
  // Flush of the previous tile's four per-wave column sums (written before the barrier
  // that precedes this call): one atomic per key per workgroup.
  auto replay_flush = [&](int kb_prev, int buf_prev) {
    if (tid < BN) {
      const float* rr = red + buf_prev * 4 * BN;
      const float sum = (rr[tid] + rr[BN + tid]) + (rr[2 * BN + tid] + rr[3 * BN + tid]);
      const int key = kb_prev + tid;
      if (sum != 0.f && key < N) unsafeAtomicAdd(imp_row + key, sum);
    }
  };
  auto replay_store = [&](int buf, float (&cs)[2]) {
    cs[0] = half_swap_sum(cs[0]);
    cs[1] = half_swap_sum(cs[1]);
    if (hh == 0) {
      float* rb = red + buf * 4 * BN + wv * BN;
      rb[l32] = cs[0];
      rb[32 + l32] = cs[1];
    }
  };

  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();  // every wave is done reading the traversal-1 tiles
  dma_tile<DP>(krs, kt0, 0, krow, wv, lane);
#if FE_PIPELINE
  // Same pipeline as traversal 1 with K only: QK(t+1) is interleaved with the exp/column
  // sums of tile t.
  f32x16 rA[TPW][2], rB[TPW][2];
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (ntiles > 1) dma_tile<DP>(krs, kt0 + T::TILE, BN, krow, wv, lane);
  if (wave_hi_r >= 0) qk_replay(kt0, rA);

  auto t2_step = [&](int it, f32x16 (&cur)[TPW][2], f32x16 (&nxt)[TPW][2]) {
    const int kb = it * BN;
    const int buf = it & 1;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (it > 0) replay_flush(kb - BN, buf ^ 1);
    if (it + 2 < ntiles) dma_tile<DP>(krs, kt0 + buf * T::TILE, kb + 2 * BN, krow, wv, lane);
    float cs[2] = {0.f, 0.f};
    if (kb <= wave_hi_r) {
      replay_mask(kb, cur);
      // Branch-free region: QK(t+1) interleaved with the exp/column sums of tile t.
      qk_replay(kt0 + (buf ^ 1) * T::TILE, nxt);
      replay_sums(kb, cur, cs);
#pragma unroll
      for (int g = 0; g < 2 * NDC * TPW; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // six VALU
      }
    }
    replay_store(buf, cs);
  };
  for (int it = 0; it < ntiles; it += 2) {
    t2_step(it, rA, rB);
    if (it + 1 < ntiles) t2_step(it + 1, rB, rA);
  }
#else
  for (int it = 0; it < ntiles; ++it) {
    const int kb = it * BN;
    const int buf = it & 1;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (it > 0) replay_flush(kb - BN, buf ^ 1);
    if (it + 1 < ntiles) dma_tile<DP>(krs, kt0 + (buf ^ 1) * T::TILE, kb + BN, krow, wv, lane);
    float cs[2] = {0.f, 0.f};
    if (kb <= wave_hi_r) {
      f32x16 cur[TPW][2];
      qk_replay(kt0 + buf * T::TILE, cur);
      replay_mask(kb, cur);
      replay_sums(kb, cur, cs);
    }
    replay_store(buf, cs);
  }
#endif
  __syncthreads();
  if (tid < BN) {
    const int buf = (ntiles - 1) & 1;
    const float* rr = red + buf * 4 * BN;
    const float sum = (rr[tid] + rr[BN + tid]) + (rr[2 * BN + tid] + rr[3 * BN + tid]);
    const int key = (ntiles - 1) * BN + tid;
    if (key < N && sum != 0.f) unsafeAtomicAdd(imp_row + key, sum);
  }
}

namespace {

template <typename E, int DP, int TPW>
FusedPlan fast_entry(const char* name) {
  return FusedPlan{(const void*)fused_fast_kernel<E, DP, TPW>, FastTile<DP>::LDS, TPW, name};
}

FusedPlan g_fast[] = {
    fast_entry<F16, 64, 1>("fused_fast<f16,64,1>"),
    fast_entry<F16, 128, 1>("fused_fast<f16,128,1>"),
    fast_entry<BF16, 64, 1>("fused_fast<bf16,64,1>"),
    fast_entry<BF16, 128, 1>("fused_fast<bf16,128,1>"),
};

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

bool kv_ok(const void* p, const long long* st, int N, int D) {
  if (st[3] != 1 || !aligned16(p) || st[0] % 8 || st[1] % 8 || st[2] % 8 || st[2] < D) return false;
  // byte offsets of rows up to N + 64 (one tile past the end) must fit the 32-bit range
  return (unsigned long long)(N + 64) * (unsigned long long)st[2] * 2ull < (1ull << 31);
}

}  // namespace

bool fast_plan(const AttnArgs& a, int dtype, FusedPlan& plan) {
  if (a.D != 64 && a.D != 128) return false;
  if (!(a.scale_log2 > 0.f) || !a.qvec) return false;
  if (!kv_ok(a.k, a.ks, a.N, a.D) || !kv_ok(a.v, a.vs, a.N, a.D)) return false;
  const int idx = (dtype == 1 ? 2 : 0) + (a.D == 128 ? 1 : 0);
  plan = g_fast[idx];
  return true;
}

void append_fast_resources(std::string& out) {
  for (const auto& e : g_fast) {
    hipFuncAttributes attr;
    if (hipFuncGetAttributes(&attr, e.fn) != hipSuccess) continue;
    char buf[512];
    snprintf(buf, sizeof(buf),
             "{\"kernel\":\"%s\",\"registers_per_thread\":%d,\"lds_static_bytes\":%zu,"
             "\"lds_dynamic_bytes\":%zu,\"scratch_bytes_per_thread\":%zu,\"max_threads_per_block\":%d},",
             e.name, attr.numRegs, (size_t)attr.sharedSizeBytes, e.lds, (size_t)attr.localSizeBytes,
             attr.maxThreadsPerBlock);
    out += buf;
  }
}

}  // namespace fe
