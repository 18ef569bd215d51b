// Fused prefill for gfx950: online-softmax attention (traversal 1) followed by an exact
// replay of the QK^T tiles with each query row's final softmax statistics (traversal 2),
// whose weighted column sums become per-KV-token importance.
//
// Semantics follow flash_evict/prefill.py:14-83 (kernel) and :102-137 (launch):
//   * GQA map kvhead = head // (Hq/Hkv)                                    (prefill.py:26)
//   * logits scaled by scale*log2(e), causal row >= key, exp2 online softmax (:45-54)
//   * P rounded to the input dtype before P@V, FP32 accumulation            (:57)
//   * out = acc / l in the input dtype                                      (:59-60)
//   * replay only where (query block end) > N - W                           (:61)
//   * w_q = exp(decay*(q-(N-1))) for N-W <= q < N, else 0                   (:66-67)
//     (rows whose w_q underflows to exactly 0 in FP32 are not replayed: replay_rows)
//   * p = exp2(s - m_q) / l_q, column sums over queries and grouped heads   (:68-77)
//   * x ||v_k||_1 when value weighted                                       (:78-81)
//   * FP32 atomic accumulation into I[b, kvhead, k]                         (:82-83)
//
// The design is gfx950-native rather than a transcription of the Triton schedule:
//   * one workgroup = 4 waves = 4*TPW row tiles; a row tile is 32 query positions of one
//     query head, and all row tiles of a workgroup share one KV head, so every K/V tile
//     staged in LDS serves all grouped query heads (GQA packing);
//   * traversal 1 computes S^T = K Q^T on v_mfma_f32_32x32x16_{bf16,f16}: lanes hold
//     query columns, registers hold keys, so the row max/sum are in-lane plus one
//     v_permlane32_swap; O^T = V^T P^T takes P^T straight from the S^T accumulators;
//   * V is transposed while it is staged into LDS (v_perm_b32 packing), with the key order
//     inside each 16-key group permuted to match the accumulator layout of S^T, so the
//     A operand of P@V is one 16-byte LDS read per lane;
//   * traversal 2 swaps the MFMA operands (S = Q K^T) so that lanes hold keys: the column
//     sum over queries is in-lane plus one lane swap; 1/l_q and w_q are folded into one
//     exponent bias per row, so each replayed element costs one FMA, one v_exp_f32, one add;
//   * the four waves' column sums meet in LDS and each workgroup issues one FP32 atomic
//     per key; the value L1 norm multiplies the finished sums in a separate pass;
//   * workgroups are issued heaviest-causal-first, with consecutive block ids on
//     different KV heads (the hardware deals blocks round-robin over the 8 XCDs, so each
//     XCD's L2 sees a small set of KV heads).
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <mutex>
#include <string>
#include <vector>

#include "fe_attn.h"
#include "fe_internal.h"
#include "../../include/flash_evict.h"

namespace fe {

template <int DP>
struct Tile {
  static constexpr int BN = 64;                 // keys per LDS tile (two 32-key sub-tiles)
  static constexpr int NDC = DP / 16;           // 16-channel MFMA k-chunks of QK^T
  static constexpr int NDT = DP / 32;           // 32-channel row tiles of O^T
  static constexpr int KST = DP + 8;            // LDS row stride of K (elements)
  static constexpr int VST = BN + 8;            // LDS row stride of V^T (elements)
  static constexpr int KCH = DP / 8;            // 16-byte chunks per K/V row
  static constexpr int KITEMS = BN * KCH;
  static constexpr int KPT = (KITEMS + 255) / 256;
  static constexpr int VITEMS = (BN / 4) * KCH; // (4-key group, chunk) items
  static constexpr int VPT = (VITEMS + 255) / 256;
  static constexpr size_t LDS_K = (size_t)2 * BN * KST * 2;
  static constexpr size_t LDS_V = (size_t)2 * DP * VST * 2;
  static constexpr size_t LDS_RED = (size_t)2 * 4 * BN * 4;
  static constexpr size_t LDS = LDS_K + LDS_V + LDS_RED;
};

template <typename E, int DP, int TPW>
__global__ __launch_bounds__(256) void fused_attn_score_kernel(const AttnArgs a) {
  typedef Tile<DP> T;
  constexpr int BN = T::BN, NDC = T::NDC, NDT = T::NDT, KST = T::KST, VST = T::VST;
  constexpr int KCH = T::KCH, KITEMS = T::KITEMS, KPT = T::KPT, VITEMS = T::VITEMS, VPT = T::VPT;
  constexpr float NEG_INF = -__builtin_huge_valf();
  constexpr float POS_INF = __builtin_huge_valf();

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  u16* kl = (u16*)smem;                                  // [2][BN][KST]
  u16* vl = (u16*)(smem + T::LDS_K);                     // [2][DP][VST]
  float* red = (float*)(smem + T::LDS_K + T::LDS_V);     // [2][4][BN]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6, l32 = lane & 31, hh = lane >> 5;
  const int N = a.N, D = a.D;

  // ---- work decode: heaviest query blocks first, consecutive ids on different KV heads
  const int bh = (int)(blockIdx.x % (unsigned)a.BH);
  const int wg = a.wg_bh - 1 - (int)(blockIdx.x / (unsigned)a.BH);
  const int b = bh / a.Hkv, hkv = bh - b * a.Hkv;
  const int t_begin = wg * 4 * TPW;
  const int t_end = min(a.tiles_bh, t_begin + 4 * TPW);
  const int wg_q_hi = min(N, ((t_end - 1) / a.G + 1) * 32);  // exclusive query bound
  const int kv_end = a.causal ? wg_q_hi : N;
  const int ntiles = (kv_end + BN - 1) / BN;

  int q0[TPW];
  bool tv[TPW];
  int head[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int t = t_begin + wv * TPW + j;
    tv[j] = t < t_end;
    const int tt = tv[j] ? t : t_begin;
    q0[j] = (tt / a.G) * 32;
    head[j] = hkv * a.G + (tt - (tt / a.G) * a.G);
  }

  // ---- Q fragments: lane (row l32, half hh) holds channels [16c + 8hh, +8)
  u32x4 qf[TPW][NDC];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int qr = q0[j] + l32;
    const bool ok = tv[j] && qr < N;
    const u16* qp = a.q + b * a.qs[0] + head[j] * a.qs[1] + (long long)(ok ? qr : 0) * a.qs[2];
#pragma unroll
    for (int c = 0; c < NDC; ++c)
      qf[j][c] = ok ? load8(qp, a.qs[3], 16 * c + 8 * hh, D, a.qvec) : (u32x4){0u, 0u, 0u, 0u};
  }

  const u16* kbase = a.k + b * a.ks[0] + hkv * a.ks[1];
  const u16* vbase = a.v + b * a.vs[0] + hkv * a.vs[1];

  auto kload = [&](int kb, u32x4 (&kr)[KPT]) {
#pragma unroll
    for (int r = 0; r < KPT; ++r) {
      const int i = tid + 256 * r;
      if (KITEMS % 256 == 0 || i < KITEMS) {
        const int key = i / KCH, ch = i - key * KCH;
        const int gk = kb + key;
        kr[r] = gk < N ? load8(kbase + (long long)gk * a.ks[2], a.ks[3], ch * 8, D, a.kvec)
                       : (u32x4){0u, 0u, 0u, 0u};
      }
    }
  };
  auto kstore = [&](int buf, const u32x4 (&kr)[KPT]) {
#pragma unroll
    for (int r = 0; r < KPT; ++r) {
      const int i = tid + 256 * r;
      if (KITEMS % 256 == 0 || i < KITEMS) {
        const int key = i / KCH, ch = i - key * KCH;
        *(u32x4*)(kl + buf * BN * KST + key * KST + ch * 8) = kr[r];
      }
    }
  };
  // V item (kg, ch): keys 4kg..4kg+3 of the tile, channels 8ch..8ch+7. kg varies fastest so
  // that one wave's transposed 8-byte writes cover all LDS banks.
  auto vload = [&](int kb, u32x4 (&vr)[VPT][4]) {
#pragma unroll
    for (int r = 0; r < VPT; ++r) {
      const int i = tid + 256 * r;
      if (VITEMS % 256 == 0 || i < VITEMS) {
        const int kg = i & 15, ch = i >> 4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int gk = kb + 4 * kg + e;
          vr[r][e] = gk < N ? load8(vbase + (long long)gk * a.vs[2], a.vs[3], ch * 8, D, a.vvec)
                            : (u32x4){0u, 0u, 0u, 0u};
        }
      }
    }
  };
  auto vstore = [&](int buf, const u32x4 (&vr)[VPT][4]) {
#pragma unroll
    for (int r = 0; r < VPT; ++r) {
      const int i = tid + 256 * r;
      if (VITEMS % 256 == 0 || i < VITEMS) {
        const int kg = i & 15, ch = i >> 4;
        // 4-key group g of a 16-key chunk lands at position 4*{0,2,1,3}[g]: the P^T
        // accumulator row order of a 32x32 MFMA (row = 8*(i/4) + 4*half + i%4).
        const int gi = kg & 3;
        const int pos = 16 * (kg >> 2) + 4 * (((gi & 1) << 1) | (gi >> 1));
        u16* dst = vl + buf * DP * VST + (ch * 8) * VST + pos;
#pragma unroll
        for (int dd = 0; dd < 8; ++dd) {
          const u32 sel = (dd & 1) ? 0x07060302u : 0x05040100u;
          const int w = dd >> 1;
          const u32 lo = __builtin_amdgcn_perm(vr[r][1][w], vr[r][0][w], sel);
          const u32 hi = __builtin_amdgcn_perm(vr[r][3][w], vr[r][2][w], sel);
          *(u32x2*)(dst + dd * VST) = (u32x2){lo, hi};
        }
      }
    }
  };

  // ---- traversal 1: online-softmax attention
  f32x16 o[TPW][NDT];
  float m_run[TPW], l_run[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    m_run[j] = NEG_INF;
    l_run[j] = 0.f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[j][dt] = (f32x16){};
  }

  {
    u32x4 kr[KPT];
    u32x4 vr[VPT][4];
    kload(0, kr);
    vload(0, vr);
    kstore(0, kr);
    vstore(0, vr);
  }
  __syncthreads();

  for (int it = 0; it < ntiles; ++it) {
    const int cur = it & 1;
    const int kb = it * BN;
    const bool more = it + 1 < ntiles;
    u32x4 kr[KPT];
    u32x4 vr[VPT][4];
    if (more) {
      kload(kb + BN, kr);
      vload(kb + BN, vr);
    }
    const u16* kc = kl + cur * BN * KST;
    const u16* vc = vl + cur * DP * VST;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int kbs = kb + 32 * s;
      if (kbs >= kv_end) break;
      bool act[TPW];
      bool any = false;
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        act[j] = tv[j] && (!a.causal || kbs <= q0[j] + 31);
        any |= act[j];
      }
      if (!any) continue;

      f32x16 sacc[TPW];
#pragma unroll
      for (int j = 0; j < TPW; ++j) sacc[j] = (f32x16){};
#pragma unroll
      for (int c = 0; c < NDC; ++c) {
        const u32x4 kf = *(const u32x4*)(kc + (32 * s + l32) * KST + 16 * c + 8 * hh);
#pragma unroll
        for (int j = 0; j < TPW; ++j)
          if (act[j]) sacc[j] = E::mfma(kf, qf[j][c], sacc[j]);
      }

      u32x4 pb[TPW][2];
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        if (!act[j]) continue;
        const int qi = q0[j] + l32;
        const bool need_mask = (a.causal && kbs + 31 > q0[j]) || kbs + 32 > N;
        float p[16];
        float mn, corr;
        if (need_mask) {
          bool ok[16];
          float mr = NEG_INF;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = kbs + 8 * (i >> 2) + 4 * hh + (i & 3);
            ok[i] = key < N && (!a.causal || key <= qi);
            const float sv = a.neg_scale ? -sacc[j][i] : sacc[j][i];
            mr = fmaxf(mr, ok[i] ? sv : NEG_INF);
          }
          mr = half_swap_max(mr);
          const float mt = (mr == NEG_INF) ? NEG_INF : mr * a.abs_scale_log2;
          mn = fmaxf(m_run[j], mt);
          corr = (mn == m_run[j]) ? 1.f : fast_exp2(m_run[j] - mn);
#pragma unroll
          for (int i = 0; i < 16; ++i)
            p[i] = ok[i] ? fast_exp2(fmaf(sacc[j][i], a.scale_log2, -mn)) : 0.f;
        } else {
          float mr = NEG_INF;
          if (a.neg_scale) {
#pragma unroll
            for (int i = 0; i < 16; ++i) mr = fmaxf(mr, -sacc[j][i]);
          } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) mr = fmaxf(mr, sacc[j][i]);
          }
          mr = half_swap_max(mr);
          const float mt = mr * a.abs_scale_log2;
          mn = fmaxf(m_run[j], mt);
          corr = (mn == m_run[j]) ? 1.f : fast_exp2(m_run[j] - mn);
#pragma unroll
          for (int i = 0; i < 16; ++i) p[i] = fast_exp2(fmaf(sacc[j][i], a.scale_log2, -mn));
        }
        float ps = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) ps += p[i];
        l_run[j] = l_run[j] * corr + ps;
        m_run[j] = mn;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) o[j][dt] *= corr;
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2)
          pb[j][c2] = (u32x4){E::pack2(p[8 * c2 + 0], p[8 * c2 + 1]), E::pack2(p[8 * c2 + 2], p[8 * c2 + 3]),
                              E::pack2(p[8 * c2 + 4], p[8 * c2 + 5]), E::pack2(p[8 * c2 + 6], p[8 * c2 + 7])};
      }

#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) {
          const u32x4 vf = *(const u32x4*)(vc + (32 * dt + l32) * VST + 32 * s + 16 * c2 + 8 * hh);
#pragma unroll
          for (int j = 0; j < TPW; ++j)
            if (act[j]) o[j][dt] = E::mfma(vf, pb[j][c2], o[j][dt]);
        }
      }
    }
    if (more) {
      kstore(cur ^ 1, kr);
      vstore(cur ^ 1, vr);
    }
    __syncthreads();
  }

  // ---- finish rows: O = acc / l, stored in the input dtype
  float l_tot[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    l_tot[j] = half_swap_sum(l_run[j]);
    const int qi = q0[j] + l32;
    if (!tv[j] || qi >= N) continue;
    const float inv = 1.f / l_tot[j];
    u16* op = a.out + ((long long)(b * a.Hq + head[j]) * N + qi) * D;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d0 = 32 * dt + 8 * g4 + 4 * hh;
        const float x0 = o[j][dt][4 * g4 + 0] * inv, x1 = o[j][dt][4 * g4 + 1] * inv;
        const float x2 = o[j][dt][4 * g4 + 2] * inv, x3 = o[j][dt][4 * g4 + 3] * inv;
        const u32 w0 = E::pack2(x0, x1), w1 = E::pack2(x2, x3);
        if (a.ovec && d0 + 3 < D) {
          *(u32x2*)(op + d0) = (u32x2){w0, w1};
        } else {
          if (d0 + 0 < D) op[d0 + 0] = (u16)(w0 & 0xffffu);
          if (d0 + 1 < D) op[d0 + 1] = (u16)(w0 >> 16);
          if (d0 + 2 < D) op[d0 + 2] = (u16)(w1 & 0xffffu);
          if (d0 + 3 < D) op[d0 + 3] = (u16)(w1 >> 16);
        }
      }
    }
  }

  // ---- traversal 2: replay with final statistics, weighted column sums -> importance
  if (!a.score || wg_q_hi - 1 < a.win_lo) return;

  // Row bias b_q = m_q + log2(l_q) - log2(w_q): p_q,k * w_q = exp2(s*scale - b_q).
  // Rows outside the observation window (or past N) get +inf, i.e. weight 0.
  float bias[TPW][16];
  bool rin[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int qi = q0[j] + l32;
    const bool live = tv[j] && qi < N && qi >= a.win_lo;
    const float br = live ? (m_run[j] + fast_log2(l_tot[j]) - a.decay_log2 * (float)(qi - (N - 1))) : POS_INF;
#pragma unroll
    for (int i = 0; i < 16; ++i) bias[j][i] = __shfl(br, 8 * (i >> 2) + 4 * hh + (i & 3));
    rin[j] = tv[j] && q0[j] + 31 >= a.win_lo;
  }

  __syncthreads();  // all waves are done with the traversal-1 LDS buffers
  {
    u32x4 kr[KPT];
    kload(0, kr);
    kstore(0, kr);
  }
  __syncthreads();

  float* imp_row = a.imp + (long long)bh * N;
  for (int it = 0; it < ntiles; ++it) {
    const int cur = it & 1;
    const int kb = it * BN;
    const bool more = it + 1 < ntiles;
    u32x4 kr[KPT];
    if (more) kload(kb + BN, kr);
    const u16* kc = kl + cur * BN * KST;
    float cs[2] = {0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int kbs = kb + 32 * s;
      if (kbs >= kv_end) break;
      bool act[TPW];
      bool any = false;
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        act[j] = rin[j] && (!a.causal || kbs <= q0[j] + 31);
        any |= act[j];
      }
      if (!any) continue;
      f32x16 sacc[TPW];
#pragma unroll
      for (int j = 0; j < TPW; ++j) sacc[j] = (f32x16){};
#pragma unroll
      for (int c = 0; c < NDC; ++c) {
        const u32x4 kf = *(const u32x4*)(kc + (32 * s + l32) * KST + 16 * c + 8 * hh);
#pragma unroll
        for (int j = 0; j < TPW; ++j)
          if (act[j]) sacc[j] = E::mfma(qf[j][c], kf, sacc[j]);
      }
      const int key = kbs + l32;
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        if (!act[j]) continue;
        const bool need_mask = a.causal && kbs + 31 > q0[j];
        if (need_mask) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int qr = q0[j] + 8 * (i >> 2) + 4 * hh + (i & 3);
            const float x = fast_exp2(fmaf(sacc[j][i], a.scale_log2, -bias[j][i]));
            cs[s] += key > qr ? 0.f : x;
          }
        } else {
#pragma unroll
          for (int i = 0; i < 16; ++i) cs[s] += fast_exp2(fmaf(sacc[j][i], a.scale_log2, -bias[j][i]));
        }
      }
    }
    cs[0] = half_swap_sum(cs[0]);
    cs[1] = half_swap_sum(cs[1]);
    float* rb = red + cur * 4 * BN + wv * BN;
    if (hh == 0) {
      rb[l32] = cs[0];
      rb[32 + l32] = cs[1];
    }
    if (more) kstore(cur ^ 1, kr);
    __syncthreads();
    if (tid < BN) {
      const float* rr = red + cur * 4 * BN;
      const float sum = (rr[tid] + rr[BN + tid]) + (rr[2 * BN + tid] + rr[3 * BN + tid]);
      const int key = kb + tid;
      if (key < N && sum != 0.f) unsafeAtomicAdd(imp_row + key, sum);
    }
  }
}

// importance[b, j, n] *= sum_d |v[b, j, n, d]|; eight lanes per token row.
template <typename E>
__global__ __launch_bounds__(256) void value_l1_scale_kernel(const u16* v, long long vs0, long long vs1,
                                                             long long vs2, long long vs3, int Hkv, int N,
                                                             int D, int vec, float* imp, long long rows) {
  const long long row = (long long)blockIdx.x * 32 + (threadIdx.x >> 3);
  const int sub = threadIdx.x & 7;
  float s = 0.f, cur = 0.f;
  if (row < rows) {
    if (sub == 0) cur = imp[row];
    const long long bh = row / N;
    const int n = (int)(row - bh * N);
    const long long b = bh / Hkv, h = bh - b * Hkv;
    const u16* p = v + b * vs0 + h * vs1 + (long long)n * vs2;
    // channels 8*sub + 64*i (D <= 256): every load is issued before the first is used
    u32x4 w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d0 = 8 * sub + 64 * i;
      w[i] = d0 < D ? load8(p, vs3, d0, D, vec) : (u32x4){0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s += fabsf(E::to_f32((u16)(w[i][e] & 0xffffu)));
        s += fabsf(E::to_f32((u16)(w[i][e] >> 16)));
      }
  }
  s += __shfl_xor(s, 1);
  s += __shfl_xor(s, 2);
  s += __shfl_xor(s, 4);
  if (row < rows && sub == 0) imp[row] = cur * s;
}

// Zero n floats at p and nc 32-bit words at c (the work-item counters of the dynamic
// schedule), in one launch.
__global__ __launch_bounds__(256) void zero_f32_kernel(float* p, long long n, int* c, int nc) {
  const long long stride = (long long)gridDim.x * 256;
  const long long i0 = (long long)blockIdx.x * 256 + threadIdx.x;
  for (long long i = i0; i < n; i += stride) p[i] = 0.f;
  for (long long i = i0; i < nc; i += stride) c[i] = 0;
}

hipError_t launch_zero(float* p, int64_t n, int* ctr, int nctr, hipStream_t stream) {
  if (n <= 0 && nctr <= 0) return hipSuccess;
  long long blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(zero_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, p, (long long)(n > 0 ? n : 0), ctr,
                     nctr);
  return hipGetLastError();
}

hipError_t launch_zero_f32(float* p, int64_t n, hipStream_t stream) { return launch_zero(p, n, nullptr, 0, stream); }

// K or V rows that the fast kernels' tile DMA cannot read (rows off 16-byte alignment, a
// channel stride other than 1, a broadcast, a head dim not a multiple of 8), copied into the
// caller's workspace: out[b, h, n, 0:Dp) = x[b, h, n, 0:D) (element strides s0..s3, any
// alignment) and zero in D..Dp-1, Dp = D rounded up to 8, rows contiguous. One 16-byte chunk
// of eight channels per thread.
__global__ __launch_bounds__(256) void repack_rows_kernel(const u16* x, long long s0, long long s1, long long s2,
                                                          long long s3, int H, int N, int D, int Dp, u16* out,
                                                          long long chunks) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= chunks) return;
  const int cpr = Dp >> 3;
  const long long row = i / cpr;
  const int c = (int)(i - row * cpr);
  const long long bh = row / N;
  const int n = (int)(row - bh * N);
  const long long b = bh / H, h = bh - b * H;
  const u16* p = x + b * s0 + h * s1 + (long long)n * s2;
  *(u32x4*)(out + row * Dp + 8 * c) = load8(p, s3, 8 * c, D, 0);
}

hipError_t launch_repack(const u16* x, const int64_t* st, int64_t B, int64_t H, int64_t N, int64_t D, int64_t Dp,
                         u16* out, hipStream_t stream) {
  const long long chunks = (long long)(B * H * N) * (Dp / 8);
  const long long blocks = (chunks + 255) / 256;
  hipLaunchKernelGGL(repack_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, x, (long long)st[0],
                     (long long)st[1], (long long)st[2], (long long)st[3], (int)H, (int)N, (int)D, (int)Dp, out,
                     chunks);
  return hipGetLastError();
}

// Bytes of one repacked K or V area: B*Hkv*N rows of Dp = D rounded up to 8 channels, 256-byte
// aligned.
size_t repack_bytes(int64_t B, int64_t Hkv, int64_t N, int64_t D) {
  const size_t b = (size_t)(B * Hkv * N) * (size_t)((D + 7) / 8 * 8) * 2;
  return (b + 255) & ~(size_t)255;
}

namespace {

// Workgroups of a kernel that the device holds at once: the CU count times the kernel's
// occupancy, looked up once per device and kernel.
std::mutex g_res_mu;
std::vector<std::pair<std::pair<int, const void*>, int64_t>> g_res;   // ((device, kernel), workgroups)

hipError_t resident_blocks(const void* fn, int threads, size_t lds, hipStream_t stream, int64_t* out) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  if (stream) {
    hipDevice_t d = 0;
    if ((err = hipStreamGetDevice(stream, &d)) != hipSuccess) return err;
    dev = (int)d;
  }
  std::lock_guard<std::mutex> lock(g_res_mu);
  for (const auto& e : g_res)
    if (e.first.first == dev && e.first.second == fn) {
      *out = e.second;
      return hipSuccess;
    }
  int cus = 0, per_cu = 0;
  if ((err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return err;
  if ((err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, lds)) != hipSuccess) return err;
  const int64_t blocks = (int64_t)(cus > 0 ? cus : 1) * (per_cu > 0 ? per_cu : 1);
  g_res.push_back({{dev, fn}, blocks});
  *out = blocks;
  return hipSuccess;
}

}  // namespace


namespace {

typedef void (*FusedFn)(AttnArgs);

struct FusedEntry {
  FusedFn fn;
  size_t lds;
  const char* name;
};

template <typename E, int DP, int TPW>
FusedEntry make_entry(const char* name) {
  return FusedEntry{fused_attn_score_kernel<E, DP, TPW>, Tile<DP>::LDS, name};
}

// Padded channel counts: D is rounded up to the next entry.
constexpr int kDP[] = {32, 64, 96, 128, 160, 192, 224, 256};
constexpr int kNumDP = sizeof(kDP) / sizeof(kDP[0]);

std::vector<FusedEntry>& fused_table() {
  static std::vector<FusedEntry> t = {
      make_entry<F16, 32, 1>("fused_attn_score<f16,32,1>"),   make_entry<F16, 64, 1>("fused_attn_score<f16,64,1>"),
      make_entry<F16, 96, 1>("fused_attn_score<f16,96,1>"),   make_entry<F16, 128, 1>("fused_attn_score<f16,128,1>"),
      make_entry<F16, 160, 1>("fused_attn_score<f16,160,1>"), make_entry<F16, 192, 1>("fused_attn_score<f16,192,1>"),
      make_entry<F16, 224, 1>("fused_attn_score<f16,224,1>"), make_entry<F16, 256, 1>("fused_attn_score<f16,256,1>"),
      make_entry<BF16, 32, 1>("fused_attn_score<bf16,32,1>"),   make_entry<BF16, 64, 1>("fused_attn_score<bf16,64,1>"),
      make_entry<BF16, 96, 1>("fused_attn_score<bf16,96,1>"),   make_entry<BF16, 128, 1>("fused_attn_score<bf16,128,1>"),
      make_entry<BF16, 160, 1>("fused_attn_score<bf16,160,1>"), make_entry<BF16, 192, 1>("fused_attn_score<bf16,192,1>"),
      make_entry<BF16, 224, 1>("fused_attn_score<bf16,224,1>"), make_entry<BF16, 256, 1>("fused_attn_score<bf16,256,1>"),
  };
  return t;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int vec_ok(const void* p, const int64_t* st, int64_t D) {
  return st[3] == 1 && D % 8 == 0 && aligned16(p) && st[0] % 8 == 0 && st[1] % 8 == 0 && st[2] % 8 == 0;
}

}  // namespace

// The generic kernels take their LDS dynamically (up to 143 KiB at DP = 256), above the
// default dynamic limit: raise it for every kernel of the table, once per process, on first
// use (a function-local static, so the initialisation is thread-safe and nothing is mutated
// afterwards). The fast kernels use static LDS only and need nothing.
hipError_t prepare_plan(const FusedPlan& plan) {
  if (plan.lds == 0) return hipSuccess;
  static const hipError_t err = [] {
    for (const auto& e : fused_table()) {
      const hipError_t r =
          hipFuncSetAttribute((const void*)e.fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)e.lds);
      if (r != hipSuccess) return r;
    }
    return hipSuccess;
  }();
  return err;
}

void append_attn_resources(std::string& out) {
  append_fast_resources(out);
  for (auto& e : fused_table()) {
    hipFuncAttributes attr;
    if (hipFuncGetAttributes(&attr, (const void*)e.fn) != hipSuccess) continue;
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

using namespace fe;

extern "C" int fe_zero_f32(float* p, int64_t n, void* hip_stream) {
  clear_error();
  if (n < 0 || (n > 0 && p == nullptr)) {
    set_error("fe_zero_f32: invalid pointer or size");
    return FE_ERR_INVALID;
  }
  hipError_t err = launch_zero_f32(p, n, (hipStream_t)hip_stream);
  if (err != hipSuccess) {
    set_error(std::string("fe_zero_f32: ") + hipGetErrorString(err));
    return FE_ERR_HIP;
  }
  return FE_OK;
}

namespace fe {

// Body of fe_prefill / fe_prefill_ws. With a workspace of fe_prefill_workspace_bytes()
// bytes and the fast layouts, the replay runs as its own kernel (split schedule): the
// attention kernel leaves each row's replay bias in the workspace, and replay_fast_kernel
// runs the replay traversal at twice the occupancy. Otherwise one fused kernel does both.
// Query rows the replay must visit: the last `window` rows, less those whose recency weight
// is exactly zero in FP32. A row at distance t = N-1-q from the end has weight
// exp(-decay*t) (reference flash_evict/prefill.py:66, reference.py:19), which is below
// 2^-151 once decay*t >= 105 and rounds to 0 in FP32, so the row adds exactly nothing to any
// column; the replay's own term exp2(s*scale*log2e - b_q) is bounded by
// 2^(-decay*log2e*t) <= 2^-151.4 there and underflows to 0 as well. Rows with t < 105/decay
// are kept: ceil(105/decay) of them, or all `window` rows when that is fewer.
// Build option: -D FE_DYNAMIC_SCHEDULE=0 keeps the static schedule (item = workgroup index) even
// with the whole workspace (for A/B measurements).
#ifndef FE_DYNAMIC_SCHEDULE
#define FE_DYNAMIC_SCHEDULE 1
#endif

// Workgroups launched for `items` work items of a kernel that runs one item per workgroup
// under the dynamic schedule (the replay kernel): one eighth more, rounded up to the 8 XCDs
// the hardware deals workgroups over in turn, so that an XCD that runs faster than the others
// can start more than its eighth of them. The workgroups that find every item taken exit at
// once.
int64_t one_shot_grid(int64_t items) { return items + ((items / 8 + 7) & ~(int64_t)7); }

// Shares of a launch's work in the light parts of the dynamic schedule's queues (take_item in
// fe_attn_fast.hip): the lightest items, which other XCDs take before any heavy one once their
// own queues are empty, so that the XCDs' different speeds (several percent under these
// kernels) even out on small items at the end. Build options, for measurement.
#ifndef FE_TAIL_ATTN
#define FE_TAIL_ATTN 0.2
#endif
#ifndef FE_TAIL_REPLAY
#define FE_TAIL_REPLAY 0.0
#endif

// Rounds of resident workgroups up to which the small-grid attention kernel (fast_plan_small)
// stands in: for the 8-wave kernel at tile dims 32 and 64, and for the two-row-tile kernel at 96
// and 128. Build options, for measurement.
#ifndef FE_SMALL_GRID_ROUNDS
#define FE_SMALL_GRID_ROUNDS 1.0
#endif
#ifndef FE_SMALL_GRID_ROUNDS_RT2
#define FE_SMALL_GRID_ROUNDS_RT2 1.5
#endif

// Replay items in the two-row-tile attention launch (prefill_impl) for observation windows of at
// most this share of the rows. Build options, for measurement.
#ifndef FE_REPLAY_ITEMS
#define FE_REPLAY_ITEMS 1
#endif
#ifndef FE_REPLAY_ITEMS_MAX
#define FE_REPLAY_ITEMS_MAX 0.25
#endif
#ifndef FE_REPLAY_ITEMS_PER_WG
#define FE_REPLAY_ITEMS_PER_WG 2
#endif
// Key tiles a replay item holds at least (where the rows' keys allow).
#ifndef FE_SMALL_LAUNCH_ITEMS
#define FE_SMALL_LAUNCH_ITEMS 1
#endif
#ifndef FE_SMALL_LAUNCH_MAX_D
#define FE_SMALL_LAUNCH_MAX_D 128
#endif
// Tail replay items on fused_fast_kernel too (build option: the reference harness's shape at
// 32K 3% faster with them; D = 64 at the headline head counts within run-to-run drift).
#ifndef FE_TAIL_FAST
#define FE_TAIL_FAST 1
#endif
// Replay kernel key split in whole rounds of resident blocks for launches without the causal mask
// (build option).
#ifndef FE_REPLAY_ROUNDS_SPLIT
#define FE_REPLAY_ROUNDS_SPLIT 1
#endif
#ifndef FE_REPLAY_ITEM_MIN_TILES
#define FE_REPLAY_ITEM_MIN_TILES 8
#endif
#ifndef FE_REPLAY_ITEMS_FAST
#define FE_REPLAY_ITEMS_FAST 1
#endif
#ifndef FE_TAIL_REPLAY_FRAC
#define FE_TAIL_REPLAY_FRAC 0.03
#endif
#ifndef FE_COOP_LAUNCH
#define FE_COOP_LAUNCH 0
#endif

// Key tiles of the query rows of row tiles [.., t_end) of one (batch, KV head): causal rows see
// keys up to their own position.
int64_t item_key_tiles(int64_t t_end, int64_t G, int64_t N, bool causal) {
  const int64_t q_hi = ((t_end - 1) / G + 1) * 32;
  const int64_t kv_end = causal ? (q_hi < N ? q_hi : N) : N;
  return (kv_end + 63) / 64;
}

// First item of the queues' light parts. Items are numbered heaviest first in groups of BH (one
// per (batch, KV head), equal work within a group); the tail is the lightest groups holding at
// most `share` of the launch's work (work(g): of group g, in key tiles, plus two tiles of fixed
// cost per item), never starting below nstatic.
template <typename W>
int64_t tail_start(int64_t ngroups, int64_t BH, int64_t nstatic, double share, W work) {
  const int64_t nitems = ngroups * BH;
  if (!(share > 0.0)) return nitems;
  double total = 0.0;
  for (int64_t g = 0; g < ngroups; ++g) total += (double)(work(g) + 2);
  double acc = 0.0;
  int64_t g = ngroups;
  while (g > 0 && acc + (double)(work(g - 1) + 2) <= share * total) acc += (double)(work(--g) + 2);
  const int64_t t = g * BH;
  return t < nstatic ? nstatic : t;
}

int64_t replay_rows(int64_t N, int64_t window, float recency_decay) {
  if (!(recency_decay > 0.f)) return window;
  const double span = ceil(105.0 / (double)recency_decay);
  return span < (double)window ? (int64_t)span : window;
}

// Kernels of the calling thread's last prefill launch (fe_last_plan).
thread_local std::string g_last_plan;

static int prefill_impl(const void* q, const void* k, const void* v, void* out, float* importance, int64_t B,
                        int64_t Hq, int64_t Hkv, int64_t N, int64_t D, const int64_t* q_strides,
                        const int64_t* k_strides, const int64_t* v_strides, int dtype, float scale, int causal,
                        int value_weighted, int score, float recency_decay, int64_t window, void* workspace,
                        size_t workspace_bytes, void* hip_stream, bool allow_timing = true) {
  if (!q || !k || !v || !out || !q_strides || !k_strides || !v_strides || (score && !importance)) {
    set_error("fe_prefill: null pointer argument");
    return FE_ERR_INVALID;
  }
  if (B < 1 || Hq < 1 || Hkv < 1 || N < 1 || D < 1 || Hq % Hkv != 0) {
    set_error("fe_prefill: expected nonempty shapes with Hq divisible by Hkv");
    return FE_ERR_INVALID;
  }
  if (D > 256) {
    set_error("fe_prefill: head dimension must be <= 256");
    return FE_ERR_INVALID;
  }
  if (dtype != FE_DTYPE_F16 && dtype != FE_DTYPE_BF16) {
    set_error("fe_prefill: dtype must be FE_DTYPE_F16 or FE_DTYPE_BF16");
    return FE_ERR_INVALID;
  }
  if (!isfinite(scale) || !isfinite(recency_decay) || recency_decay < 0.f) {
    set_error("fe_prefill: scale must be finite and recency_decay finite and nonnegative");
    return FE_ERR_INVALID;
  }
  if (window < 1 || window > N) {
    set_error("fe_prefill: window must be the clamped observation window in [1, N]");
    return FE_ERR_INVALID;
  }
  const int64_t G = Hq / Hkv;
  const int64_t nqs = (N + 31) / 32;
  const int64_t tiles_bh = G * nqs;
  const int64_t wg_bh = (tiles_bh + 3) / 4;   // the most workgroups any plan uses
  const int64_t blocks = B * Hkv * wg_bh;
  if (N > (1LL << 30) || tiles_bh > (1LL << 30) || blocks > 0x7fffffffLL || B * Hkv > (1LL << 30)) {
    set_error("fe_prefill: problem too large for one launch");
    return FE_ERR_UNSUPPORTED;
  }

  AttnArgs a;
  a.q = (const u16*)q;
  a.k = (const u16*)k;
  a.v = (const u16*)v;
  a.out = (u16*)out;
  a.imp = importance;
  a.bias = nullptr;
  a.rsplit = 1;
  a.queue = nullptr;
  a.nitems = 0;
  a.nstatic = 0;
  a.tail = 0;
  a.nattn = 0x7fffffff;
  a.rwg0 = -1;
  a.done = nullptr;
  // Polls of a replay item's dependency before it runs the attention item itself: 4096 plus 64
  // per key tile (each poll sleeps about 0.27 us). FLASH_EVICT_REPLAY_WAIT=0 makes every replay
  // item run its dependency at once (tests of that path).
  {
    const char* w = getenv("FLASH_EVICT_REPLAY_WAIT");
    const bool none = w && w[0] == '0' && w[1] == 0;
    a.wait_base = none ? 0 : 4096;
    a.wait_per_tile = none ? 0 : 64;
  }
  for (int i = 0; i < 4; ++i) {
    a.qs[i] = q_strides[i];
    a.ks[i] = k_strides[i];
    a.vs[i] = v_strides[i];
  }
  a.N = (int)N;
  a.D = (int)D;
  a.Dq = (int)D;
  a.qmask = 0xffffffffu;
  a.G = (int)G;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.BH = (int)(B * Hkv);
  a.tiles_bh = (int)tiles_bh;
  a.wg_bh = (int)wg_bh;
  const double log2e = 1.4426950408889634;
  a.scale_log2 = (float)((double)scale * log2e);
  a.abs_scale_log2 = fabsf(a.scale_log2);
  a.neg_scale = a.scale_log2 < 0.f;
  a.decay_log2 = (float)((double)recency_decay * log2e);
  a.causal = causal ? 1 : 0;
  a.score = score ? 1 : 0;
  a.win_lo = (int)(N - replay_rows(N, window, recency_decay));
  a.qvec = vec_ok(q, q_strides, D);
  a.kvec = vec_ok(k, k_strides, D);
  a.vvec = vec_ok(v, v_strides, D);
  a.ovec = (D % 4 == 0) && (((uintptr_t)out & 7u) == 0);

  FusedPlan plan;
  ReplayPlan rplan;
  // Workspace: the replay bias of every query row (scoring calls), then the dynamic
  // schedule's item counters at the next 256-byte boundary, then (K/V layouts the fast kernels
  // cannot read) the repacked K and V.
  const size_t ws_bias = score ? (size_t)(B * Hq * N) * sizeof(float) : 0;
  const size_t ws_ctr = (ws_bias + 255) & ~(size_t)255;
  const size_t ws_kv = ws_ctr + kQueueBytes, kv_bytes = repack_bytes(B, Hkv, N, D);
  const bool repack = !fast_layout(a) && workspace && workspace_bytes >= ws_kv + 2 * kv_bytes;
  if (repack) {
    const int64_t Dp = (D + 7) / 8 * 8;
    AttnArgs r = a;
    r.k = (const u16*)((char*)workspace + ws_kv);
    r.v = (const u16*)((char*)workspace + ws_kv + kv_bytes);
    const long long st[4] = {(long long)(Hkv * N * Dp), (long long)(N * Dp), (long long)Dp, 1};
    for (int i = 0; i < 4; ++i) r.ks[i] = r.vs[i] = st[i];
    r.D = (int)Dp;
    r.kvec = r.vvec = 1;
    if (fast_layout(r)) a = r;
  }
  // A zero scale runs on the fast kernels with Q zeroed at load: every logit is then exactly
  // 0 (the reference's 0 * (q.k) for finite q.k), and masked keys stay at -inf.
  if (!(a.abs_scale_log2 > 0.f)) {
    AttnArgs z = a;
    z.qmask = 0;
    z.abs_scale_log2 = 1.f;
    if (fast_plan(z, dtype, plan)) a = z;
  }
  const bool split = score && workspace && workspace_bytes >= ws_bias && replay_plan(a, dtype, rplan);
  if (split) a.bias = (float*)workspace;
  bool fast = fast_plan(a, dtype, plan);
  if (!fast) {
    int dpi = 0;
    while (dpi < kNumDP - 1 && kDP[dpi] < D) ++dpi;
    const FusedEntry& ent = fused_table()[(dtype == FE_DTYPE_BF16 ? kNumDP : 0) + dpi];
    plan = FusedPlan{(const void*)ent.fn, ent.lds, 4, 4, ent.name};
  }
  hipStream_t stream = (hipStream_t)hip_stream;
  // Small grids at tile dims 32 and 64: where the 8-wave attention kernel's work items would
  // fill at most FE_SMALL_GRID_ROUNDS rounds of its resident workgroups, the 4-wave kernel
  // (twice the items, four workgroups per CU) fills the chip better.
  // At tile dims 96 and 128, where the two-row-tile kernel's 16-row-tile items would fill at most
  // FE_SMALL_GRID_ROUNDS_RT2 (1.5) rounds of its workgroups (one per CU), the 4-wave kernel (four
  // row tiles per item, two workgroups per CU): 3-12.5% faster at 1.2-1.5 rounds, 2-8% slower at
  // 1.7-1.8 rounds, 12% slower at 2 (llama8k).
  FusedPlan small;
  if (fast && (plan.rows == 8 || plan.rows == 16) && fast_plan_small(a, dtype, small)) {
    int64_t res = 0;
    const double rounds = plan.rows == 8 ? FE_SMALL_GRID_ROUNDS : FE_SMALL_GRID_ROUNDS_RT2;
    if (resident_blocks(plan.fn, 64 * plan.waves, plan.lds, stream, &res) == hipSuccess &&
        (double)(B * Hkv * ((tiles_bh + plan.rows - 1) / plan.rows)) <= rounds * (double)res)
      plan = small;
  }
  // Dynamic schedule (fast attention-only kernels, and the replay kernel): needs the
  // counters, i.e. the whole workspace of fe_prefill_workspace_bytes.
  int* ctr = nullptr;
  if (FE_DYNAMIC_SCHEDULE && fast && (split || !score) && workspace && workspace_bytes >= ws_ctr + kQueueBytes)
    ctr = (int*)((char*)workspace + ws_ctr);
  // Workgroups are sized by the plan's row tiles per workgroup.
  a.wg_bh = (int)((tiles_bh + plan.rows - 1) / plan.rows);
  const int64_t items = B * Hkv * (int64_t)a.wg_bh;
  int64_t grid = items;

  hipError_t err = prepare_plan(plan);
  if (err != hipSuccess) {
    set_error(std::string("fe_prefill: hipFuncSetAttribute: ") + hipGetErrorString(err));
    return FE_ERR_HIP;
  }
  int64_t resident = 0;
  if (ctr) {
    if ((err = resident_blocks(plan.fn, 64 * plan.waves, plan.lds, stream, &resident)) != hipSuccess) {
      set_error(std::string("fe_prefill: occupancy query: ") + hipGetErrorString(err));
      return FE_ERR_HIP;
    }
    a.queue = ctr;
    a.nitems = (int)items;
    a.nstatic = (int)(items < resident ? items : resident);
    const int64_t rows = plan.rows, wgb = a.wg_bh;
    a.tail = (int)tail_start(wgb, B * Hkv, a.nstatic, FE_TAIL_ATTN, [&](int64_t g) {
      const int64_t wg = wgb - 1 - g;
      const int64_t t_end = (wg + 1) * rows < tiles_bh ? (wg + 1) * rows : tiles_bh;
      return item_key_tiles(t_end, G, N, causal != 0);
    });
    grid = a.nstatic;
  }
  // Replay items: the replay runs as work items of the attention launch, numbered after its
  // attention items (so in every XCD queue they follow them), each waiting for its rows' attention
  // item to publish their biases (a bit per attention item after the counters), or running that
  // item itself if the wait runs out. Item = (batch and KV head, row group of the attention
  // kernel's row tiles holding window rows, key range): key ranges chosen for about two items per
  // resident workgroup (four measured 1.3% slower at llama8k), of at least
  // FE_REPLAY_ITEM_MIN_TILES key tiles where the keys allow (a window of 128 rows at N = 32K
  // otherwise made items of two tiles, 0.4% slower overall).
  bool replay_items = false;
  // Causal launches at tile dims up to 128 whose attention items do not fill the resident
  // workgroups: a grid of every resident workgroup, and all the replay as items in ascending row
  // groups, so the light rows' replay (their attention items end first) runs beside the heaviest
  // attention items on CUs that would idle, and the replay kernel's launch after the heaviest
  // item goes (the reference harness's shape at 8K: 8% faster; B1 Hq8/Hkv2 N4000 D128: 8.6%).
  // Without the causal mask every attention item ends at once (the same shape non-causal, B2:
  // 13% slower).
  if (FE_REPLAY_ITEMS && FE_SMALL_LAUNCH_ITEMS && split && ctr && fast && causal && D <= FE_SMALL_LAUNCH_MAX_D &&
      plan.rows <= 8 && items < resident && items <= kMaxDoneItems) {
    const int64_t wg_lo = ((int64_t)(a.win_lo / 32) * G) / plan.rows;
    const int64_t nwg = B * Hkv * ((int64_t)a.wg_bh - wg_lo);
    const int64_t max_tiles = (N + 63) / 64;
    const int64_t rs_max = (max_tiles + FE_REPLAY_ITEM_MIN_TILES - 1) / FE_REPLAY_ITEM_MIN_TILES;
    int64_t rs = nwg > 0 ? (FE_REPLAY_ITEMS_PER_WG * resident + nwg - 1) / nwg : 1;
    rs = rs < 1 ? 1 : (rs > rs_max ? rs_max : rs);
    if (nwg > 0 && items + nwg * rs < (int64_t)0x7fffffff) {
      replay_items = true;
      a.nattn = (int)items;
      a.nitems = (int)(items + nwg * rs);
      a.rsplit = (int)rs;
      a.rwg0 = (int)wg_lo;
      a.done = (unsigned*)(ctr + kQueueDone);
      a.nstatic = (int)((int64_t)a.nitems < resident ? (int64_t)a.nitems : resident);
      if (a.tail < a.nstatic) a.tail = a.nstatic;
      grid = a.nstatic;
    }
  }
  // Replay items run on the two-row-tile kernel and on fused_fast_kernel at tile dims 32 and 64
  // (FE_REPLAY_ITEMS_FAST; D = 32 and 64 short windows and the reference harness's shape at 32K
  // 2-3.5% faster, tile dim 256 7.5% slower), in launches whose attention items fill every resident
  // workgroup: a smaller launch runs one workgroup per item, so its replay items would queue
  // behind the attention items on those workgroups while the replay kernel spreads over the whole
  // chip (the reference harness's shape at 8K: 5.8% slower).
  const bool item_plan = fast && (plan.rows == 16 || (FE_REPLAY_ITEMS_FAST && plan.rows <= 8 && D <= 64)) &&
                         items >= resident;
  // Short observation windows (at most FE_REPLAY_ITEMS_MAX of the rows replayed): all the replay
  // as items, heaviest rows first. They fill the end of the attention launch, where the replay
  // kernel would start only once the last attention item is done.
  if (FE_REPLAY_ITEMS && !replay_items && split && ctr && item_plan && items <= kMaxDoneItems &&
      (double)(N - a.win_lo) <= FE_REPLAY_ITEMS_MAX * (double)N) {
    const int64_t wg_lo = ((int64_t)(a.win_lo / 32) * G) / plan.rows;
    const int64_t nwg = B * Hkv * ((int64_t)a.wg_bh - wg_lo);
    const int64_t max_tiles = (N + 63) / 64;
    const int64_t rs_max = (max_tiles + FE_REPLAY_ITEM_MIN_TILES - 1) / FE_REPLAY_ITEM_MIN_TILES;
    int64_t rs = (FE_REPLAY_ITEMS_PER_WG * (int64_t)a.nstatic + nwg - 1) / nwg;
    rs = rs < 1 ? 1 : (rs > rs_max ? rs_max : rs);
    if (items + nwg * rs < (int64_t)0x7fffffff) {
      replay_items = true;
      a.nattn = (int)items;
      a.nitems = (int)(items + nwg * rs);
      a.rsplit = (int)rs;
      a.done = (unsigned*)(ctr + kQueueDone);
    }
  }
  // Longer windows: the heaviest FE_TAIL_REPLAY_FRAC (3%) of the row groups of each (batch, KV
  // head) replay as items of the attention launch, where they fill its tail (their attention
  // items are the first taken, so the biases are ready when they start); the replay kernel
  // replays the rows below them (every row replayed: 0.2-1.4% faster pairs; 6% was slower).
  int64_t tail_groups = 0;
  if (FE_TAIL_REPLAY_FRAC > 0.0 && !replay_items && FE_REPLAY_ITEMS && split && ctr && item_plan &&
      (FE_TAIL_FAST || plan.rows == 16) && items <= kMaxDoneItems) {
    const int64_t wg_lo = ((int64_t)(a.win_lo / 32) * G) / plan.rows;
    const int64_t ng_max = (int64_t)a.wg_bh - wg_lo - 1;
    int64_t ng = (int64_t)ceil(FE_TAIL_REPLAY_FRAC * (double)((int64_t)a.wg_bh - wg_lo));
    // the replay kernel's rows end on a boundary of its own row groups
    while (ng < ng_max && (((int64_t)a.wg_bh - ng) * plan.rows) % rplan.rows != 0) ++ng;
    if (ng > 0 && ng <= ng_max && (((int64_t)a.wg_bh - ng) * plan.rows) % rplan.rows == 0) {
      const int64_t nwg = B * Hkv * ng;
      const int64_t max_tiles = (N + 63) / 64;
      const int64_t rs_max = (max_tiles + FE_REPLAY_ITEM_MIN_TILES - 1) / FE_REPLAY_ITEM_MIN_TILES;
      int64_t rs = (FE_REPLAY_ITEMS_PER_WG * (int64_t)a.nstatic + nwg - 1) / nwg;
      rs = rs < 1 ? 1 : (rs > rs_max ? rs_max : rs);
      if (items + nwg * rs < (int64_t)0x7fffffff) {
        replay_items = true;
        tail_groups = ng;
        a.nattn = (int)items;
        a.nitems = (int)(items + nwg * rs);
        a.rsplit = (int)rs;
        a.done = (unsigned*)(ctr + kQueueDone);
      }
    }
  }
  if (score || ctr) {
    err = launch_zero(score ? importance : nullptr, score ? B * Hkv * N : 0, ctr, ctr ? kQueueWords : 0, stream);
    if (err != hipSuccess) {
      set_error(std::string("fe_prefill: zero-init launch: ") + hipGetErrorString(err));
      return FE_ERR_HIP;
    }
  }
  if (a.k != (const u16*)k) {
    err = launch_repack((const u16*)k, k_strides, B, Hkv, N, D, a.D, (u16*)a.k, stream);
    if (err == hipSuccess) err = launch_repack((const u16*)v, v_strides, B, Hkv, N, D, a.D, (u16*)a.v, stream);
    if (err != hipSuccess) {
      set_error(std::string("fe_prefill: K/V repack launch: ") + hipGetErrorString(err));
      return FE_ERR_HIP;
    }
  }
  // Optional timing of the attention (+ replay) kernels on the caller's stream: the event
  // pair goes to the calling thread's record once both events are recorded, and is
  // destroyed on every earlier return.
  struct EventPair {
    hipEvent_t e[2] = {nullptr, nullptr};
    ~EventPair() {
      for (hipEvent_t x : e)
        if (x) (void)hipEventDestroy(x);
    }
  } ev;
  const bool timed = allow_timing && fused_timing_enabled();
  if (timed) {
    if (hipEventCreate(&ev.e[0]) != hipSuccess || hipEventCreate(&ev.e[1]) != hipSuccess ||
        hipEventRecord(ev.e[0], stream) != hipSuccess) {
      set_error("fe_prefill: timing event setup failed");
      return FE_ERR_HIP;
    }
  }
  g_last_plan = replay_items ? std::string(plan.name) + " with replay items" + (tail_groups ? std::string(" + ") + rplan.name : std::string())
                : (split ? std::string(plan.name) + " + " + rplan.name : std::string(plan.name));
  void* kargs[] = {&a};
  if (replay_items && FE_COOP_LAUNCH) {
    // a cooperative launch fails rather than start with some workgroups not resident, which the
    // replay items' waits need; on failure the call runs the replay kernel instead
    err = hipLaunchCooperativeKernel(plan.fn, dim3((unsigned)grid), dim3(64 * plan.waves), kargs, (unsigned)plan.lds,
                                     stream);
    if (err != hipSuccess) {
      (void)hipGetLastError();
      replay_items = false;
      tail_groups = 0;
      a.rwg0 = -1;
      a.nattn = 0x7fffffff;
      a.nitems = (int)items;
      a.rsplit = 1;
      a.done = nullptr;
      g_last_plan = std::string(plan.name) + " + " + rplan.name;
      err = hipLaunchKernel(plan.fn, dim3((unsigned)grid), dim3(64 * plan.waves), kargs, plan.lds, stream);
    }
  } else {
    err = hipLaunchKernel(plan.fn, dim3((unsigned)grid), dim3(64 * plan.waves), kargs, plan.lds, stream);
  }
  if (err != hipSuccess) {
    set_error(std::string("fe_prefill: fused kernel launch: ") + hipGetErrorString(err));
    return FE_ERR_HIP;
  }
  if (split && (!replay_items || tail_groups)) {
    // Workgroups of rplan.rows row tiles; only those holding window rows are launched
    // (tiles before query block win_lo/32 have none), heaviest first; with tail groups, only
    // the row tiles below them.
    AttnArgs r = a;
    r.wg_bh = tail_groups ? (int)((((int64_t)a.wg_bh - tail_groups) * plan.rows) / rplan.rows)
                          : (int)((tiles_bh + rplan.rows - 1) / rplan.rows);
    const int64_t wg_lo = ((int64_t)(a.win_lo / 32) * G) / rplan.rows;
    const int64_t nwg = B * Hkv * ((int64_t)r.wg_bh - wg_lo);
    // Split the keys of each workgroup when there are too few workgroups to fill the chip
    // (short observation windows): about 1024 blocks, at least one key tile per split.
    const int64_t max_tiles = (N + 63) / 64;
    int64_t rs = (1024 + nwg - 1) / nwg;
    rs = rs < 1 ? 1 : (rs > max_tiles ? max_tiles : rs);
    int64_t rresident = 0;
    if ((err = resident_blocks(rplan.fn, 64 * rplan.waves, 0, stream, &rresident)) != hipSuccess) {
      set_error(std::string("fe_prefill: occupancy query: ") + hipGetErrorString(err));
      return FE_ERR_HIP;
    }
    if (FE_REPLAY_ROUNDS_SPLIT && !causal && nwg > 0 && rresident > 0) {
      // Without the causal mask every block of a split holds the same key tiles, so the launch
      // takes whole rounds of resident blocks: choose the split with the fewest key tiles per
      // resident slot, rounds x (tiles per block + one tile of per-block set-up), the smaller split
      // on a tie (B2 Hkv2 N4000: 252 row groups x 3 = 756 blocks in one round of 21 key tiles,
      // instead of x 5 = 1260 blocks in two rounds of 13).
      int64_t best = -1;
      for (int64_t s = 1; s <= max_tiles && (s - 1) * nwg <= 4 * rresident; ++s) {
        const int64_t rounds = (nwg * s + rresident - 1) / rresident;
        const int64_t cost = rounds * ((max_tiles + s - 1) / s + 1);
        if (best < 0 || cost < best) {
          best = cost;
          rs = s;
        }
      }
    }
    r.rsplit = (int)rs;
    int64_t rgrid = nwg * rs;
    if (ctr) {
      r.queue = ctr + kQueueReplay;
      r.nitems = (int)rgrid;
      r.nstatic = (int)(rgrid < rresident ? rgrid : rresident);
      const int64_t rrows = rplan.rows, rwgb = r.wg_bh;
      r.tail = (int)tail_start(rgrid / (B * Hkv), B * Hkv, r.nstatic, FE_TAIL_REPLAY, [&](int64_t g) {
        const int64_t ks = g % rs, wg = rwgb - 1 - g / rs;
        const int64_t t_end = (wg + 1) * rrows < tiles_bh ? (wg + 1) * rrows : tiles_bh;
        const int64_t all = item_key_tiles(t_end, G, N, causal != 0), per = (all + rs - 1) / rs;
        const int64_t lo = ks * per, hi = lo + per < all ? lo + per : all;
        return hi > lo ? hi - lo : (int64_t)0;
      });
      rgrid = one_shot_grid(rgrid);
    }
    void* rargs[] = {&r};
    err = hipLaunchKernel(rplan.fn, dim3((unsigned)rgrid), dim3(64 * rplan.waves), rargs, 0, stream);
    if (err != hipSuccess) {
      set_error(std::string("fe_prefill: replay kernel launch: ") + hipGetErrorString(err));
      return FE_ERR_HIP;
    }
  }
  if (timed) {
    if (hipEventRecord(ev.e[1], stream) != hipSuccess) {
      set_error("fe_prefill: timing event record failed");
      return FE_ERR_HIP;
    }
    fused_timing_push(ev.e[0], ev.e[1]);
    ev.e[0] = ev.e[1] = nullptr;
  }
  if (score && value_weighted) {
    // the caller's V (a repacked copy may be what the attention kernels read)
    const int vvec = vec_ok(v, v_strides, D);
    const long long rows = B * Hkv * N;
    const long long nb = (rows + 31) / 32;
    if (dtype == FE_DTYPE_BF16)
      hipLaunchKernelGGL(value_l1_scale_kernel<BF16>, dim3((unsigned)nb), dim3(256), 0, stream, (const u16*)v,
                         (long long)v_strides[0], (long long)v_strides[1], (long long)v_strides[2],
                         (long long)v_strides[3], (int)Hkv, (int)N, (int)D, vvec, importance, rows);
    else
      hipLaunchKernelGGL(value_l1_scale_kernel<F16>, dim3((unsigned)nb), dim3(256), 0, stream, (const u16*)v,
                         (long long)v_strides[0], (long long)v_strides[1], (long long)v_strides[2],
                         (long long)v_strides[3], (int)Hkv, (int)N, (int)D, vvec, importance, rows);
    err = hipGetLastError();
    if (err != hipSuccess) {
      set_error(std::string("fe_prefill: value-norm launch: ") + hipGetErrorString(err));
      return FE_ERR_HIP;
    }
  }
  return FE_OK;
}

}  // namespace fe

extern "C" int fe_prefill(const void* q, const void* k, const void* v, void* out, float* importance, int64_t B,
                          int64_t Hq, int64_t Hkv, int64_t N, int64_t D, const int64_t* q_strides,
                          const int64_t* k_strides, const int64_t* v_strides, int dtype, float scale, int causal,
                          int value_weighted, int score, float recency_decay, int64_t window, void* hip_stream) {
  clear_error();
  return prefill_impl(q, k, v, out, importance, B, Hq, Hkv, N, D, q_strides, k_strides, v_strides, dtype, scale,
                      causal, value_weighted, score, recency_decay, window, nullptr, 0, hip_stream);
}

extern "C" int fe_last_plan(char* buf, size_t cap) {
  clear_error();
  const std::string& s = fe::g_last_plan;
  if (!buf || cap < s.size() + 1) {
    set_error("fe_last_plan: buffer too small; need " + std::to_string(s.size() + 1) + " bytes");
    return FE_ERR_INVALID;
  }
  memcpy(buf, s.c_str(), s.size() + 1);
  return FE_OK;
}

extern "C" int64_t fe_replay_rows(int64_t N, int64_t window, float recency_decay) {
  if (N < 1 || window < 1 || window > N || !isfinite(recency_decay) || recency_decay < 0.f) return -1;
  return replay_rows(N, window, recency_decay);
}

extern "C" size_t fe_prefill_workspace_bytes(int64_t B, int64_t Hq, int64_t N, int score) {
  if (B < 1 || Hq < 1 || N < 1) return 0;
  const size_t bias = score ? (size_t)(B * Hq * N) * sizeof(float) : 0;
  return ((bias + 255) & ~(size_t)255) + kQueueBytes;
}

extern "C" size_t fe_prefill_workspace_bytes_kv(int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D, int score,
                                                const void* k, const int64_t* k_strides, const void* v,
                                                const int64_t* v_strides) {
  const size_t base = fe_prefill_workspace_bytes(B, Hq, N, score);
  if (base == 0 || Hkv < 1 || D < 1 || D > 256 || !k || !v || !k_strides || !v_strides || N > (1LL << 30)) return base;
  AttnArgs a = {};
  a.k = (const u16*)k;
  a.v = (const u16*)v;
  for (int i = 0; i < 4; ++i) {
    a.ks[i] = k_strides[i];
    a.vs[i] = v_strides[i];
  }
  a.N = (int)N;
  a.D = (int)D;
  if (fast_layout(a)) return base;
  return base + 2 * repack_bytes(B, Hkv, N, D);
}

extern "C" int fe_prefill_ws(const void* q, const void* k, const void* v, void* out, float* importance, int64_t B,
                             int64_t Hq, int64_t Hkv, int64_t N, int64_t D, const int64_t* q_strides,
                             const int64_t* k_strides, const int64_t* v_strides, int dtype, float scale, int causal,
                             int value_weighted, int score, float recency_decay, int64_t window, void* workspace,
                             size_t workspace_bytes, void* hip_stream) {
  clear_error();
  return prefill_impl(q, k, v, out, importance, B, Hq, Hkv, N, D, q_strides, k_strides, v_strides, dtype, scale,
                      causal, value_weighted, score, recency_decay, window, workspace, workspace_bytes, hip_stream);
}

extern "C" int fe_prefill_static(const void* q, const void* k, const void* v, void* out, float* importance,
                                 int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                                 const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                                 int dtype, float scale, int causal, int value_weighted, int score,
                                 float recency_decay, int64_t window, void* hip_stream) {
  clear_error();
  float* ws = nullptr;
  size_t ws_bytes = 0;
  if (B >= 1 && Hq >= 1 && N >= 1) {
    const int64_t R = FE_STATIC_BIAS_ROWS;
    if (score && (B > R || Hq > R || N > R || B * Hq > R || B * Hq * N > R)) {
      char msg[256];
      snprintf(msg, sizeof(msg),
               "fe_prefill_static: B*Hq*N = %.0f query rows exceed the static replay-bias buffer of %lld rows; "
               "use fe_prefill_ws with a workspace",
               (double)B * (double)Hq * (double)N, (long long)R);
      set_error(msg);
      return FE_ERR_WORKSPACE;
    }
    const hipError_t err = fe::static_scratch((hipStream_t)hip_stream, &ws);
    if (err != hipSuccess) {
      set_error(std::string("fe_prefill_static: static buffer lookup: ") + hipGetErrorString(err));
      return FE_ERR_HIP;
    }
    ws_bytes = fe_prefill_workspace_bytes(B, Hq, N, score);
  }
  return prefill_impl(q, k, v, out, importance, B, Hq, Hkv, N, D, q_strides, k_strides, v_strides, dtype, scale,
                      causal, value_weighted, score, recency_decay, window, ws, ws_bytes, hip_stream,
                      /*allow_timing=*/false);
}
