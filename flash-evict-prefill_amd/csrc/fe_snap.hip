// SnapKV observation-window scores for gfx950 (the baseline path of the reference,
// flash_evict/baselines.py:15-25, `snap_scores`):
//
//   W = min(window, N); the last W query positions of every query head observe all keys
//   logits = (q[:, :, -W:] @ repeat_interleave(k, G)^T) in the input dtype     (:21)
//   logits = float(logits) * D^-0.5, causal mask key > query position -> -inf   (:22-25)
//   p = softmax(logits) in FP32; scores[b, j, n] = mean over the G heads of group j of
//   sum over the W window rows of p                                               (:26-27)
//
// The dot products accumulate in FP32 on MFMA and are rounded to the input dtype before
// the FP32 softmax, as the native-dtype matmul of the reference does. Three kernels:
//   snap_stats_kernel    per (b, kv head, 32-row tile, key split): partial row max and
//                        sum of exponentials over the split's keys (lanes hold rows)
//   snap_combine_kernel  per row: merges the splits into the row max and 1/sum
//   snap_scores_kernel   per (b, kv head, 64 keys): every window row of the group, p
//                        summed over rows in-lane (lanes hold keys), / G, one store per key
// No atomics: every score is written once, in a fixed summation order.
#include <math.h>
#include <string>

#include "fe_attn.h"
#include "fe_internal.h"
#include "../../include/flash_evict.h"

namespace fe {

struct SnapArgs {
  const u16* q;
  const u16* k;
  float* scores;
  float2* part;          // [BH][RT][S][32] (max, sum) partials
  float2* stats;         // [BH][RT][32] (max, 1/sum)
  long long qs[4], ks[4];
  int N, D, G, Hkv, BH;
  int W, R, RT;          // window rows per head, rows per group (G*W), 32-row tiles
  int S, tiles_per_split, ntiles;
  float scale;           // D^-0.5 as float
};

// Row r of a group: head g = r / W of the group, query position N - W + r % W.
__device__ __forceinline__ void snap_row(const SnapArgs& a, int hkv, int r, int& head, int& qpos) {
  const int g = r / a.W;
  head = hkv * a.G + g;
  qpos = a.N - a.W + (r - g * a.W);
}

template <typename E>
__device__ __forceinline__ float round_logit(float acc) {
  return E::to_f32((unsigned short)(E::pack2(acc, 0.f) & 0xffffu));
}

template <typename E, int DP, int VEC>
__global__ __launch_bounds__(64) void snap_stats_kernel(const SnapArgs a) {
  constexpr int NDC = DP / 16;
  constexpr float NEG_INF = -__builtin_huge_valf();
  const int lane = threadIdx.x, l32 = lane & 31, hh = lane >> 5;
  const int s_idx = (int)(blockIdx.x % (unsigned)a.S);
  const int rest = (int)(blockIdx.x / (unsigned)a.S);
  const int rt = rest % a.RT, bh = rest / a.RT;
  const int b = bh / a.Hkv, hkv = bh - b * a.Hkv;
  const int r = rt * 32 + l32;
  const bool row_ok = r < a.R;
  int head = 0, qpos = -1;
  if (row_ok) snap_row(a, hkv, r, head, qpos);

  // Q fragments (B operand): query row r, channels 16c + 8h .. +7
  u32x4 qf[NDC];
  const u16* qrow = a.q + b * a.qs[0] + head * a.qs[1] + (long long)(row_ok ? qpos : 0) * a.qs[2];
#pragma unroll
  for (int c = 0; c < NDC; ++c)
    qf[c] = row_ok ? load8(qrow, a.qs[3], 16 * c + 8 * hh, a.D, VEC) : (u32x4){0u, 0u, 0u, 0u};
  const u16* kbase = a.k + b * a.ks[0] + hkv * a.ks[1];

  float m = NEG_INF, l = 0.f;
  const int t_lo = s_idx * a.tiles_per_split;
  const int t_hi = min(a.ntiles, t_lo + a.tiles_per_split);
  for (int t = t_lo; t < t_hi; ++t) {
    const int kb = t * 64;
    f32x16 sacc[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int key = kb + 32 * s + l32;
      const bool kok = key < a.N;
      const u16* krow = kbase + (long long)(kok ? key : 0) * a.ks[2];
      sacc[s] = (f32x16){};
#pragma unroll
      for (int c = 0; c < NDC; ++c) {
        const u32x4 kf = kok ? load8(krow, a.ks[3], 16 * c + 8 * hh, a.D, VEC) : (u32x4){0u, 0u, 0u, 0u};
        sacc[s] = E::mfma(kf, qf[c], sacc[s]);
      }
    }
    // lanes hold query row r; register i of half s holds key kb + 32s + 8(i/4) + 4h + i%4
    float x[2][16];
    float tmax = NEG_INF;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kb + 32 * s + 8 * (i >> 2) + 4 * hh + (i & 3);
        const float v = round_logit<E>(sacc[s][i]) * a.scale;
        x[s][i] = key <= qpos ? v : NEG_INF;
        tmax = fmaxf(tmax, x[s][i]);
      }
    tmax = half_swap_max(tmax);
    const float mn = fmaxf(m, tmax);
    if (mn != NEG_INF) {
      float sum = 0.f;
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int i = 0; i < 16; ++i) sum += expf(x[s][i] - mn);
      l = l * expf(m - mn) + half_swap_sum(sum);
      m = mn;
    }
  }
  if (hh == 0) a.part[((long long)(bh * a.RT + rt) * a.S + s_idx) * 32 + l32] = make_float2(m, l);
}

__global__ __launch_bounds__(256) void snap_combine_kernel(const SnapArgs a) {
  const long long row = (long long)blockIdx.x * blockDim.x + threadIdx.x;   // (bh*RT + rt)*32 + i
  const long long rows = (long long)a.BH * a.RT * 32;
  if (row >= rows) return;
  constexpr float NEG_INF = -__builtin_huge_valf();
  const long long tile = row / 32, i = row - tile * 32;
  const float2* p = a.part + tile * a.S * 32 + i;
  float m = NEG_INF;
  for (int s = 0; s < a.S; ++s) m = fmaxf(m, p[s * 32].x);
  float l = 0.f;
  if (m != NEG_INF)
    for (int s = 0; s < a.S; ++s) {
      const float2 v = p[s * 32];
      if (v.x != NEG_INF) l += v.y * expf(v.x - m);
    }
  // rows with no visible key (padding rows of the last tile) contribute nothing
  a.stats[row] = m == NEG_INF ? make_float2(0.f, 0.f) : make_float2(m, 1.f / l);
}

template <typename E, int DP, int VEC>
__global__ __launch_bounds__(64) void snap_scores_kernel(const SnapArgs a) {
  constexpr int NDC = DP / 16;
  const int lane = threadIdx.x, l32 = lane & 31, hh = lane >> 5;
  const int nkb = (a.N + 63) / 64;
  const int kt = (int)(blockIdx.x % (unsigned)nkb);
  const int bh = (int)(blockIdx.x / (unsigned)nkb);
  const int b = bh / a.Hkv, hkv = bh - b * a.Hkv;
  const int kb = kt * 64;
  const u16* kbase = a.k + b * a.ks[0] + hkv * a.ks[1];

  // K fragments (B operand) of the block's 64 keys, loaded once for every row tile
  u32x4 kf[2][NDC];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int key = kb + 32 * s + l32;
    const bool kok = key < a.N;
    const u16* krow = kbase + (long long)(kok ? key : 0) * a.ks[2];
#pragma unroll
    for (int c = 0; c < NDC; ++c)
      kf[s][c] = kok ? load8(krow, a.ks[3], 16 * c + 8 * hh, a.D, VEC) : (u32x4){0u, 0u, 0u, 0u};
  }
  float acc[2] = {0.f, 0.f};
  for (int rt = 0; rt < a.RT; ++rt) {
    // this lane's query row (A operand) and its statistics
    const int r = rt * 32 + l32;
    const bool row_ok = r < a.R;
    int head = 0, qpos = -1;
    if (row_ok) snap_row(a, hkv, r, head, qpos);
    // rows with no work in this key block: every key of the block is past their position
    if (__all(!row_ok || qpos < kb)) continue;
    const u16* qrow = a.q + b * a.qs[0] + head * a.qs[1] + (long long)(row_ok ? qpos : 0) * a.qs[2];
    u32x4 qf[NDC];
#pragma unroll
    for (int c = 0; c < NDC; ++c)
      qf[c] = row_ok ? load8(qrow, a.qs[3], 16 * c + 8 * hh, a.D, VEC) : (u32x4){0u, 0u, 0u, 0u};
    const float2 st = a.stats[(long long)(bh * a.RT + rt) * 32 + l32];
    // statistics of the 16 rows a lane holds in the accumulator: 8(i/4) + 4h + i%4
    float m_r[16], il_r[16];
    int qp_r[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int ri = 8 * (i >> 2) + 4 * hh + (i & 3);
      m_r[i] = __shfl(st.x, ri);
      il_r[i] = __shfl(st.y, ri);
      qp_r[i] = __shfl(qpos, ri);
    }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int key = kb + 32 * s + l32;
      f32x16 sacc = (f32x16){};
#pragma unroll
      for (int c = 0; c < NDC; ++c) sacc = E::mfma(qf[c], kf[s][c], sacc);
      // lanes hold key kb + 32s + l32; register i holds row 8(i/4) + 4h + i%4 of the tile
      float sum = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float v = round_logit<E>(sacc[i]) * a.scale;
        sum += key <= qp_r[i] ? expf(v - m_r[i]) * il_r[i] : 0.f;
      }
      acc[s] += sum;
    }
  }
  // lanes h = 0 and 1 hold the two halves of the rows of each key; lane l of half s stores
  // key kb + 32s + l32
  const float t0 = half_swap_sum(acc[0]), t1 = half_swap_sum(acc[1]);
  const int key = kb + 32 * hh + l32;
  if (key < a.N) a.scores[(long long)bh * a.N + key] = (hh == 0 ? t0 : t1) / (float)a.G;
}

struct SnapKernel {
  const void* fn;
  const char* name;
};

// Index (dtype, DP, VEC) -> 2 * (4 * dtype + 2 * dpi + vec) (+1 for the scores kernel);
// VEC = 1: 16-byte row loads (channel stride 1, 16-byte aligned rows), 0: element loads.
#define FE_SNAP_KERNELS(E, DP, V, TAG)                                                            \
  {(const void*)snap_stats_kernel<E, DP, V>, "snap_stats_kernel<" TAG "," #DP "," #V ">"},         \
      {(const void*)snap_scores_kernel<E, DP, V>, "snap_scores_kernel<" TAG "," #DP "," #V ">"}

const SnapKernel kSnapKernels[] = {
    FE_SNAP_KERNELS(F16, 64, 0, "f16"),   FE_SNAP_KERNELS(F16, 64, 1, "f16"),
    FE_SNAP_KERNELS(F16, 128, 0, "f16"),  FE_SNAP_KERNELS(F16, 128, 1, "f16"),
    FE_SNAP_KERNELS(BF16, 64, 0, "bf16"), FE_SNAP_KERNELS(BF16, 64, 1, "bf16"),
    FE_SNAP_KERNELS(BF16, 128, 0, "bf16"), FE_SNAP_KERNELS(BF16, 128, 1, "bf16"),
    FE_SNAP_KERNELS(F16, 256, 0, "f16"),  FE_SNAP_KERNELS(F16, 256, 1, "f16"),
    FE_SNAP_KERNELS(BF16, 256, 0, "bf16"), FE_SNAP_KERNELS(BF16, 256, 1, "bf16"),
    {(const void*)snap_combine_kernel, "snap_combine_kernel"},
};
#undef FE_SNAP_KERNELS

void append_snap_resources(std::string& out) {
  for (const auto& e : kSnapKernels) {
    hipFuncAttributes attr;
    if (hipFuncGetAttributes(&attr, e.fn) != hipSuccess) continue;
    char buf[512];
    snprintf(buf, sizeof(buf),
             "{\"kernel\":\"%s\",\"registers_per_thread\":%d,\"lds_static_bytes\":%zu,"
             "\"lds_dynamic_bytes\":0,\"scratch_bytes_per_thread\":%zu,\"max_threads_per_block\":%d},",
             e.name, attr.numRegs, (size_t)attr.sharedSizeBytes, (size_t)attr.localSizeBytes,
             attr.maxThreadsPerBlock);
    out += buf;
  }
}

// Key splits of the statistics pass: enough waves to cover the chip (about 2048), at
// least one 64-key tile per split.
void snap_split(long long BH, long long RT, long long ntiles, int& S, int& per) {
  long long s = (2048 + BH * RT - 1) / (BH * RT);
  if (s < 1) s = 1;
  if (s > ntiles) s = ntiles;
  per = (int)((ntiles + s - 1) / s);
  S = (int)((ntiles + per - 1) / per);
}

bool snap_vec(const void* p, const int64_t* st, int64_t D) {
  return st[3] == 1 && D % 8 == 0 && ((uintptr_t)p % 16) == 0 && st[0] % 8 == 0 && st[1] % 8 == 0 &&
         st[2] % 8 == 0;
}

}  // namespace fe

using namespace fe;

extern "C" size_t fe_snap_scores_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t window) {
  if (B < 1 || Hq < 1 || Hkv < 1 || N < 1 || window < 1 || Hq % Hkv != 0) return 0;
  const long long W = window < N ? window : N;
  const long long BH = B * Hkv, R = (Hq / Hkv) * W, RT = (R + 31) / 32, ntiles = (N + 63) / 64;
  int S, per;
  snap_split(BH, RT, ntiles, S, per);
  return (size_t)(BH * RT * 32) * sizeof(float2) * (size_t)(S + 1);
}

extern "C" int fe_snap_scores(const void* q, const void* k, float* scores, int64_t B, int64_t Hq, int64_t Hkv,
                              int64_t N, int64_t D, const int64_t* q_strides, const int64_t* k_strides, int dtype,
                              int64_t window, void* workspace, size_t workspace_bytes, void* hip_stream) {
  clear_error();
  if (!q || !k || !scores || !q_strides || !k_strides) {
    set_error("fe_snap_scores: null pointer argument");
    return FE_ERR_INVALID;
  }
  if (B < 1 || Hq < 1 || Hkv < 1 || N < 1 || D < 1 || Hq % Hkv != 0 || window < 1) {
    set_error("fe_snap_scores: expected nonempty shapes, Hq divisible by Hkv and window >= 1");
    return FE_ERR_INVALID;
  }
  if (D > 256) {
    set_error("fe_snap_scores: head dimension must be <= 256");
    return FE_ERR_INVALID;
  }
  if (dtype != FE_DTYPE_F16 && dtype != FE_DTYPE_BF16) {
    set_error("fe_snap_scores: dtype must be FE_DTYPE_F16 or FE_DTYPE_BF16");
    return FE_ERR_INVALID;
  }
  for (int i = 0; i < 4; ++i)
    if (q_strides[i] < 0 || k_strides[i] < 0) {
      set_error("fe_snap_scores: negative strides are not supported");
      return FE_ERR_INVALID;
    }
  const long long W = window < N ? window : N;
  const long long G = Hq / Hkv, BH = B * Hkv, R = G * W, RT = (R + 31) / 32, ntiles = (N + 63) / 64;
  if (N > (1LL << 30) || R > (1LL << 30) || BH * RT * 32 > (1LL << 40) || BH * ntiles > 0x7fffffffLL) {
    set_error("fe_snap_scores: problem too large");
    return FE_ERR_UNSUPPORTED;
  }
  int S, per;
  snap_split(BH, RT, ntiles, S, per);
  if (BH * RT * S > 0x7fffffffLL) {
    set_error("fe_snap_scores: problem too large");
    return FE_ERR_UNSUPPORTED;
  }
  const size_t need = fe_snap_scores_workspace_bytes(B, Hq, Hkv, N, window);
  if (!workspace || workspace_bytes < need) {
    set_error("fe_snap_scores: needs a workspace of fe_snap_scores_workspace_bytes() bytes");
    return FE_ERR_WORKSPACE;
  }
  SnapArgs a;
  a.q = (const u16*)q;
  a.k = (const u16*)k;
  a.scores = scores;
  a.part = (float2*)workspace;
  a.stats = a.part + BH * RT * 32 * S;
  for (int i = 0; i < 4; ++i) {
    a.qs[i] = q_strides[i];
    a.ks[i] = k_strides[i];
  }
  a.N = (int)N;
  a.D = (int)D;
  a.G = (int)G;
  a.Hkv = (int)Hkv;
  a.BH = (int)BH;
  a.W = (int)W;
  a.R = (int)R;
  a.RT = (int)RT;
  a.S = S;
  a.tiles_per_split = per;
  a.ntiles = (int)ntiles;
  a.scale = (float)pow((double)D, -0.5);
  const int vec = snap_vec(q, q_strides, D) && snap_vec(k, k_strides, D) ? 1 : 0;
  const int bf = dtype == FE_DTYPE_BF16 ? 1 : 0;
  const int ki = D <= 128 ? 4 * bf + 2 * (D <= 64 ? 0 : 1) + vec : 8 + 2 * bf + vec;
  const void* stats_fn = kSnapKernels[2 * ki].fn;
  const void* scores_fn = kSnapKernels[2 * ki + 1].fn;
  hipStream_t stream = (hipStream_t)hip_stream;
  void* kargs[] = {&a};
  hipError_t err = hipLaunchKernel(stats_fn, dim3((unsigned)(BH * RT * S)), dim3(64), kargs, 0, stream);
  if (err == hipSuccess) {
    const long long rows = BH * RT * 32;
    err = hipLaunchKernel((const void*)snap_combine_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), kargs,
                          0, stream);
  }
  if (err == hipSuccess)
    err = hipLaunchKernel(scores_fn, dim3((unsigned)(BH * ntiles)), dim3(64), kargs, 0, stream);
  if (err != hipSuccess) {
    set_error(std::string("fe_snap_scores: launch: ") + hipGetErrorString(err));
    return FE_ERR_HIP;
  }
  return FE_OK;
}
