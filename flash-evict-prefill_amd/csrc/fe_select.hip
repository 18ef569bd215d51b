// Token selection for gfx950: optional SnapKV average pooling, radix top-k, and the
// keep/evict mask plus ascending kept indices, honouring the reserved recent suffix.
//
// Semantics follow flash_evict/prefill.py:140-180 (select_tokens / evict):
//   past = scores[..., :n-recent]                                           (:160)
//   if pool_kernel > 1 and budget > recent:
//       past = avg_pool1d(past, k, stride 1, pad k//2)  (count_include_pad)  (:161-163)
//   top = past.topk(budget - recent)                                        (:164)
//   indices = sort(cat(top, arange(n-recent, n)))                           (:165-168)
//   keep = zeros.scatter_(indices, True); evict returns ~keep               (:169, :180)
// torch.topk leaves tie order unspecified (prefill.py:144); this build fixes it: among
// equal scores the lower index is kept. -0.0 ties with +0.0; NaN ranks above +inf.
//
// Schedule: no sort at all. A three-digit (11/11/10-bit) MSB radix select per row finds
// the threshold key T of the (budget-recent)-th largest score with LDS histograms; one
// ordered pass then keeps key > T plus the first ties at T, and a block prefix sum gives
// each kept token its output slot, so indices come out ascending and the mask is written
// in the same pass. One 1024-thread workgroup per row; the passes over a row read 16-byte
// vectors when the row is 16-byte aligned.
#include <math.h>
#include <string>

#include "fe_common.h"
#include "fe_internal.h"
#include "../../include/flash_evict.h"

namespace fe {

__device__ __forceinline__ u32 order_key(float f) {
  u32 u = __float_as_uint(f);
  if (f != f) return 0xffffffffu;  // NaN: above every number (torch.topk convention)
  if (u == 0x80000000u) u = 0u;    // -0.0 ties with +0.0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

constexpr int kSelThreads = 1024;               // threads of a selection workgroup (one row)
constexpr int kSelWaves = kSelThreads / 64;

// Exclusive prefix sum over the threads of a selection workgroup; `total` receives the sum.
__device__ __forceinline__ int block_exclusive_scan(int v, int* tmp, int& total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  if (lane == 63) tmp[w] = x;
  __syncthreads();
  int before = 0;
  total = 0;
#pragma unroll
  for (int i = 0; i < kSelWaves; ++i) {
    const int t = tmp[i];
    before += (i < w) ? t : 0;
    total += t;
  }
  __syncthreads();
  return before + x - v;
}

// out[r, i] = (sum_{j=i-k/2}^{i+k/2} past[r, j], zeros outside [0, m)) / k, summed left to
// right (the order of torch's avg_pool kernels).
__global__ __launch_bounds__(256) void avg_pool_kernel(const float* s, long long rs, int m, int k,
                                                       long long blocks_per_row, float* out) {
  const long long row = (long long)blockIdx.x / blocks_per_row;
  const int i = (int)(((long long)blockIdx.x - row * blocks_per_row) * 256 + threadIdx.x);
  if (i >= m) return;
  const float* x = s + row * rs;
  const int half = k >> 1;
  const int lo = i - half < 0 ? 0 : i - half;
  const int hi = i + half > m - 1 ? m - 1 : i + half;
  float acc = 0.f;
  for (int j = lo; j <= hi; ++j) acc += x[j];
  out[row * (long long)m + i] = acc / (float)k;
}

__global__ __launch_bounds__(kSelThreads) void select_rows_kernel(const float* src, long long src_stride, int m,
                                                                  int K, int n, int recent, long long* idx,
                                                                  int budget, unsigned char* mask, int invert) {
  constexpr int ST = kSelThreads;
  __shared__ u32 hist[2048];
  __shared__ int scan_tmp[kSelWaves];
  __shared__ u32 sh_prefix;
  __shared__ int sh_kk;
  __shared__ u32 sh_eq;
  const int tid = threadIdx.x;
  const long long row = blockIdx.x;
  const float* x = src + row * src_stride;
  const bool vec = ((uintptr_t)x & 15u) == 0;   // 16-byte loads of 4 scores
  long long* irow = idx ? idx + row * (long long)budget : nullptr;
  unsigned char* mrow = mask ? mask + row * (long long)n : nullptr;
  const unsigned char keep_v = invert ? 0 : 1, drop_v = invert ? 1 : 0;

  if (K > 0) {
    u32 prefix = 0, pmask = 0;
    int kk = K;
    u32 eq_total = 0;
    for (int pass = 0; pass < 3; ++pass) {
      const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
      const int bits = pass == 2 ? 10 : 11;
      const int nb = 1 << bits;
      for (int i = tid; i < nb; i += ST) hist[i] = 0u;
      __syncthreads();
      auto count = [&](float f) __attribute__((always_inline)) {
        const u32 key = order_key(f);
        if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & (u32)(nb - 1)], 1u);
      };
      for (int i = 4 * tid; i < m; i += 4 * ST) {
        if (vec && i + 3 < m) {
          const float4 v = *(const float4*)(x + i);
          count(v.x);
          count(v.y);
          count(v.z);
          count(v.w);
        } else {
          for (int e = 0; e < 4 && i + e < m; ++e) count(x[i + e]);
        }
      }
      __syncthreads();
      // Thread t owns bins [nb - (t+1)*bpt, nb - t*bpt): thread 0 holds the highest digits.
      const int bpt = nb / ST;
      const int hi_bin = nb - 1 - tid * bpt;
      int local = 0;
      for (int e = 0; e < bpt; ++e) local += (int)hist[hi_bin - e];
      int total;
      int cum = block_exclusive_scan(local, scan_tmp, total);
      for (int e = 0; e < bpt; ++e) {
        const int bin = hi_bin - e;
        const int h = (int)hist[bin];
        if (cum < kk && cum + h >= kk) {
          sh_prefix = prefix | ((u32)bin << shift);
          sh_kk = kk - cum;
          sh_eq = (u32)h;
        }
        cum += h;
      }
      __syncthreads();
      prefix = sh_prefix;
      kk = sh_kk;
      eq_total = sh_eq;
      pmask |= (u32)(nb - 1) << shift;
      __syncthreads();
    }
    const u32 T = prefix;       // key of the K-th largest score
    const int need_eq = kk;     // ties at T still to keep, lowest index first
    const bool all_eq = (int)eq_total == need_eq;
    int out_base = 0, eq_base = 0;
    for (int c0 = 0; c0 < m; c0 += ST * 8) {
      const int i0 = c0 + tid * 8;
      float xv[8];
      if (vec && i0 + 7 < m) {
        const float4 a0 = *(const float4*)(x + i0), a1 = *(const float4*)(x + i0 + 4);
        xv[0] = a0.x; xv[1] = a0.y; xv[2] = a0.z; xv[3] = a0.w;
        xv[4] = a1.x; xv[5] = a1.y; xv[6] = a1.z; xv[7] = a1.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[e] = i0 + e < m ? x[i0 + e] : 0.f;
      }
      bool gt[8], eq[8];
      int neq = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int i = i0 + e;
        const bool valid = i < m;
        const u32 key = valid ? order_key(xv[e]) : 0u;
        gt[e] = valid && key > T;
        eq[e] = valid && key == T;
        neq += eq[e] ? 1 : 0;
      }
      int eq_before = 0;
      if (!all_eq) {
        int tot;
        eq_before = block_exclusive_scan(neq, scan_tmp, tot) + eq_base;
        eq_base += tot;
      }
      bool sel[8];
      int nsel = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sel[e] = gt[e] || (eq[e] && (all_eq || eq_before < need_eq));
        eq_before += eq[e] ? 1 : 0;
        nsel += sel[e] ? 1 : 0;
      }
      int tot2;
      int pos = block_exclusive_scan(nsel, scan_tmp, tot2) + out_base;
      out_base += tot2;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int i = i0 + e;
        if (sel[e] && irow && pos < K) irow[pos] = i;
        pos += sel[e] ? 1 : 0;
        if (mrow && i < m) mrow[i] = sel[e] ? keep_v : drop_v;
      }
    }
  } else if (mrow) {
    for (int i = tid; i < m; i += ST) mrow[i] = drop_v;
  }
  for (int j = tid; j < recent; j += ST) {
    if (irow) irow[K + j] = (long long)(m + j);
    if (mrow) mrow[m + j] = keep_v;
  }
}

namespace {

struct SelKernel {
  const void* fn;
  const char* name;
};

const SelKernel kSelKernels[] = {
    {(const void*)avg_pool_kernel, "avg_pool"},
    {(const void*)select_rows_kernel, "select_rows"},
};

}  // namespace

void append_select_resources(std::string& out) {
  for (const auto& e : kSelKernels) {
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

// Shared argument validation of fe_select / fe_select_host.
int check_select_args(const float* scores, int64_t rows, int64_t n, int64_t row_stride, int64_t budget,
                      int64_t recent, int pool_kernel, const char* who) {
  if (rows < 0 || n < 1 || (rows > 0 && !scores)) {
    set_error(std::string(who) + ": invalid scores pointer or shape");
    return FE_ERR_INVALID;
  }
  if (budget < 1 || budget > n) {
    set_error(std::string(who) + ": budget must be an integer in [1, sequence length]");
    return FE_ERR_INVALID;
  }
  if (recent < 0 || recent > budget) {
    set_error(std::string(who) + ": recent must be an integer in [0, budget]");
    return FE_ERR_INVALID;
  }
  if (pool_kernel < 1 || pool_kernel % 2 != 1) {
    set_error(std::string(who) + ": pool_kernel must be a positive odd integer");
    return FE_ERR_INVALID;
  }
  if (rows > 1 && row_stride < n) {
    set_error(std::string(who) + ": row_stride must be >= n");
    return FE_ERR_INVALID;
  }
  if (n > 0x7fffffffLL || rows > 0x7fffffffLL) {
    set_error(std::string(who) + ": sizes exceed the supported range");
    return FE_ERR_UNSUPPORTED;
  }
  return FE_OK;
}

}  // namespace fe

using namespace fe;

extern "C" size_t fe_select_workspace_bytes(int64_t rows, int64_t n, int64_t budget, int64_t recent,
                                            int pool_kernel) {
  if (rows <= 0 || n <= 0 || recent < 0 || recent > n) return 0;
  if (pool_kernel > 1 && budget > recent) return (size_t)rows * (size_t)(n - recent) * sizeof(float);
  return 0;
}

extern "C" int fe_select(const float* scores, int64_t rows, int64_t n, int64_t row_stride, int64_t budget,
                         int64_t recent, int pool_kernel, int64_t* indices_out, uint8_t* mask_out, int invert,
                         void* workspace, size_t workspace_bytes, void* hip_stream) {
  clear_error();
  int rc = check_select_args(scores, rows, n, row_stride, budget, recent, pool_kernel, "fe_select");
  if (rc) return rc;
  if (rows == 0) return FE_OK;
  hipStream_t stream = (hipStream_t)hip_stream;
  const int m = (int)(n - recent);
  const int K = (int)(budget - recent);
  const float* src = scores;
  long long src_stride = rows > 1 ? row_stride : n;
  if (pool_kernel > 1 && budget > recent) {
    const size_t need = fe_select_workspace_bytes(rows, n, budget, recent, pool_kernel);
    if (!workspace || workspace_bytes < need) {
      set_error("fe_select: pooling needs a workspace of fe_select_workspace_bytes() bytes");
      return FE_ERR_WORKSPACE;
    }
    const long long bpr = (m + 255) / 256;
    if (bpr * rows > 0x7fffffffLL) {
      set_error("fe_select: pooling grid too large");
      return FE_ERR_UNSUPPORTED;
    }
    hipLaunchKernelGGL(avg_pool_kernel, dim3((unsigned)(bpr * rows)), dim3(256), 0, stream, scores, src_stride,
                       m, pool_kernel, bpr, (float*)workspace);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
      set_error(std::string("fe_select: pool launch: ") + hipGetErrorString(err));
      return FE_ERR_HIP;
    }
    src = (const float*)workspace;
    src_stride = m;
  }
  hipLaunchKernelGGL(select_rows_kernel, dim3((unsigned)rows), dim3(kSelThreads), 0, stream, src, src_stride, m, K,
                     (int)n,
                     (int)recent, (long long*)indices_out, (int)budget, (unsigned char*)mask_out, invert ? 1 : 0);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error(std::string("fe_select: select launch: ") + hipGetErrorString(err));
    return FE_ERR_HIP;
  }
  return FE_OK;
}
