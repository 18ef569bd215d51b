// KV compaction gather for gfx950: out[b,h,j,:] = x[b,h,indices[b,h,j],:].
//
// This is the consumer of the kept indices: `gather_tokens(state['k'], indices)` at
// flash_evict/kv_distill_adapter.py:38-39, streaming_adapter.py:86 and
// quality_adapter.py:109-110 of the reference (kv_distill.cache.gather_tokens, a local
// research package that the reference does not vendor). From those call sites: x is a
// [B,H,N,D] cache tensor (often a transposed view, channel stride 1), indices is
// [B,H,K] int64 (select_tokens output, or an expanded arange with zero leading strides),
// and the result is the contiguous [B,H,K,D] tensor of the selected rows, i.e.
// x.gather(2, indices[..., None].expand(..., D)).
//
// HBM-bound byte work: K*D*elem bytes read and written per (b,h) plus 8*K index bytes.
// Rows are moved as 16-byte chunks, one chunk per lane, so a wave moves 1 KiB per
// instruction and consecutive lanes touch consecutive bytes of one row on both sides.
// Layouts without 16-byte rows take an element-wise kernel. An index outside [0, N)
// yields a zero row (torch.gather would raise a device-side assertion instead).
#include <string>

#include "fe_common.h"
#include "fe_internal.h"
#include "../../include/flash_evict.h"

namespace fe {

struct GatherArgs {
  const unsigned char* x;
  const long long* idx;
  unsigned char* out;
  long long H, K, N;
  long long xs0, xs1, xs2;   // x strides in bytes (b, h, n); channel stride is elem bytes
  long long is0, is1, is2;   // index strides in elements
  long long cpr;             // 16-byte chunks per row (vector kernel) or elements per row
  long long total;           // chunks (vector) or elements (scalar) of the output
};

__device__ __forceinline__ long long gather_src_row(const GatherArgs& a, long long r, bool& ok) {
  const long long j = r % a.K;
  const long long bh = r / a.K;
  const long long h = bh % a.H, b = bh / a.H;
  const long long t = a.idx[b * a.is0 + h * a.is1 + j * a.is2];
  ok = t >= 0 && t < a.N;
  return b * a.xs0 + h * a.xs1 + (ok ? t : 0) * a.xs2;
}

// Four chunks per thread, strided by the grid so every load of a wave is one contiguous
// KiB; the four loads are issued before the four stores.
__global__ __launch_bounds__(256) void gather_rows16_kernel(const GatherArgs a) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long c0 = (long long)blockIdx.x * blockDim.x + threadIdx.x; c0 < a.total; c0 += 4 * stride) {
    u32x4 v[4];
    long long dst[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const long long c = c0 + u * stride;
      dst[u] = -1;
      if (c < a.total) {
        const long long r = c / a.cpr, ch = c - r * a.cpr;
        bool ok;
        const long long src = gather_src_row(a, r, ok);
        v[u] = ok ? *(const u32x4*)(a.x + src + ch * 16) : (u32x4){0u, 0u, 0u, 0u};
        dst[u] = c * 16;
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (dst[u] >= 0) *(u32x4*)(a.out + dst[u]) = v[u];
  }
}

// Element-wise fallback for any strides and element sizes of 1, 2, 4 or 8 bytes.
template <typename T>
__global__ __launch_bounds__(256) void gather_elems_kernel(const GatherArgs a, long long xs3) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x; e < a.total; e += stride) {
    const long long r = e / a.cpr, d = e - r * a.cpr;
    bool ok;
    const long long src = gather_src_row(a, r, ok);
    ((T*)a.out)[e] = ok ? *(const T*)(a.x + src + d * xs3) : (T)0;
  }
}

struct GatherKernel {
  const void* fn;
  const char* name;
};
const GatherKernel kGatherKernels[] = {
    {(const void*)gather_rows16_kernel, "gather_rows16_kernel"},
    {(const void*)gather_elems_kernel<unsigned char>, "gather_elems_kernel<u8>"},
    {(const void*)gather_elems_kernel<unsigned short>, "gather_elems_kernel<u16>"},
    {(const void*)gather_elems_kernel<unsigned int>, "gather_elems_kernel<u32>"},
    {(const void*)gather_elems_kernel<unsigned long long>, "gather_elems_kernel<u64>"},
};

void append_gather_resources(std::string& out) {
  for (const auto& e : kGatherKernels) {
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

}  // namespace fe

using namespace fe;

extern "C" int fe_gather_rows(const void* x, const int64_t* indices, void* out, int64_t B, int64_t H, int64_t N,
                              int64_t D, int64_t K, const int64_t* x_strides, const int64_t* index_strides,
                              int elem_bytes, void* hip_stream) {
  clear_error();
  if (B < 0 || H < 0 || N < 1 || D < 1 || K < 0 || !x_strides || !index_strides) {
    set_error("fe_gather_rows: invalid shape or stride arrays");
    return FE_ERR_INVALID;
  }
  if (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4 && elem_bytes != 8) {
    set_error("fe_gather_rows: elem_bytes must be 1, 2, 4 or 8");
    return FE_ERR_INVALID;
  }
  const long long rows = (long long)B * H * K;
  if (rows == 0) return FE_OK;
  if (!x || !indices || !out) {
    set_error("fe_gather_rows: null pointer argument");
    return FE_ERR_INVALID;
  }
  for (int i = 0; i < 4; ++i)
    if (x_strides[i] < 0 || (i < 3 && index_strides[i] < 0)) {
      set_error("fe_gather_rows: negative strides are not supported");
      return FE_ERR_INVALID;
    }
  if (rows > (1LL << 40) || D > (1LL << 30) || (double)rows * (double)D > 1e15) {
    set_error("fe_gather_rows: sizes exceed the supported range");
    return FE_ERR_UNSUPPORTED;
  }
  GatherArgs a;
  a.x = (const unsigned char*)x;
  a.idx = (const long long*)indices;
  a.out = (unsigned char*)out;
  a.H = H;
  a.K = K;
  a.N = N;
  a.xs0 = x_strides[0] * elem_bytes;
  a.xs1 = x_strides[1] * elem_bytes;
  a.xs2 = x_strides[2] * elem_bytes;
  a.is0 = index_strides[0];
  a.is1 = index_strides[1];
  a.is2 = index_strides[2];
  const long long row_bytes = D * elem_bytes;
  const bool vec = x_strides[3] == 1 && row_bytes % 16 == 0 && ((uintptr_t)x % 16) == 0 &&
                   ((uintptr_t)out % 16) == 0 && (B <= 1 || a.xs0 % 16 == 0) && (H <= 1 || a.xs1 % 16 == 0) &&
                   a.xs2 % 16 == 0;
  a.cpr = vec ? row_bytes / 16 : D;
  a.total = rows * a.cpr;
  const long long per_block = vec ? 4 * 256 : 256;
  const long long blocks = (a.total + per_block - 1) / per_block;
  const unsigned grid = (unsigned)(blocks < 65536 ? blocks : 65536);
  hipStream_t stream = (hipStream_t)hip_stream;
  if (vec) {
    hipLaunchKernelGGL(gather_rows16_kernel, dim3(grid), dim3(256), 0, stream, a);
  } else {
    const long long xs3 = x_strides[3] * elem_bytes;
    switch (elem_bytes) {
      case 1: hipLaunchKernelGGL(gather_elems_kernel<unsigned char>, dim3(grid), dim3(256), 0, stream, a, xs3); break;
      case 2: hipLaunchKernelGGL(gather_elems_kernel<unsigned short>, dim3(grid), dim3(256), 0, stream, a, xs3); break;
      case 4: hipLaunchKernelGGL(gather_elems_kernel<unsigned int>, dim3(grid), dim3(256), 0, stream, a, xs3); break;
      default: hipLaunchKernelGGL(gather_elems_kernel<unsigned long long>, dim3(grid), dim3(256), 0, stream, a, xs3); break;
    }
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error(std::string("fe_gather_rows: launch: ") + hipGetErrorString(err));
    return FE_ERR_HIP;
  }
  return FE_OK;
}
