// Host-side entry points of libflash_evict_hip.so: error state, fused-kernel timing,
// kernel resource dump, and the CPU-memory selection path.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <string>
#include <utility>
#include <vector>

#include "fe_internal.h"
#include "../../include/flash_evict.h"

namespace fe {

int check_select_args(const float* scores, int64_t rows, int64_t n, int64_t row_stride, int64_t budget,
                      int64_t recent, int pool_kernel, const char* who);

namespace {
thread_local std::string g_error;

// Fused-kernel timing is per calling thread: a thread that enables it times only its own
// fe_prefill calls, and reads back only its own events. (No destructor: event pairs still
// unread when a thread exits are left to the runtime's teardown rather than destroyed from
// a thread-exit hook that may run after it.)
struct TimingState {
  bool on = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> events;
};
thread_local TimingState g_timing;

// Same order map as the device kernels: larger float <=> larger key, -0 == +0, NaN on top.
inline uint32_t order_key(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if (f != f) return 0xffffffffu;
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
}  // namespace

void set_error(const std::string& msg) { g_error = msg; }
void clear_error() { g_error.clear(); }

bool fused_timing_enabled() { return g_timing.on; }

void fused_timing_push(hipEvent_t start, hipEvent_t stop) { g_timing.events.emplace_back(start, stop); }

}  // namespace fe

using namespace fe;

extern "C" const char* fe_last_error(void) { return g_error.c_str(); }

extern "C" int fe_abi_version(void) { return 1; }

extern "C" int fe_fused_timing_enable(int enable) {
  clear_error();
  g_timing.on = enable != 0;
  return FE_OK;
}

extern "C" int fe_fused_timing_read(int64_t* launches, double* total_ms) {
  clear_error();
  std::vector<std::pair<hipEvent_t, hipEvent_t>> ev;
  ev.swap(g_timing.events);
  double total = 0.0;
  int rc = FE_OK;
  for (auto& p : ev) {
    float ms = 0.f;
    if (rc == FE_OK) {
      if (hipEventSynchronize(p.second) != hipSuccess || hipEventElapsedTime(&ms, p.first, p.second) != hipSuccess) {
        set_error("fe_fused_timing_read: event query failed");
        rc = FE_ERR_HIP;
      }
      total += ms;
    }
    (void)hipEventDestroy(p.first);
    (void)hipEventDestroy(p.second);
  }
  if (launches) *launches = (int64_t)ev.size();
  if (total_ms) *total_ms = total;
  return rc;
}

extern "C" int fe_kernel_resources(char* buf, size_t cap) {
  clear_error();
  std::string s = "[";
  append_attn_resources(s);
  append_select_resources(s);
  append_gather_resources(s);
  append_snap_resources(s);
  if (s.size() > 1 && s.back() == ',') s.pop_back();
  s += "]";
  if (s == "[]") {
    set_error("fe_kernel_resources: no kernel attributes available (no HIP device?)");
    return FE_ERR_HIP;
  }
  if (!buf || cap < s.size() + 1) {
    set_error("fe_kernel_resources: buffer too small; need " + std::to_string(s.size() + 1) + " bytes");
    return FE_ERR_INVALID;
  }
  memcpy(buf, s.c_str(), s.size() + 1);
  return FE_OK;
}

extern "C" int fe_select_host(const float* scores, int64_t rows, int64_t n, int64_t row_stride, int64_t budget,
                              int64_t recent, int pool_kernel, int64_t* indices_out, uint8_t* mask_out,
                              int invert) {
  clear_error();
  int rc = check_select_args(scores, rows, n, row_stride, budget, recent, pool_kernel, "fe_select_host");
  if (rc) return rc;
  const int64_t m = n - recent;
  const int64_t K = budget - recent;
  const bool pool = pool_kernel > 1 && budget > recent;
  const uint8_t keep_v = invert ? 0 : 1, drop_v = invert ? 1 : 0;
  const int64_t stride = rows > 1 ? row_stride : n;
  std::vector<float> pooled(pool ? (size_t)m : 0);
  std::vector<uint32_t> keys((size_t)m), work;
  for (int64_t r = 0; r < rows; ++r) {
    const float* x = scores + r * stride;
    if (pool) {
      const int64_t half = pool_kernel / 2;
      for (int64_t i = 0; i < m; ++i) {
        const int64_t lo = std::max<int64_t>(0, i - half), hi = std::min<int64_t>(m - 1, i + half);
        float acc = 0.f;
        for (int64_t j = lo; j <= hi; ++j) acc += x[j];
        pooled[(size_t)i] = acc / (float)pool_kernel;
      }
      x = pooled.data();
    }
    int64_t* irow = indices_out ? indices_out + r * budget : nullptr;
    uint8_t* mrow = mask_out ? mask_out + r * n : nullptr;
    int64_t out = 0;
    if (K > 0) {
      for (int64_t i = 0; i < m; ++i) keys[(size_t)i] = order_key(x[i]);
      work = keys;
      std::nth_element(work.begin(), work.begin() + (K - 1), work.end(), std::greater<uint32_t>());
      const uint32_t T = work[(size_t)(K - 1)];
      int64_t n_gt = 0;
      for (int64_t i = 0; i < m; ++i) n_gt += keys[(size_t)i] > T;
      int64_t need_eq = K - n_gt;
      for (int64_t i = 0; i < m; ++i) {
        const uint32_t key = keys[(size_t)i];
        bool sel = key > T;
        if (!sel && key == T && need_eq > 0) {
          sel = true;
          --need_eq;
        }
        if (sel && irow) irow[out] = i;
        out += sel;
        if (mrow) mrow[i] = sel ? keep_v : drop_v;
      }
    } else if (mrow) {
      for (int64_t i = 0; i < m; ++i) mrow[i] = drop_v;
    }
    for (int64_t j = 0; j < recent; ++j) {
      if (irow) irow[K + j] = m + j;
      if (mrow) mrow[m + j] = keep_v;
    }
  }
  return FE_OK;
}
