// Workspace of fe_prefill_static (fe_attn.hip): a file-scope device array, so that entry point
// allocates nothing. It lives in a translation unit of its own, with no kernels: the runtime
// loads this unit's code object, and with it the array, on a device only when
// hipGetSymbolAddress first asks for the array there, so processes that never call
// fe_prefill_static do not hold it (in the attention kernels' unit, every prefill call reserved
// its 16 MiB on each device it ran on).
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/flash_evict.h"
#include "fe_attn.h"
#include "fe_internal.h"

namespace fe {
namespace {

// FE_STATIC_BIAS_ROWS floats of replay biases plus the dynamic schedule's item counters (16 MiB
// + 4 KiB) on every GPU fe_prefill_static runs on, held until the process ends. Its contents
// persist between calls (the last call's biases and counters); the attention kernel writes every
// bias the replay kernel reads, and each call zeroes the counters (with a fill kernel) before its
// kernels run.
__device__ __align__(256) float scratch[FE_STATIC_BIAS_ROWS + kQueueWords];

// Device address of `scratch`, per device: looked up with that device current, on the first
// fe_prefill_static call that runs there, and kept. Host code passes this address to the
// kernels; the array's name is only a host-side stand-in symbol. Only a successful lookup is
// kept: a failed one (say, a call made while the device was busy with another context)
// returns its error and the next call tries again. The lookup (and the first call's occupancy
// queries) are host API calls, not stream work; a caller that captures fe_prefill_static in a
// HIP graph makes one eager call on each device first, so the capture finds them done.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

}  // namespace

hipError_t static_scratch(hipStream_t stream, float** out) {
  int cur = 0;
  hipError_t err = hipGetDevice(&cur);
  if (err != hipSuccess) return err;
  int dev = cur;
  if (stream) {
    hipDevice_t d = 0;
    if ((err = hipStreamGetDevice(stream, &d)) != hipSuccess) return err;
    dev = (int)d;
  }
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    if (dev != cur && (err = hipSetDevice(dev)) != hipSuccess) return err;
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (dev != cur) {
      const hipError_t back = hipSetDevice(cur);
      if (err == hipSuccess) err = back;
    }
    if (err != hipSuccess) return err;
    if (!ptr) return hipErrorInvalidSymbol;
    g_scratch[dev] = ptr;
  }
  *out = (float*)g_scratch[dev];
  return hipSuccess;
}

}  // namespace fe
