// Host-side internals shared by the translation units of libflash_evict_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

namespace fe {

// Thread-local error message; every entry point clears it on entry.
void set_error(const std::string& msg);
void clear_error();

// Fill n floats with zero on `stream` (a kernel, not hipMemsetAsync).
hipError_t launch_zero_f32(float* p, int64_t n, hipStream_t stream);

// Resource dump helpers: each kernel family appends JSON objects to `out`.
void append_attn_resources(std::string& out);
void append_select_resources(std::string& out);
void append_gather_resources(std::string& out);
void append_snap_resources(std::string& out);

// Device address of fe_prefill_static's workspace on the device of `stream` (fe_static.hip).
hipError_t static_scratch(hipStream_t stream, float** out);

// Fused-kernel timing (enabled through fe_fused_timing_enable).
bool fused_timing_enabled();
void fused_timing_push(hipEvent_t start, hipEvent_t stop);

}  // namespace fe
