// Shared device/host definitions for the flash_evict gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fe {

typedef unsigned int u32;
typedef u32 u32x4 __attribute__((ext_vector_type(4)));
typedef u32 u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Element tags: storage is always 16-bit; the tag selects MFMA flavour and rounding.
// Rescale headroom of the bf16 attention kernels (build option; 0 takes the exact max).
#ifndef FE_RESCALE_HEADROOM_BF16
#define FE_RESCALE_HEADROOM_BF16 16.f
#endif

struct BF16 {
  typedef __bf16 scalar;
  // Largest per-lane sum of one step's probabilities (relative to a row's reference max)
  // the attention kernels accept before taking a new reference max: bf16 and the FP32
  // accumulation have FP32's range. A row then gains at most 2 * 2^32 per 32 keys (two
  // lanes hold its keys), so its sum stays below 2^33 * ceil(N/32) and |O| below that times
  // max|v|: O stays finite for max|v| < 2^95 / ceil(N/32) (2^83, about 1e25, at N = 131072).
  // The reference's running max keeps every probability at most 1, so its accumulator stays
  // finite up to max|v| < 2^128 / N. Between the two bounds the output overflows here and
  // not there; below 2^95 / ceil(N/32) every rounding is relative, and scaling V by a power
  // of two scales the output and importance exactly.
  static constexpr float kMaxTileSum = 4294967296.f;
  // A step that overflows takes as its new reference the step's exact max plus this headroom
  // (log2 units), so that later keys may rise 32 + 16 above the step's max before the next
  // rescale. Its probabilities are then at most 2^-16, which bf16 and FP32 hold with full
  // relative precision; rows that never overflow are unaffected.
  static constexpr float kRescaleHeadroom = FE_RESCALE_HEADROOM_BF16;
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // Round-to-nearest-even pack of two floats (lo in bits 0..15).
  static __device__ __forceinline__ u32 pack2(float lo, float hi) {
    bf16x2 r = __builtin_convertvector((f32x2){lo, hi}, bf16x2);
    return __builtin_bit_cast(u32, r);
  }
  static __device__ __forceinline__ float to_f32(unsigned short bits) {
    return __uint_as_float(((u32)bits) << 16);
  }
  // acc + lo + hi of a packed pair, the rounded values (v_dot2c_f32_bf16 against ones2 =
  // (1, 1) of the type, kOnes2, which callers keep in a scalar register: as a 32-bit
  // literal operand v_dot2c issues measurably slower)
  static constexpr u32 kOnes2 = 0x3f803f80u;
  static __device__ __forceinline__ float sum2(u32 packed, u32 ones2, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, packed), __builtin_bit_cast(bf16x2, ones2), acc,
                                           false);
  }
  // lo + hi of a packed pair (sum2 with acc = 0) as one VOP3P v_dot2_f32_bf16 with an inline
  // zero: sum2(p, ones2, 0.f) compiles to the accumulating v_dot2c form after a v_mov of 0.
  static __device__ __forceinline__ float sum2_0(u32 packed, u32 ones2) {
    float r;
    asm("v_dot2_f32_bf16 %0, %1, %2, 0" : "=v"(r) : "v"(packed), "s"(ones2));
    return r;
  }
};

struct F16 {
  typedef _Float16 scalar;
  // probabilities stay below the fp16 maximum; |O| < 2^16 * ceil(N/32) * 65504 is always finite
  static constexpr float kMaxTileSum = 32768.f;
  // no headroom: probabilities far below the reference max would fall into fp16's subnormal
  // range, where the rounding of P for P@V is no longer relative
  static constexpr float kRescaleHeadroom = 0.f;
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ u32 pack2(float lo, float hi) {
    f16x2 r = __builtin_convertvector((f32x2){lo, hi}, f16x2);
    return __builtin_bit_cast(u32, r);
  }
  static __device__ __forceinline__ float to_f32(unsigned short bits) {
    return (float)__builtin_bit_cast(_Float16, bits);
  }
  static constexpr u32 kOnes2 = 0x3c003c00u;
  static __device__ __forceinline__ float sum2(u32 packed, u32 ones2, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, packed), __builtin_bit_cast(f16x2, ones2), acc, false);
  }
  static __device__ __forceinline__ float sum2_0(u32 packed, u32 ones2) {
    float r;
    asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(r) : "v"(packed), "s"(ones2));
    return r;
  }
};

// max/sum of a value with its counterpart in the other 32-lane half of the wave.
// v_permlane32_swap(x, x) returns {lanes 0-31: x[l], lanes 32-63: x[l-32]} and
// {lanes 0-31: x[l+32], lanes 32-63: x[l]}; combining both halves is symmetric.
__device__ __forceinline__ float half_swap_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_swap_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Workgroup barrier that orders LDS accesses only (waits for the wave's LDS operations, not
// for its outstanding global loads, stores or LDS-destination DMA). Where global memory or
// DMA-written LDS must be complete first, the caller waits for it explicitly.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

}  // namespace fe
