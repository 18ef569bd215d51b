// Argument block and launch hooks shared by the fused attention + score kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "fe_common.h"

namespace fe {

typedef unsigned short u16;

struct AttnArgs {
  const u16* q;
  const u16* k;
  const u16* v;
  u16* out;
  float* imp;
  float* bias;                      // split schedule: per-row replay bias out of traversal 1 (else null)
  long long qs[4], ks[4], vs[4];   // element strides {b, h, n, d}
  int N, D, G, Hq, Hkv, BH;           // D: channels of the K/V rows the kernel reads
  int Dq;                           // channels of Q and out (D, or less when K/V were repacked)
  unsigned qmask;                   // ANDed into Q at load: 0 runs a zero scale on the fast kernels
  int tiles_bh;                     // row tiles per (b, kv head): G * ceil(N/32)
  int wg_bh;                        // workgroups per (b, kv head)
  float scale_log2;                 // softmax scale * log2(e)
  float abs_scale_log2;
  float decay_log2;                 // recency_decay * log2(e)
  int neg_scale;
  int causal, score, win_lo;        // win_lo = N - W
  int rsplit;                       // replay kernel: key splits per workgroup of row tiles
  int* queue;                       // dynamic schedule: item counter, zero at launch (else null)
  int nitems;                       // dynamic schedule: work items of the launch
  int nstatic;                      // dynamic schedule: workgroups launched (each starts with item blockIdx.x)
  int tail;                         // dynamic schedule: first item of the queues' light parts (nitems: none)
  int nattn;                        // attention items; items past them are replay items
  int rwg0;                         // replay items in ascending row groups from rwg0 (-1: heaviest first)
  unsigned* done;                   // replay items: one bit per attention item, set once its biases are out
  int wait_base, wait_per_tile;     // replay items: polls of a dependency's bit (plus per key tile) before running it
  int qvec, kvec, vvec, ovec;       // 16-byte (q/k/v) and 8-byte (out) vector access allowed
};

// Work-item counters of the dynamic schedule, at the end of the prefill workspace (the
// next 256-byte boundary after the replay biases): eight per kernel (one per XCD queue), each
// on its own 128-byte line, the attention kernel's from word 0 and the replay kernel's from
// word kQueueReplay; a queue's counters are the 64-bit words at ints 0 and 2 of its line (its
// heavy and light parts, take_item in fe_attn_fast.hip). Then, from word kQueueDone, one bit per
// attention item for the replay items of attn_rt2_kernel (kMaxDoneItems bits). Zeroed before
// every launch.
constexpr int kQueueStride = 32;
constexpr int kQueueReplay = 8 * kQueueStride;
constexpr int kQueueDone = 2 * kQueueReplay;
constexpr int kMaxDoneItems = 16384;
constexpr int kQueueWords = kQueueDone + kMaxDoneItems / 32;
constexpr size_t kQueueBytes = kQueueWords * sizeof(int);
// s_getreg_b32 operand of hwreg(HW_REG_XCC_ID): register 20, bits 0-31 (the XCC index is bits 0-3)
constexpr int kHwRegXccId = (31 << 11) | 20;

// Load 8 consecutive channels [d0, d0+8) of one row; zero beyond D.
__device__ __forceinline__ u32x4 load8(const u16* row, long long sd, int d0, int D, int vec) {
  if (vec) {
    if (d0 < D) return *(const u32x4*)(row + d0);
    return (u32x4){0u, 0u, 0u, 0u};
  }
  u32 w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int da = d0 + 2 * i, db = da + 1;
    const u32 lo = da < D ? (u32)row[(long long)da * sd] : 0u;
    const u32 hi = db < D ? (u32)row[(long long)db * sd] : 0u;
    w[i] = lo | (hi << 16);
  }
  return (u32x4){w[0], w[1], w[2], w[3]};
}

// A launch plan: the kernel, its grid and dynamic LDS, and the rows per workgroup.
struct FusedPlan {
  const void* fn;
  size_t lds;
  int waves;          // waves per workgroup
  int rows;           // row tiles (32 queries of one head) per workgroup
  const char* name;
};

// Fast path (fe_attn_fast.hip): D a multiple of 8 up to 256, nonzero scale, 16-byte unit-stride
// buffer-addressable K/V rows (Q of any strides). Returns false (and leaves `plan` untouched) when it does not apply.
bool fast_plan(const AttnArgs& a, int dtype, FusedPlan& plan);
// Whether the fast kernels can read K and V as laid out (D a multiple of 8 up to 256; aligned,
// unit-stride rows within 32-bit byte offsets).
bool fast_layout(const AttnArgs& a);
// Replay kernel of the split schedule (fe_attn_fast.hip): same layout rules as fast_plan;
// launched with ReplayPlan::waves waves and ReplayPlan::rows row tiles per workgroup.
struct ReplayPlan {
  const void* fn;
  int waves;
  int rows;
  const char* name;
};
// The small-grid attention kernel at tile dims 32 and 64 (4-wave workgroups), where it applies.
bool fast_plan_small(const AttnArgs& a, int dtype, FusedPlan& plan);
bool replay_plan(const AttnArgs& a, int dtype, ReplayPlan& plan);
hipError_t prepare_plan(const FusedPlan& plan);
void append_fast_resources(std::string& out);

}  // namespace fe
