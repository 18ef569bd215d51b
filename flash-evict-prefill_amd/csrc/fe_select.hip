// Token selection for gfx950: optional SnapKV average pooling, top-k, and the keep/evict
// mask plus ascending kept indices, honouring the reserved recent suffix.
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
// No sort anywhere. Scores map to order-preserving 32-bit keys; the (budget-recent)-th
// largest key T is found by a three-digit (11/11/10-bit) MSB radix select, and the kept set
// is {key > T} plus the lowest-index ties at T, so indices come out ascending from a block
// prefix sum. One 1024-thread workgroup per row. Two schedules, both reading the row from
// HBM once:
//   * rows of up to kLdsRowMax past scores: the row's keys are staged in LDS by one
//     coalesced pass, and the radix passes (restricted to a bracket taken from an evenly
//     spaced sample of the staged keys) and the ordered output pass run from LDS;
//   * longer rows (up to kBitRowMax): 512 evenly spaced 8-key segments are sampled first,
//     and two radix selects on the sample bracket T between two keys. One pass over the
//     row, with no workgroup barrier, then writes the mask of every key above the bracket
//     (kept) and below it (dropped), records the kept keys in an LDS bitmap, and holds the
//     keys inside the bracket as (key, index) candidates in LDS. T is resolved exactly among
//     the candidates (ties by index), their bits and mask bytes are set, and one ordered
//     pass over the bitmap writes the ascending indices. A bracket that misses (possible
//     only for unusual score layouts), and longer rows, take the radix passes over the row
//     in HBM: the result never depends on the sample.
#include <math.h>
#include <string>
#include <type_traits>

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

// The float whose order key is k, for keys from -inf (0x007fffff) to +inf (0xff800000);
// keys above +inf give a NaN pattern, with which every ordered compare is false. For
// thresholds between keys: v >= key_float(k) holds exactly when order_key(v) >= k, for every
// non-NaN v (-0 == +0 under IEEE compares, and key 0x7fffffff, which no float has, maps to
// -0 so that both zeros pass). FP32 denormals take part in compares as numbers.
__device__ __forceinline__ float key_float(u32 k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

constexpr int kSelThreads = 1024;                  // threads of a selection workgroup (one row)
constexpr int kSelWaves = kSelThreads / 64;
// Longest row staged whole in LDS. Up to 36864 keys fit (144 KiB); from 16K keys on the
// sampled schedule is faster (8 x 32768 rows: 27.4 against 29.9 us), its single pass
// beating the LDS schedule's bracket, three radix passes and ordered pass over every key.
#ifndef FE_SEL_LDS_ROW_MAX
#define FE_SEL_LDS_ROW_MAX 16384
#endif
constexpr int kLdsRowMax = FE_SEL_LDS_ROW_MAX;
static_assert(kLdsRowMax <= 36864 && kLdsRowMax >= 4096, "LDS capacity; sampled rows hold at least kSamples keys");
constexpr int kSegs = 512, kSegLen = 8;            // sample of the long-row schedule
constexpr int kSamples = kSegs * kSegLen;
constexpr int kCandMax = 12288;                    // (key, index) candidates held in LDS
constexpr int kBitRowMax = 262144;                 // longest row of the sampled schedule (32 KiB bitmap)
constexpr int kTieList = 64;                       // ties at the threshold listed in LDS (more: radix select)

// The selection kernels synchronise through LDS with lds_barrier() (fe_common.h):
// __syncthreads() also waits for every outstanding global load and store of the wave, which
// would stall the row's streaming loads (and the mask stores) at each prefix sum. A full
// barrier is used only where global memory written by one thread is then read or
// overwritten by another.

// Inclusive prefix sum over the 64 lanes of a wave with DPP moves: shifts by 1, 2, 4 and 8
// lanes inside each 16-lane row, then the last lane of row r added to row r+1 (row_bcast:15,
// rows 1 and 3) and lane 31 to rows 2 and 3 (row_bcast:31). Lanes without a source add 0.
__device__ __forceinline__ int wave_inclusive_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);   // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);   // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);   // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);   // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);   // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);   // row_bcast:31
  return x;
}

// Inclusive running minimum / maximum over the 64 lanes of a wave, the same DPP pattern as
// wave_inclusive_scan (lanes without a source take the identity): lane 63 holds the wave's.
__device__ __forceinline__ u32 wave_inclusive_min(u32 x) {
  int v = (int)x;
  v = min((u32)v, (u32)__builtin_amdgcn_update_dpp(-1, v, 0x111, 0xf, 0xf, false));
  v = min((u32)v, (u32)__builtin_amdgcn_update_dpp(-1, v, 0x112, 0xf, 0xf, false));
  v = min((u32)v, (u32)__builtin_amdgcn_update_dpp(-1, v, 0x114, 0xf, 0xf, false));
  v = min((u32)v, (u32)__builtin_amdgcn_update_dpp(-1, v, 0x118, 0xf, 0xf, false));
  v = min((u32)v, (u32)__builtin_amdgcn_update_dpp(-1, v, 0x142, 0xa, 0xf, false));
  v = min((u32)v, (u32)__builtin_amdgcn_update_dpp(-1, v, 0x143, 0xc, 0xf, false));
  return (u32)v;
}
__device__ __forceinline__ u32 wave_inclusive_max(u32 x) {
  int v = (int)x;
  v = max((u32)v, (u32)__builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false));
  v = max((u32)v, (u32)__builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false));
  v = max((u32)v, (u32)__builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false));
  v = max((u32)v, (u32)__builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false));
  v = max((u32)v, (u32)__builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false));
  v = max((u32)v, (u32)__builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false));
  return (u32)v;
}

// Exclusive prefix sum over the threads of a selection workgroup; `total` receives the sum.
// tmp: kSelWaves ints, 16-byte aligned.
__device__ __forceinline__ int block_exclusive_scan(int v, int* tmp, int& total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int x = wave_inclusive_scan(v);
  if (lane == 63) tmp[w] = x;
  lds_barrier();
  int before = 0;
  total = 0;
#pragma unroll
  for (int i = 0; i < kSelWaves; ++i) {
    const int t = tmp[i];
    before += (i < w) ? t : 0;
    total += t;
  }
  lds_barrier();
  return before + x - v;
}

struct SelShared {
  u32 prefix;
  int kk;
  u32 eq;
};

// Radix select over n keys (key i = get(i)) for T = the K-th largest key (1 <= K <= n),
// need = how many keys equal to T are among the K largest, eq = how many keys equal T.
// Only keys in [lo, hi] are histogrammed; keys above hi are counted first. Returns false
// (T undetermined) when the K-th largest key lies outside [lo, hi]; the full range
// [0, 0xffffffff] always succeeds. The leading digits that lo and hi share are the same for
// every key in [lo, hi], so their passes are skipped.
//
// Three LDS-only barriers per pass: after the histogram (whose successor, in the other half
// of hist, is cleared meanwhile), after the per-wave sums of the bins each wave owns (every
// thread then finds the wave holding the K-th key from 16 sums), and after the digit, found
// by that wave alone, is published. hist: 2 x 2048 u32; tmp: 2 x kSelWaves ints.
template <typename Get>
__device__ __forceinline__ bool radix_select(Get get, int n, int K, u32 lo, u32 hi, u32* hist, int* tmp,
                                             SelShared* sh, u32& T, int& need, int& eq) {
  constexpr int ST = kSelThreads;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  u32 prefix = 0, pmask = 0, eq_total = 0;
  int kk = K;
  int first = 0;
  if ((lo >> 21) == (hi >> 21)) {
    first = 1;
    pmask = 0xffe00000u;
    if ((lo >> 10) == (hi >> 10)) {
      first = 2;
      pmask = 0xfffffc00u;
    }
    prefix = lo & pmask;
  }
  for (int i = tid; i < (first == 2 ? 1024 : 2048); i += ST) hist[(first & 1) * 2048 + i] = 0u;
  lds_barrier();
  for (int pass = first; pass < 3; ++pass) {
    const int shift = pass == 0 ? 21 : (pass == 1 ? 10 : 0);
    const int nb = pass == 2 ? 1024 : 2048;
    u32* h = hist + (pass & 1) * 2048;
    if (pass < 2) {
      // the next pass's histogram: its last reader finished before this pass began
      u32* hn = hist + ((pass + 1) & 1) * 2048;
      for (int i = tid; i < (pass + 1 == 2 ? 1024 : 2048); i += ST) hn[i] = 0u;
    }
    int above = 0;
#pragma unroll 8
    for (int i = tid; i < n; i += ST) {
      const u32 key = get(i);
      if (pass == first) above += key > hi ? 1 : 0;
      if (key >= lo && key <= hi && (key & pmask) == prefix) atomicAdd(&h[(key >> shift) & (u32)(nb - 1)], 1u);
    }
    lds_barrier();
    // wave w owns bins [nb - (w+1)*bpw, nb - w*bpw), lane l the bpl of them below
    // nb - 1 - w*bpw - l*bpl: wave 0, lane 0 hold the highest digits
    const int bpw = nb / kSelWaves, bpl = bpw / 64;
    const int top = nb - 1 - w * bpw - lane * bpl;
    int lsum = 0;
    for (int e = 0; e < bpl; ++e) lsum += (int)h[top - e];
    const int incl = wave_inclusive_scan(lsum);
    const int wa = pass == first ? wave_inclusive_scan(above) : 0;
    if (lane == 63) {
      tmp[w] = incl;
      tmp[kSelWaves + w] = wa;
    }
    lds_barrier();
    int total = 0, n_above = 0, cw = -1, before = 0;
#pragma unroll
    for (int i = 0; i < kSelWaves; ++i) {
      total += tmp[i];
      n_above += pass == first ? tmp[kSelWaves + i] : 0;
    }
    if (pass == first) kk = K - n_above;
    if (pass == first && (kk < 1 || kk > total)) return false;   // uniform: block totals
    {
      int c = 0;
#pragma unroll
      for (int i = 0; i < kSelWaves; ++i) {
        const int t = tmp[i];
        if (cw < 0 && c + t >= kk) {
          cw = i;
          before = c;
        }
        c += t;
      }
    }
    if (w == cw) {
      int c = before + incl - lsum;            // keys in the bins above this lane's
      if (c < kk && c + lsum >= kk) {
        for (int e = 0; e < bpl; ++e) {
          const int bin = top - e;
          const int hv = (int)h[bin];
          if (c < kk && c + hv >= kk) {
            sh->prefix = prefix | ((u32)bin << shift);
            sh->kk = kk - c;
            sh->eq = (u32)hv;
          }
          c += hv;
        }
      }
    }
    lds_barrier();
    prefix = sh->prefix;
    kk = sh->kk;
    eq_total = sh->eq;
    pmask |= (u32)(nb - 1) << shift;
  }
  T = prefix;
  need = kk;
  eq = (int)eq_total;
  return true;
}

// Bracket of a sample of kSamples keys (key i = get(i)): for sample ranks k_hi < k_lo
// (1-based, from the top), the prefixes of the k_hi-th and k_lo-th largest sample keys
// down to 22 bits below the prefix all samples share, from a first radix pass shared by
// both ranks and a second pass that counts both ranks' bins at once (rank 0 in the low,
// rank 1 in the high half of each 32-bit count; a sample holds at most 4096 keys, so the
// halves never carry into each other). key_hi is the largest key with the first prefix
// (keys above it rank above T with high probability), key_lo the smallest key with the
// second; without a rank the bracket is open on that side. Seven LDS barriers: the two
// scans use opposite halves of scan_tmp, so neither needs a barrier after its reads.
struct BracketShared {
  int bin[2], rest[2], sub[2];
};

// Exclusive block scan with one barrier: tmp (kSelWaves ints) must not be written again
// before a later barrier.
__device__ __forceinline__ int block_exclusive_scan_once(int v, int* tmp, int& total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int x = wave_inclusive_scan(v);
  if (lane == 63) tmp[w] = x;
  lds_barrier();
  int before = 0;
  total = 0;
#pragma unroll
  for (int i = 0; i < kSelWaves; ++i) {
    const int t = tmp[i];
    before += (i < w) ? t : 0;
    total += t;
  }
  return before + x - v;
}

template <typename Get>
__device__ __forceinline__ void sample_bracket(Get get, int k_hi, int k_lo, bool has_hi, bool has_lo, u32* hist,
                                               int* scan_tmp, BracketShared* sh, u32& key_hi, u32& key_lo) {
  static_assert(kSamples < 65536, "packed second-pass counts");
  constexpr int ST = kSelThreads;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int target[2] = {k_hi, k_lo};
  const bool live[2] = {has_hi, has_lo};
  const int hi_bin = 2047 - 2 * tid;            // thread t owns bins hi_bin, hi_bin - 1
  u32* hist2 = hist + 2048;                     // second pass, both ranks packed
  // The two 11-bit digits start right below the prefix all sample keys share (from their
  // minimum and maximum): for scores spread over a few binades the top 11 bits hold little
  // more than the exponent, and a histogram of them piles most samples into a few bins.
  u32 smin = 0xffffffffu, smax = 0u;
  for (int i = tid; i < kSamples; i += ST) {
    const u32 k = get(i);
    smin = min(smin, k);
    smax = max(smax, k);
  }
  smin = wave_inclusive_min(smin);
  smax = wave_inclusive_max(smax);
  if (lane == 63) {
    scan_tmp[w] = (int)smin;
    scan_tmp[kSelWaves + w] = (int)smax;
  }
  for (int i = tid; i < 2 * 2048; i += ST) hist[i] = 0u;
  lds_barrier();                                                      // 1
#pragma unroll
  for (int i = 0; i < kSelWaves; ++i) {
    smin = min(smin, (u32)scan_tmp[i]);
    smax = max(smax, (u32)scan_tmp[kSelWaves + i]);
  }
  const int plen = (smin ^ smax) ? __builtin_clz(smin ^ smax) : 32;   // shared leading bits
  int s0 = 32 - plen - 11;                      // first digit: bits [s0, s0 + 11)
  s0 = s0 < 11 ? 11 : (s0 > 21 ? 21 : s0);
  const u32 pmask = s0 == 21 ? 0u : ~0u << (s0 + 11);
  const u32 prefix = smin & pmask;
  const int s1 = s0 - 11;                       // second digit: bits [s1, s0)
  // pass 1: the first digit
  for (int i = tid; i < kSamples; i += ST) atomicAdd(&hist[(get(i) >> s0) & 2047u], 1u);
  lds_barrier();                                                      // 2
  int total;
  // scan_tmp[0, kSelWaves) was last read before barrier 2
  int cum = block_exclusive_scan_once((int)(hist[hi_bin] + hist[hi_bin - 1]), scan_tmp, total);   // 3
  for (int e = 0; e < 2; ++e) {
    const int bin = hi_bin - e, h = (int)hist[bin];
    for (int t = 0; t < 2; ++t)
      if (live[t] && cum < target[t] && cum + h >= target[t]) {
        sh->bin[t] = bin;
        sh->rest[t] = target[t] - cum;
      }
    cum += h;
  }
  lds_barrier();                                                      // 4
  // pass 2: the second digit of the sample keys in either rank's bin
  const int b0 = live[0] ? sh->bin[0] : -1, b1 = live[1] ? sh->bin[1] : -1;
  for (int i = tid; i < kSamples; i += ST) {
    const u32 key = get(i);
    const int d = (int)((key >> s0) & 2047u);
    const u32 add = (d == b0 ? 1u : 0u) + (d == b1 ? 65536u : 0u);
    if (add) atomicAdd(&hist2[(key >> s1) & 2047u], add);
  }
  lds_barrier();                                                      // 5
  // scan_tmp[kSelWaves, 2 kSelWaves) was last read before barrier 2
  int c = block_exclusive_scan_once((int)(hist2[hi_bin] + hist2[hi_bin - 1]), scan_tmp + kSelWaves, total);   // 6
  const int r0 = live[0] ? sh->rest[0] : 0, r1 = live[1] ? sh->rest[1] : 0;
  for (int e = 0; e < 2; ++e) {
    const int bin = hi_bin - e, h = (int)hist2[bin];
    const int c0 = c & 0xffff, h0 = h & 0xffff, c1 = (int)((u32)c >> 16), h1 = (int)((u32)h >> 16);
    if (c0 < r0 && c0 + h0 >= r0) sh->sub[0] = bin;
    if (c1 < r1 && c1 + h1 >= r1) sh->sub[1] = bin;
    c += h;
  }
  lds_barrier();                                                      // 7
  const u32 low = (1u << s1) - 1u;
  key_hi = has_hi ? (prefix | ((u32)sh->bin[0] << s0) | ((u32)sh->sub[0] << s1) | low) : 0xffffffffu;
  key_lo = has_lo ? (prefix | ((u32)sh->bin[1] << s0) | ((u32)sh->sub[1] << s1)) : 0u;
}

// Sample ranks bracketing the K-th largest of m keys: T is expected at rank
// r = K * kSamples / m of the sample; take r -+ d, d = 4 sqrt(r + 1) + 8 (about four
// standard deviations of the sample rank).
__device__ __forceinline__ void bracket_ranks(int K, int m, int& k_hi, int& k_lo, bool& has_hi, bool& has_lo) {
  const float r = (float)K * (float)kSamples / (float)m;
  const float d = 4.f * sqrtf(r + 1.f) + 8.f;
  k_hi = (int)floorf(r - d);
  k_lo = (int)ceilf(r + d);
  has_hi = k_hi >= 1;
  has_lo = k_lo <= kSamples;
}

// f[e] for a per-lane index e without indexing the register array (which would place it in
// scratch memory): a four-level select tree.
__device__ __forceinline__ float pick16(const float (&f)[16], int e) {
  // all-ones masks from the bits of e, opaque to the compiler so that the selects are not
  // folded back into an indexed access
  u32 m[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    m[k] = 0u - (((u32)e >> k) & 1u);
    asm volatile("" : "+v"(m[k]));
  }
  auto sel = [](u32 mk, float hi, float lo) {
    return __uint_as_float((__float_as_uint(hi) & mk) | (__float_as_uint(lo) & ~mk));
  };
  float a[8], b[4];
#pragma unroll
  for (int j = 0; j < 8; ++j) a[j] = sel(m[0], f[2 * j + 1], f[2 * j]);
#pragma unroll
  for (int j = 0; j < 4; ++j) b[j] = sel(m[1], a[2 * j + 1], a[2 * j]);
  return sel(m[3], sel(m[2], b[3], b[2]), sel(m[2], b[1], b[0]));
}

// Eight consecutive mask bytes at p (one 8-byte store when aligned and whole).
__device__ __forceinline__ void store_mask8(unsigned char* p, const bool (&keep)[8], int valid,
                                            unsigned char keep_v, unsigned char drop_v) {
  if (valid == 8 && ((uintptr_t)p & 7u) == 0) {
    unsigned long long w = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) w |= (unsigned long long)(keep[e] ? keep_v : drop_v) << (8 * e);
    *(unsigned long long*)p = w;
  } else {
    for (int e = 0; e < valid; ++e) p[e] = keep[e] ? keep_v : drop_v;
  }
}

// Ordered output pass: keep key > T plus the first `need_eq` keys equal to T (all of them
// when all_eq); mask bytes of [0, m) and the ascending kept indices (positions from block
// prefix sums over chunks of 8 keys per thread).
template <typename Get>
__device__ __forceinline__ void ordered_output(Get get, int m, int K, u32 T, int need_eq, bool all_eq,
                                               long long* irow, unsigned char* mrow, unsigned char keep_v,
                                               unsigned char drop_v, int* scan_tmp) {
  constexpr int ST = kSelThreads;
  const int tid = threadIdx.x;
  int out_base = 0, eq_base = 0;
  for (int c0 = 0; c0 < m; c0 += ST * 8) {
    const int i0 = c0 + tid * 8;
    bool gt[8], eq[8];
    int neq = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool valid = i0 + e < m;
      const u32 key = valid ? get(i0 + e) : 0u;
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
    if (irow) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (sel[e] && pos < K) irow[pos] = i0 + e;
        pos += sel[e] ? 1 : 0;
      }
    }
    if (mrow && i0 < m) store_mask8(mrow + i0, sel, min(8, m - i0), keep_v, drop_v);
  }
}

// The reserved suffix [m, m + recent) and, with nothing to select (K == 0), the dropped past.
__device__ __forceinline__ void write_suffix(int m, int K, int recent, long long* irow, unsigned char* mrow,
                                             unsigned char keep_v, unsigned char drop_v) {
  const int tid = threadIdx.x;
  if (K == 0 && mrow)
    for (int i = tid; i < m; i += kSelThreads) mrow[i] = drop_v;
  for (int j = tid; j < recent; j += kSelThreads) {
    if (irow) irow[K + j] = (long long)(m + j);
    if (mrow) mrow[m + j] = keep_v;
  }
}

// out[r, i] = (sum_{j=i-k/2}^{i+k/2} past[r, j], zeros outside [0, m)) / k, summed left to
// right (the order of torch's avg_pool kernels). Each 256-thread block stages its `tile`
// outputs' inputs (plus the k/2 halo on each side) in LDS once; the window sum is unrolled
// for the usual small k (KT > 0), a loop otherwise. The host picks the tile: kPoolTile
// outputs per block on large inputs, halved down to 256 until the grid has enough blocks to
// fill the chip (8 rows x 32K scores: 64 blocks of 4096 outputs took 9 us). The tile's loads
// are all issued before they are written to LDS (256 x 131072 scores with k = 5: 65 -> 44 us,
// about 6 TB/s of reads and writes).
constexpr int kPoolTile = 4096;
constexpr int kPoolMinTile = 256;
constexpr long long kPoolFillBlocks = 1024;
constexpr int kPoolHalo = 64;          // largest k/2 served from LDS (k <= 129); larger k reads HBM
template <int KT>
__global__ __launch_bounds__(256) void avg_pool_kernel(const float* s, long long rs, int m, int k,
                                                       long long blocks_per_row, int ntile, float* out) {
  __shared__ float tile[kPoolTile + 2 * kPoolHalo];
  const long long row = (long long)blockIdx.x / blocks_per_row;
  const int i0 = (int)(((long long)blockIdx.x - row * blocks_per_row) * ntile);
  const float* x = s + row * rs;
  if (KT > 0) k = KT;
  const int half = k >> 1;
  float* o = out + row * (long long)m;
  if (half <= kPoolHalo) {
    const int span = min(ntile, m - i0) + 2 * half;
    // every load of the thread's share is issued before the first LDS write: written as one
    // loop, each iteration waited for its own load (vmcnt(0)) before the next was issued
    constexpr int kLoads = (kPoolTile + 2 * kPoolHalo + 255) / 256;
    float v[kLoads];
#pragma unroll
    for (int r = 0; r < kLoads; ++r) {
      const int t = (int)threadIdx.x + 256 * r;
      const int j = i0 - half + t;
      v[r] = (t < span && j >= 0 && j < m) ? x[j] : 0.f;
    }
#pragma unroll
    for (int r = 0; r < kLoads; ++r) {
      const int t = (int)threadIdx.x + 256 * r;
      if (t < span) tile[t] = v[r];
    }
    __syncthreads();
    for (int t = threadIdx.x; t < ntile; t += 256) {
      const int i = i0 + t;
      if (i >= m) break;
      // left to right over the window; the zero padding adds exact zeros
      float acc = 0.f;
      if constexpr (KT > 0) {
#pragma unroll
        for (int j = 0; j < KT; ++j) acc += tile[t + j];
      } else {
        for (int j = 0; j < k; ++j) acc += tile[t + j];
      }
      o[i] = acc / (float)k;
    }
  } else {
    for (int t = threadIdx.x; t < ntile; t += 256) {
      const int i = i0 + t;
      if (i >= m) break;
      const int lo = i - half < 0 ? 0 : i - half;
      const int hi = i + half > m - 1 ? m - 1 : i + half;
      float acc = 0.f;
      for (int j = lo; j <= hi; ++j) acc += x[j];
      o[i] = acc / (float)k;
    }
  }
}

// Rows of up to kLdsRowMax past scores: stage the keys in LDS, select, write.
__global__ __launch_bounds__(kSelThreads) void select_lds_kernel(const float* src, long long src_stride, int m,
                                                                 int K, int recent, long long* idx, int budget,
                                                                 unsigned char* mask, long long mask_stride,
                                                                 int invert) {
  constexpr int ST = kSelThreads;
  __shared__ u32 keys[kLdsRowMax];
  __shared__ u32 hist[2 * 2048];
  __shared__ __attribute__((aligned(16))) int scan_tmp[2 * kSelWaves];
  __shared__ SelShared sh;
  __shared__ BracketShared bsh;
  const int tid = threadIdx.x;
  const long long row = blockIdx.x;
  const float* x = src + row * src_stride;
  long long* irow = idx ? idx + row * (long long)budget : nullptr;
  unsigned char* mrow = mask ? mask + row * mask_stride : nullptr;
  const unsigned char keep_v = invert ? 0 : 1, drop_v = invert ? 1 : 0;
  if (K > 0) {
    // 16-byte loads, four in flight per thread before any LDS store
    if (((uintptr_t)x & 15u) == 0) {
      const int m4 = m & ~3;
      for (int b = 4 * tid; b < m4; b += 4 * ST * 4) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          // unconditional load (an index past the end rereads key 0 and is not stored), so
          // that the four loads stay in flight together
          const int i = b + u * 4 * ST;
          v[u] = *(const float4*)(x + (i < m4 ? i : 0));
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int i = b + u * 4 * ST;
          if (i < m4) {
            keys[i] = order_key(v[u].x);
            keys[i + 1] = order_key(v[u].y);
            keys[i + 2] = order_key(v[u].z);
            keys[i + 3] = order_key(v[u].w);
          }
        }
      }
      for (int i = m4 + tid; i < m; i += ST) keys[i] = order_key(x[i]);
    } else {
      for (int i = tid; i < m; i += ST) keys[i] = order_key(x[i]);
    }
    lds_barrier();
    u32 T;
    int need, eq;
    auto lds_key = [&](int i) { return keys[i]; };
    // Long rows: bracket T from an evenly spaced sample of the staged keys, so the radix
    // passes histogram only the keys inside the bracket (real scores crowd a few top-digit
    // bins, and LDS atomics on one bin serialise); a bracket that misses T takes the
    // passes over every key.
    bool found = false;
    if (m > 4 * kSamples) {
      int k_hi, k_lo;
      bool has_hi, has_lo;
      bracket_ranks(K, m, k_hi, k_lo, has_hi, has_lo);
      u32 key_hi, key_lo;
      auto s_key = [&](int i) { return keys[(int)(((long long)i * m) >> 12)]; };   // kSamples = 4096
      sample_bracket(s_key, k_hi, k_lo, has_hi, has_lo, hist, scan_tmp, &bsh, key_hi, key_lo);
      found = radix_select(lds_key, m, K, key_lo, key_hi, hist, scan_tmp, &sh, T, need, eq);
    }
    if (!found) radix_select(lds_key, m, K, 0u, 0xffffffffu, hist, scan_tmp, &sh, T, need, eq);
    ordered_output(lds_key, m, K, T, need, eq == need, irow, mrow, keep_v, drop_v, scan_tmp);
  }
  write_suffix(m, K, recent, irow, mrow, keep_v, drop_v);
}

// Rows longer than kLdsRowMax (up to kBitRowMax): sample bracket, one classifying pass,
// exact resolution among the candidates, indices from a bitmap of the kept keys.
//
// The classifying pass needs no workgroup barrier: every thread classifies its own chunks
// of 16 keys, records their kept bits in an LDS bitmap (one 16-bit word per chunk), counts
// them, and appends its candidates to the LDS pool at a slot its wave reserves with one LDS
// atomic. Candidates land in no particular order; ties at the threshold are then broken by
// index: up to kTieList tied candidates are listed and ranked by index directly (a second
// radix select over the indices took 6 us of a 42 us row), more by a second radix select
// over the tied candidates' indices. The ascending kept
// indices come from one ordered pass over the bitmap (a single block prefix sum). Rows the
// bitmap cannot hold, and brackets that miss, take the radix passes over HBM.
__global__ __launch_bounds__(kSelThreads) void select_sample_kernel(const float* src, long long src_stride, int m,
                                                                    int K, int recent, long long* idx, int budget,
                                                                    unsigned char* mask, long long mask_stride,
                                                                    int invert) {
  constexpr int ST = kSelThreads;
  constexpr int CH = 16;                       // keys per thread per classifying step
  static_assert(kBitRowMax / 32 >= kSamples, "the bitmap's LDS also holds the sample");
  __shared__ u32 work[kBitRowMax / 32];        // the sample, then the bitmap of kept keys
  __shared__ u32 hist[2 * 2048];
  __shared__ u32 ckey[kCandMax];               // candidate keys
  __shared__ int cidx[kCandMax];               // candidate indices
  __shared__ __attribute__((aligned(16))) int scan_tmp[2 * kSelWaves];
  __shared__ SelShared sh;
  __shared__ BracketShared bsh;
  __shared__ int n_cand_lds;
  const int tid = threadIdx.x, lane = tid & 63;
  const long long row = blockIdx.x;
  const float* x = src + row * src_stride;
  long long* irow = idx ? idx + row * (long long)budget : nullptr;
  unsigned char* mrow = mask ? mask + row * mask_stride : nullptr;
  const unsigned char keep_v = invert ? 0 : 1, drop_v = invert ? 1 : 0;
  auto hbm_key = [&](int i) { return order_key(x[i]); };

  bool bracketed = K > 0 && m <= kBitRowMax;
  int n_def = 0, n_cand = 0;
  u32 key_hi = 0u, key_lo = 0u;                // the bracket
  u32 c_lo = 0xffffffffu, c_hi = 0u;            // range of the candidate keys (per thread, then all)
  if (bracketed) {
    if (tid == 0) n_cand_lds = 0;
    // ---- sample: thread t reads keys 4(t%2) .. +3 of segment t/2. Short segments keep the
    // sample close to uniform: a dense run of large scores (the recent tokens of an
    // importance row) then takes no more of the sample than of the row. The loads are
    // issued before the streaming pass's first chunks, so they do not queue behind them.
    float sv[4];
    auto sample_load = [&]() __attribute__((always_inline)) {
      const int seg = tid >> 1, off = (tid & 1) * 4;
      const long long start = (long long)seg * (m - kSegLen) / (kSegs - 1);
#pragma unroll
      for (int e = 0; e < 4; ++e) sv[e] = x[start + off + e];
    };
    auto bracket = [&]() __attribute__((always_inline)) {
      // opaque to the compiler: it would otherwise hoist the first use of the sample (part
      // of order_key) above the branch between the aligned and unaligned loops, waiting
      // for the sample before the streaming pass's loads are issued
      asm volatile("" : "+v"(sv[0]), "+v"(sv[1]), "+v"(sv[2]), "+v"(sv[3]));
#pragma unroll
      for (int e = 0; e < 4; ++e) work[4 * tid + e] = order_key(sv[e]);
      lds_barrier();
      // ---- bracket: T is expected at sample rank r = K * kSamples / m; take ranks r -+ d,
      // d = 4 sqrt(r + 1) + 8 (about four standard deviations of the sample rank)
      int k_hi, k_lo;
      bool has_hi, has_lo;
      bracket_ranks(K, m, k_hi, k_lo, has_hi, has_lo);
      auto s_key = [&](int i) { return work[i]; };
      sample_bracket(s_key, k_hi, k_lo, has_hi, has_lo, hist, scan_tmp, &bsh, key_hi, key_lo);
    };
    // the kept-key bitmap shares `work` with the sample, which bracket() consumes first
    unsigned short* bits16 = (unsigned short*)work;

    // ---- classify every key once: above the bracket kept, below dropped, inside a candidate.
    // Two chunks ahead of the one being classified are in flight (16-byte loads, 128 bytes
    // per thread, 128 KiB per workgroup). No load sits under a branch, per-lane or uniform:
    // the compiler waits for a load at the end of the branch around it, which would
    // serialise the prefetch. So the aligned and unaligned rows run separate instances of
    // the loop, and a fetch past the end of the row rereads its first keys (a valid
    // address), which are then ignored.
    int n_keep = 0;                               // this thread's kept keys
    // Classification by float compares against the bracket: kept iff key > key_hi, i.e.
    // v >= g_hi with g_hi = key_float(key_hi + 1), or v NaN while the bracket is bounded
    // above; candidate iff key_lo <= key <= key_hi, i.e. v >= g_lo and not kept, or v NaN
    // with the bracket open above (NaN's key is the largest).
    bool nan_kept = false;
    float g_hi = 0.f, g_lo = 0.f;
    auto thresholds = [&]() __attribute__((always_inline)) {
      nan_kept = key_hi != 0xffffffffu;
      g_hi = nan_kept ? key_float(key_hi + 1u) : __builtin_nanf("");
      g_lo = key_lo <= 0x007fffffu ? -__builtin_huge_valf() : key_float(key_lo);
    };
    constexpr int STEP = ST * CH;
    auto classify_row = [&](auto aligned) __attribute__((always_inline)) {
      constexpr bool VEC = decltype(aligned)::value;
      float4 buf0[CH / 4], buf1[CH / 4];
      auto fetch = [&](float4 (&b)[CH / 4], int c0) __attribute__((always_inline)) {
        if constexpr (VEC) {
          const int i0 = c0 + tid * CH;
          const int ii = i0 + CH <= m ? i0 : 0;
#pragma unroll
          for (int u = 0; u < CH / 4; ++u) b[u] = *(const float4*)(x + ii + 4 * u);
        }
      };
      auto classify = [&](float4 (&b)[CH / 4], int c0) __attribute__((always_inline)) {
        const int i0 = c0 + tid * CH;
        float f[CH];
        if (VEC && i0 + CH <= m) {
#pragma unroll
          for (int u = 0; u < CH / 4; ++u) {
            f[4 * u] = b[u].x;
            f[4 * u + 1] = b[u].y;
            f[4 * u + 2] = b[u].z;
            f[4 * u + 3] = b[u].w;
          }
        } else {
#pragma unroll
          for (int e = 0; e < CH; ++e) f[e] = i0 + e < m ? x[i0 + e] : 0.f;
        }
        fetch(b, c0 + 2 * STEP);
        // bit e of kept / cand: key i0 + e is above / inside the bracket
        u32 kept = 0u, cand = 0u;
#pragma unroll
        for (int e = 0; e < CH; ++e) {
          const float v = f[e];
          const bool nan = v != v;
          const bool ge_hi = v >= g_hi;
          kept |= ((nan && nan_kept) || ge_hi ? 1u : 0u) << e;
          cand |= ((nan && !nan_kept) || (v >= g_lo && !ge_hi) ? 1u : 0u) << e;
        }
        const int nv = m - i0;                 // keys of this chunk inside the row
        const u32 vmask = nv >= CH ? 0xffffu : (nv > 0 ? (1u << nv) - 1u : 0u);
        kept &= vmask;
        cand &= vmask;
        if (i0 < m) bits16[i0 >> 4] = (unsigned short)kept;
        n_keep += __builtin_popcount(kept);
        // candidates: a slot range per wave from one LDS atomic; most chunks of a wave hold none
        const int nc = __builtin_popcount(cand);
        if (__any(nc != 0)) {
          const int incl = wave_inclusive_scan(nc);
          int base = 0;
          if (lane == 63) base = atomicAdd(&n_cand_lds, incl);
          int pc = __builtin_amdgcn_readlane(base, 63) + incl - nc;
          // a lane holds few candidates: visit its set bits only
          for (u32 c = cand; c != 0u; c &= c - 1u, ++pc) {
            const int e = __builtin_ctz(c);
            if (pc < kCandMax) {
              const u32 ck = order_key(pick16(f, e));
              ckey[pc] = ck;
              c_lo = min(c_lo, ck);
              c_hi = max(c_hi, ck);
              cidx[pc] = i0 + e;
            }
          }
        }
        if (mrow) {
#pragma unroll
          for (int h = 0; h < CH / 8; ++h) {
            const int j0 = i0 + 8 * h;
            if (j0 + 8 <= m && ((uintptr_t)(mrow + j0) & 7u) == 0) {
              // spread the 8 kept bits of this group into 8 bytes of 0/1
              unsigned long long w = (unsigned long long)((kept >> (8 * h)) & 0xffu) * 0x0101010101010101ull;
              w &= 0x8040201008040201ull;
              w = ((w + 0x7f7f7f7f7f7f7f7full) & 0x8080808080808080ull) >> 7;
              *(unsigned long long*)(mrow + j0) = keep_v ? w : w ^ 0x0101010101010101ull;
            } else {
              for (int e = 0; e < 8 && j0 + e < m; ++e)
                mrow[j0 + e] = ((kept >> (8 * h + e)) & 1u) ? keep_v : drop_v;
            }
          }
        }
      };
      // the first two chunks' loads are in flight while the sample is bracketed
      sample_load();
      fetch(buf0, 0);
      fetch(buf1, STEP);
      bracket();
      thresholds();
      for (int c0 = 0; c0 < m; c0 += 2 * STEP) {
        classify(buf0, c0);
        if (c0 + STEP < m) classify(buf1, c0 + STEP);
      }
    };
    if (((uintptr_t)x & 15u) == 0)
      classify_row(std::true_type{});
    else
      classify_row(std::false_type{});
    // full barrier: the pass's mask stores must be complete before candidates rewrite bytes
    __syncthreads();
    {
      // kept count, and the range of the candidate keys: the radix select below skips the
      // digits all candidates share (with the bracket open above, the bracket's own ends
      // share none, and a first pass would pile every candidate into one histogram bin)
      const int w = tid >> 6;
      const int x = wave_inclusive_scan(n_keep);
      const u32 wlo = wave_inclusive_min(c_lo), whi = wave_inclusive_max(c_hi);
      if (lane == 63) {
        scan_tmp[w] = x;
        scan_tmp[kSelWaves + w] = (int)wlo;
        hist[w] = whi;                           // free until the radix select clears it
      }
      lds_barrier();
      n_def = 0;
#pragma unroll
      for (int i = 0; i < kSelWaves; ++i) {
        n_def += scan_tmp[i];
        c_lo = min(c_lo, (u32)scan_tmp[kSelWaves + i]);
        c_hi = max(c_hi, hist[i]);
      }
      lds_barrier();
    }
    n_cand = n_cand_lds;
    bracketed = n_def <= K && n_def + n_cand >= K && n_cand <= kCandMax;
  }

  if (K > 0 && !bracketed) {
    // fallback: radix passes over the row in HBM, rewriting every mask byte and index (the
    // full barrier orders those rewrites after the classifying pass's stores)
    __syncthreads();
    u32 T;
    int need, eq;
    radix_select(hbm_key, m, K, 0u, 0xffffffffu, hist, scan_tmp, &sh, T, need, eq);
    ordered_output(hbm_key, m, K, T, need, eq == need, irow, mrow, keep_v, drop_v, scan_tmp);
  } else if (K > 0) {
    const int K2 = K - n_def;                  // candidates still to keep
    if (K2 > 0) {
      u32 T, T2 = 0u;
      int need, eq;
      auto c_key = [&](int j) { return ckey[j]; };
      radix_select(c_key, n_cand, K2, c_lo, c_hi, hist, scan_tmp, &sh, T, need, eq);
      const bool all_eq = eq == need;
      // ties at T keep the `need` lowest indices among them. A few ties (the usual case)
      // are listed in LDS and each tied candidate counts the listed indices below its own;
      // many take a radix select over ~index (the `need` largest).
      const bool tie_list = !all_eq && eq <= kTieList;
      int* tie_idx = (int*)hist;                 // free: radix_select's reads of hist are behind its last barrier
      if (tie_list) {
        if (tid == 0) n_cand_lds = 0;            // every thread read n_cand before radix_select's barriers
        lds_barrier();
        for (int j = tid; j < n_cand; j += ST) {
          if (ckey[j] == T) {
            const int s = atomicAdd(&n_cand_lds, 1);
            if (s < kTieList) tie_idx[s] = cidx[j];
          }
        }
        lds_barrier();
      } else if (!all_eq) {
        auto tie_key = [&](int j) { return ckey[j] == T ? ~(u32)cidx[j] : 0u; };
        int need2, eq2;
        radix_select(tie_key, n_cand, need, 0u, 0xffffffffu, hist, scan_tmp, &sh, T2, need2, eq2);
      }
      auto tie_kept = [&](int ci) -> bool {
        if (!tie_list) return ~(u32)ci >= T2;
        int below = 0;
        for (int t = 0; t < eq; ++t) below += tie_idx[t] < ci ? 1 : 0;
        return below < need;
      };
      u32* bits = work;
      for (int j = tid; j < n_cand; j += ST) {
        const u32 key = ckey[j];
        const int ci = cidx[j];
        if (key > T || (key == T && (all_eq || tie_kept(ci)))) {
          atomicOr(&bits[ci >> 5], 1u << (ci & 31));
          if (mrow) mrow[ci] = keep_v;
        }
      }
      lds_barrier();
    }
    if (irow) {
      // ascending kept indices: thread t owns bitmap words [t*wpt, (t+1)*wpt)
      const u32* bits = work;
      const int words = (m + 31) >> 5;
      const int wpt = (words + ST - 1) / ST;
      const int w0 = tid * wpt, w1 = min(words, w0 + wpt);
      auto word = [&](int w) -> u32 {
        const u32 v = bits[w];
        const int valid = m - 32 * w;          // the last word's bits past m are not written
        return valid >= 32 ? v : (v & ((1u << valid) - 1u));
      };
      int cnt = 0;
      for (int w = w0; w < w1; ++w) cnt += __builtin_popcount(word(w));
      int total;
      int pos = block_exclusive_scan(cnt, scan_tmp, total);
      for (int w = w0; w < w1; ++w) {
        u32 v = word(w);
        while (v) {
          const int bit = __builtin_ctz(v);
          if (pos < K) irow[pos] = 32 * w + bit;
          ++pos;
          v &= v - 1u;
        }
      }
    }
  }
  write_suffix(m, K, recent, irow, mrow, keep_v, drop_v);
}

namespace {

struct SelKernel {
  const void* fn;
  const char* name;
};

const SelKernel kSelKernels[] = {
    {(const void*)avg_pool_kernel<0>, "avg_pool"},
    {(const void*)select_lds_kernel, "select_lds"},
    {(const void*)select_sample_kernel, "select_sample"},
};

size_t pool_bytes(int64_t rows, int64_t n, int64_t budget, int64_t recent, int pool_kernel) {
  return pool_kernel > 1 && budget > recent ? (size_t)rows * (size_t)(n - recent) * sizeof(float) : 0;
}

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
  if (rows <= 0 || n <= 0 || recent < 0 || recent > n || budget < recent || budget > n) return 0;
  return pool_bytes(rows, n, budget, recent, pool_kernel);
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
  const size_t pbytes = pool_bytes(rows, n, budget, recent, pool_kernel);
  if (pbytes) {
    if (!workspace || workspace_bytes < pbytes) {
      set_error("fe_select: pooling needs a workspace of fe_select_workspace_bytes() bytes");
      return FE_ERR_WORKSPACE;
    }
    int ntile = kPoolTile;
    while (ntile > kPoolMinTile && rows * ((m + ntile - 1) / ntile) < kPoolFillBlocks) ntile /= 2;
    const long long bpr = (m + ntile - 1) / ntile;
    if (bpr * rows > 0x7fffffffLL) {
      set_error("fe_select: pooling grid too large");
      return FE_ERR_UNSUPPORTED;
    }
    const void* pool_fn = pool_kernel == 3 ? (const void*)avg_pool_kernel<3>
                          : pool_kernel == 5 ? (const void*)avg_pool_kernel<5>
                          : pool_kernel == 7 ? (const void*)avg_pool_kernel<7>
                          : pool_kernel == 9 ? (const void*)avg_pool_kernel<9>
                                             : (const void*)avg_pool_kernel<0>;
    int m_arg = (int)m, k_arg = pool_kernel;
    long long rs_arg = src_stride, bpr_arg = bpr;
    const float* s_arg = scores;
    float* o_arg = (float*)workspace;
    void* pargs[] = {&s_arg, &rs_arg, &m_arg, &k_arg, &bpr_arg, &ntile, &o_arg};
    hipError_t err = hipLaunchKernel(pool_fn, dim3((unsigned)(bpr * rows)), dim3(256), pargs, 0, stream);
    if (err == hipSuccess) err = hipGetLastError();
    if (err != hipSuccess) {
      set_error(std::string("fe_select: pool launch: ") + hipGetErrorString(err));
      return FE_ERR_HIP;
    }
    src = (const float*)workspace;
    src_stride = m;
  }
  if (m <= kLdsRowMax) {
    hipLaunchKernelGGL(select_lds_kernel, dim3((unsigned)rows), dim3(kSelThreads), 0, stream, src, src_stride, m, K,
                       (int)recent, (long long*)indices_out, (int)budget, (unsigned char*)mask_out, (long long)n,
                       invert ? 1 : 0);
  } else {
    hipLaunchKernelGGL(select_sample_kernel, dim3((unsigned)rows), dim3(kSelThreads), 0, stream, src, src_stride,
                       m, K, (int)recent, (long long*)indices_out, (int)budget, (unsigned char*)mask_out,
                       (long long)n, invert ? 1 : 0);
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error(std::string("fe_select: select launch: ") + hipGetErrorString(err));
    return FE_ERR_HIP;
  }
  return FE_OK;
}
