// Fast path of the fused prefill kernel for gfx950: head dims that are a multiple of 8 up to
// 256, on tile dims DP in {32, 64, ..., 256} (below DP the PARTIAL instantiation reads zeros
// past channel D and stores D channels); nonzero softmax scale (a negative one runs as |scale|
// on -Q), 16-byte unit-stride K/V rows, Q of any strides. Same mathematics as the generic kernel in fe_attn.hip (reference
// flash_evict/prefill.py:14-83); the differences are in data movement and instruction count:
//
//   * A workgroup is NW waves of one 32-query row tile each, all on one KV head (GQA
//     packing), so each K/V tile in LDS serves NW row tiles; waves 0-3 issue the DMA. At
//     D = 96 and 128 the kernels run 12 waves, three per SIMD; at D = 32 and 64, 8 (two
//     workgroups per CU); at 160 and 192, 8 (two per SIMD); at 224 and 256, 4 (one per SIMD).
//     At tile dims 96 and 128 the split schedule's attention-only traversal runs instead
//     attn_rt2_kernel: eight waves of two row tiles each (see there).
//   * The K/V buffers hold pairs of 64-key tiles up to tile dim 128 (one barrier per 128
//     keys), single tiles above it (one barrier per 64 keys).
//   * K and V tiles (64 keys) go HBM -> LDS with buffer_load ... lds (16 B per lane), no
//     staging registers; the tile's base and record count live in the buffer descriptor
//     (scalar arithmetic only), so rows past N read as zero and no VALU work is spent on
//     addresses. The attention kernel stores a tile channel-group-major (K: 32-byte groups,
//     V: 64-byte groups, each group's 64 rows contiguous), so each operand needs a single
//     per-lane LDS offset register and the fragment reads are bank-conflict free.
//   * Every LDS read uses that per-lane register plus an immediate (channel group, key
//     half, 16-key group, buffer, slot): the buffers are separate LDS objects and the tile
//     loop is unrolled over both buffers, so no address arithmetic remains in the loop, and
//     the waitcount pass can see that the DMA into one buffer does not alias reads of the
//     other (reads of tiles t, t+1 never wait for the DMA of t+2, t+3).
//   * The A operand of O^T = V^T P^T (eight keys of one channel per lane) comes straight
//     from the V tile (rows of one 32-channel tile) with two ds_read_b64_tr_b16 transposing
//     reads; the key order of the read matches the S^T accumulator row order that becomes
//     P^T.
//   * A row's reference max is the exact max of its first tile and changes only when a
//     later tile's probabilities could overflow; the output is normalised by the sum of the
//     probabilities as rounded for P@V (see t1_step), so O is rarely rescaled.
//   * Masked logits are set to -inf in place, so masking costs one compare/select per
//     element on diagonal and ragged tiles only.
#include <math.h>
#include <string>

#include "fe_attn.h"
#include "fe_internal.h"

namespace fe {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Raise the wave's issue priority around MFMA blocks so that, of the two waves sharing a
// SIMD, the one with matrix work ready issues it first while the other fills the MFMA
// shadow with its softmax VALU work.
#ifndef FE_SETPRIO
#define FE_SETPRIO 1
#endif
#if FE_SETPRIO
#define FE_PRIO_HI() __builtin_amdgcn_s_setprio(1)
#define FE_PRIO_LO() __builtin_amdgcn_s_setprio(0)
#else
#define FE_PRIO_HI() ((void)0)
#define FE_PRIO_LO() ((void)0)
#endif
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

template <int DP>
struct FastTile {
  static constexpr int BN = 64;                  // keys per tile
  static constexpr int CPR = DP / 8;             // 16-byte chunks per row
  static constexpr int ROWB = DP * 2;            // bytes per row
  static constexpr int TILE = BN * ROWB;         // bytes per K or V tile
  static constexpr int DMA_PER_WAVE = (BN * CPR) / 256;
  static constexpr int NDC = DP / 16;            // MFMA k-chunks of QK^T
  static constexpr int NDT = DP / 32;            // 32-channel tiles of O^T
};

// IEEE maximum (v_maximum3_f32): the operands are MFMA results or -inf, so the NaN-quieting
// canonicalisation that fmaxf implies is not needed.
__device__ __forceinline__ float vmax(float x, float y) { return __builtin_elementwise_maximum(x, y); }

__device__ __forceinline__ float half_swap_maximum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// DMA of one 64-key tile in channel-group-major order (fused_fast_kernel). The tile is
// column groups of GB bytes per row, each stored as 64 consecutive rows of GB bytes; a 1 KB
// block holds KPB = 1024 / GB rows of one group: block B is group B / BPG, rows
// (B % BPG) * KPB ... + KPB - 1 (BPG = 64 / KPB blocks per group). Wave wv moves blocks
// wv + 4r (r < DPW). BPG divides 4, so all of a wave's blocks start at the same row and
// their groups are 4 / BPG apart, 64 bytes of the global row: one buffer descriptor per wave
// (base at the first row and group, record count ending at row N) serves them all with
// soffset = 64r. Lane l fetches the same offset in every block (doff: row l / (GB/16) and
// a 16-byte chunk of the group), so one offset register serves the whole tile. Rows past N
// read as zero: a lane's offset reaches row N exactly when its row does, and 64r plus the
// group width never exceeds the row (64(DPW - 1) + GB <= 2D), so an in-range row is read
// whole. PARTIAL (a head dim D below the tile's DP, D a multiple of 8): a lane whose 16-byte
// chunk (channels g*GB/2 + dch .. +7 of block r's group g) starts at or past D takes an offset
// past the record count, so it reads zeros and touches no memory; rows are never read past
// their D channels, whatever the hardware does with the scalar offset.
template <int DPW, int GB, bool PARTIAL = false>
__device__ __forceinline__ void dma_tile_cm(const unsigned char* g, u32 rowb, u32 doff, int kb, int N,
                                            unsigned char* ldst, int wv, int D = 0, u32 dch = 0) {
  constexpr int KPB = 1024 / GB, BPG = 64 / KPB;
  static_assert(4 % BPG == 0 && (4 / BPG) * GB == 64, "one descriptor per wave");
  // recomputed per call: hoisting the per-block LDS addresses of every call site out of the
  // tile loop would hold dozens of scalar registers
  int w = wv;
  asm volatile("" : "+s"(w));
  const int k0 = kb + (w % BPG) * KPB;
  const int nrec = N > k0 ? (int)((u32)(N - k0) * rowb) : 0;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(g + (size_t)((u32)k0 * rowb) + (w / BPG) * GB), (short)0, nrec, 0x00020000);
  unsigned char* dst = ldst + w * 1024;
#pragma unroll
  for (int r = 0; r < DPW; ++r) {
    u32 off = doff;
    if constexpr (PARTIAL) {
      const u32 ch = (u32)((w / BPG + (4 / BPG) * r) * (GB / 2)) + dch;   // the lane's first channel
      off = ch < (u32)D ? doff : 0x7fffffffu;
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(dst + r * 4096), 16, off, 64 * r, 0, 0);
  }
}

// Four consecutive output channels d0 .. d0+3 of one row (w0: d0, d0+1; w1: d0+2, d0+3). Below
// the tile dim (PARTIAL) the row holds Dq channels: a group past Dq is not stored, and where Dq
// is not a multiple of 4 (rows then not 8-byte aligned) the channels are stored one by one.
template <bool PARTIAL>
__device__ __forceinline__ void store4(u16* op, int d0, int Dq, u32 w0, u32 w1) {
  if (!PARTIAL || ((Dq & 3) == 0 && d0 + 4 <= Dq)) {
    *(u32x2*)(op + d0) = (u32x2){w0, w1};
    return;
  }
  const u16 h[4] = {(u16)w0, (u16)(w0 >> 16), (u16)w1, (u16)(w1 >> 16)};
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (d0 + e < Dq) op[d0 + e] = h[e];
}

// The lane's index, recomputed where it is used: opaque to the compiler, which would
// otherwise keep values derived from it live across a loop and, at two or three waves per
// SIMD, spill them (each reload then waits behind the next tile's DMA).
__device__ __forceinline__ int lane_now() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// Work items. Without a queue a workgroup runs the one item blockIdx.x. The dynamic schedule
// launches as many workgroups as the chip holds at once (a.nstatic) and each loops over items:
// its first is blockIdx.x, and the hardware deals those over the XCDs in turn (workgroup b to
// XCD b % 8) and over each XCD's CUs in order, so no CU starts with several of the heaviest
// items. Items are numbered heaviest first, with consecutive numbers on different KV heads,
// and the rest are dealt to eight queues, one per XCD: queue x holds items x, x + 8, x + 16,
// ... past the first ones (with B*Hkv a multiple of 8, the KV heads h with h % 8 == x, whose
// K/V tiles that XCD's L2 then serves), heaviest first, in two parts: the heavy items below
// a.tail and the light ones from a.tail on (the last groups of items, holding a fixed share of
// the work, chosen by the host). A workgroup on XCD x (hardware register XCC_ID) takes the
// front of its own heavy part, then its own light part, then the light part of the nearest
// other queue with light items left, and only then the back of another queue's heavy part;
// it exits when every queue is empty. So each item goes to whichever CU frees up first within
// its XCD, without waiting for the hardware dispatcher (which starts workgroups in order and
// holds a free CU of one XCD until the next workgroup for another XCD has found room), and
// XCDs that run faster than the others (their clocks differ by several percent under these
// kernels) help the slower ones with light items: stealing heavy items instead, the fast XCDs
// ran dry while a slow XCD still held items of hundreds of microseconds, and the kernel ended
// up to 240 us after its first CUs went idle at the headline shape. The barrier before the
// fetch orders every wave's LDS reads of the previous item (and its read of the shared index)
// before the next item's first tile DMA and the next index. Returns a block-uniform index. wv
// is the wave's index in the workgroup (uniform); the lane index is taken opaquely, so nothing
// lane-derived is hoisted out of the caller's item loop and held across it.
__device__ __forceinline__ int queue_len(int nitems, int x) { return (nitems - x + 7) >> 3; }

// Counters of queue x, on its own 128-byte line: the heavy part's 64-bit word (items taken
// from its front in the low half, by the queue's own XCD, and from its back in the high half,
// by other XCDs) and the light part's word (items taken, by anyone). Every take adds one to one
// half in one atomic, so the takes of a part are totally ordered. A heavy take succeeds iff
// front + back < n (the part's items) before it, so the successful front takes are positions
// 0 .. F-1 and the back takes n-1 .. n-B with F + B <= n; a light take succeeds iff its
// counter was below the part's length. Every item is taken exactly once, and a failed take
// leaves that part exhausted for good.
__device__ __forceinline__ unsigned long long* heavy_word(const AttnArgs& a, int x) {
  return (unsigned long long*)(a.queue + kQueueStride * x);
}
__device__ __forceinline__ unsigned long long* light_word(const AttnArgs& a, int x) {
  return (unsigned long long*)(a.queue + kQueueStride * x + 2);
}

// The next item for a workgroup on XCD x, taken by wave 0 (uniform result; a.nitems when
// every queue is empty). Queue q's heavy items are positions [queue_len(nstatic, q),
// queue_len(tail, q)) and its light items [queue_len(tail, q), queue_len(nitems, q)); item =
// 8 * position + q.
__device__ __forceinline__ int take_item(const AttnArgs& a) {
  const int lane = lane_now();
  const int x = (int)(__builtin_amdgcn_s_getreg(kHwRegXccId) & 7u);
  int got = -1;
  if (lane == 0) {
    const int p0 = queue_len(a.nstatic, x), pt = queue_len(a.tail, x), n = pt - p0;
    const unsigned long long w = atomicAdd(heavy_word(a, x), 1ull);
    if ((int)(unsigned)w + (int)(w >> 32) < n) {
      got = 8 * (p0 + (int)(unsigned)w) + x;
    } else {
      const int j = (int)atomicAdd(light_word(a, x), 1ull);
      if (j < queue_len(a.nitems, x) - pt) got = 8 * (pt + j) + x;
    }
  }
  int item = __shfl(got, 0);
  // Other queues, nearest first: lanes 0-6 read queues x+1 .. x+7 at once, lane 0 takes from
  // the first with items left (light parts, then heavy ones). Each failed take leaves that
  // part exhausted for good, so at most seven rounds of each kind run.
  for (int heavy = 0; heavy < 2 && item < 0; ++heavy) {
    for (int round = 0; round < 7 && item < 0; ++round) {
      bool left = false;
      if (lane < 7) {
        const int qx = (x + 1 + lane) & 7;
        const int p0 = queue_len(a.nstatic, qx), pt = queue_len(a.tail, qx);
        if (heavy) {
          const unsigned long long w = __hip_atomic_load(heavy_word(a, qx), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          left = (int)(unsigned)w + (int)(w >> 32) < pt - p0;
        } else {
          const unsigned long long w = __hip_atomic_load(light_word(a, qx), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          left = (int)w < queue_len(a.nitems, qx) - pt;
        }
      }
      const unsigned long long m = __ballot(left);
      if (m == 0) break;
      const int qx = (x + __ffsll(m)) & 7;
      got = -1;
      if (lane == 0) {
        const int p0 = queue_len(a.nstatic, qx), pt = queue_len(a.tail, qx);
        if (heavy) {
          const unsigned long long w = atomicAdd(heavy_word(a, qx), 1ull << 32);
          const int bk = (int)(w >> 32);
          if ((int)(unsigned)w + bk < pt - p0) got = 8 * (pt - 1 - bk) + qx;
        } else {
          const int j = (int)atomicAdd(light_word(a, qx), 1ull);
          if (j < queue_len(a.nitems, qx) - pt) got = 8 * (pt + j) + qx;
        }
      }
      item = __shfl(got, 0);
    }
  }
  return item < 0 ? a.nitems : item;
}

// Item loop of the attention kernels: after the barrier (every wave done with the previous
// item's LDS tiles and the shared index), wave 0 takes the next item.
__device__ __forceinline__ int next_item(const AttnArgs& a, int* s_item, int wv) {
  __syncthreads();
  if (wv == 0) {
    const int item = take_item(a);
    if (lane_now() == 0) *s_item = item;
  }
  __syncthreads();
  return __builtin_amdgcn_readfirstlane(*s_item);
}

// One item per workgroup (the replay kernel, whose tile loop has no registers to spare for
// an item loop): the first a.nstatic workgroups run item blockIdx.x, the launch has more
// workgroups than items, and each later one takes an item from the queues when it starts
// (or exits, finding none).
__device__ __forceinline__ int block_item(const AttnArgs& a, int* s_item, int wv) {
  if (!a.queue || (int)blockIdx.x < a.nstatic) return (int)blockIdx.x;
  if (wv == 0) {
    const int item = take_item(a);
    if (lane_now() == 0) *s_item = item;
  }
  __syncthreads();
  return __builtin_amdgcn_readfirstlane(*s_item);
}

// Replay items of the attention kernels: lane 0 of the calling wave waits
// until attention item `dep` has published its rows' replay biases (its bit in a.done) and
// returns whether it has. The bias words are written and read as agent-scope relaxed atomics
// (write-through stores and loads that bypass a stale L2 line), the writer waits for its stores
// before its workgroup sets the bit, and the waiting lane's load of the bit completes before the
// workgroup barrier that precedes the bias loads, so a bias read after the bit is seen is the
// one written. Attention items are numbered before replay items in every queue and the window
// rows a replay item needs are the heaviest attention items, taken first, so the wait is short;
// it is bounded by about 17 us per key tile of the dependency (five times what a tile takes;
// a.wait_base + a.wait_per_tile polls of about 0.27 us),
// and when it runs out (the dependency's workgroup not resident, say, on a GPU another kernel
// shares) the caller computes the dependency itself: an attention item writes the same output
// and biases whoever runs it.
__device__ __forceinline__ bool wait_item_done(const AttnArgs& a, int dep, int dep_tiles) {
  bool ok = true;
  if (lane_now() == 0) {
    const unsigned bit = 1u << (dep & 31);
    unsigned* w = a.done + (dep >> 5);
    const int polls = a.wait_base + a.wait_per_tile * dep_tiles;
    ok = false;
    for (int spin = 0; spin < polls && !ok; ++spin) {
      ok = (__hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & bit) != 0;
      if (!ok) __builtin_amdgcn_s_sleep(8);
    }
  }
  return ok;
}

// NW waves of one row tile each (8: two waves per SIMD; 12: three, at D = 128, which then
// reads K fragments in two halves and V fragments without prefetch to fit 168 registers). FUSED adds the replay traversal (fe_prefill without a
// workspace); otherwise the kernel hands each row's replay bias to replay_fast_kernel.
// Waves per SIMD the fused_fast_kernel instantiation is built for: 12-wave workgroups three,
// 8-wave ones two, 4-wave ones one above tile dim 64 (tile dim 256: 128 accumulator and 64 Q
// registers per wave) and four at tile dims 32 and 64 (the small-grid kernel: four workgroups
// per CU, one wave of each per SIMD).
template <int NW, int DP>
struct FastOccupancy {
  static constexpr bool SMALL_GRID = NW == 4 && DP <= 128;
  static constexpr int WAVES_PER_EU = NW > 8 ? 3 : (NW > 4 ? 2 : (SMALL_GRID ? (DP <= 64 ? 4 : 2) : 1));
};

template <typename E, int DP, int NW, bool FUSED, bool PARTIAL>
__global__ __launch_bounds__(NW * 64, (FastOccupancy<NW, DP>::WAVES_PER_EU)) void fused_fast_kernel(const AttnArgs a) {
  typedef FastTile<DP> T;
  constexpr int BN = T::BN, NDC = T::NDC, NDT = T::NDT, TILE = T::TILE;
  constexpr int DPW = T::DMA_PER_WAVE;
  constexpr int KH = (NW > 8 || DP > 128) ? 2 : 1;   // K fragment reads per 32-key half
  // 64-key tiles per LDS buffer: two up to tile dim 128 (one barrier per pair of tiles), one
  // above it, where two double-buffered pairs of K and V tiles would not fit the LDS, and in
  // the small-grid kernel (32 KiB of LDS per workgroup at tile dim 64: four per CU)
  constexpr int SLOTS = (DP <= 128 && !FastOccupancy<NW, DP>::SMALL_GRID) ? 2 : 1;
  static_assert(NDC % KH == 0, "K fragment groups");
  static_assert(NW % 2 == 0 && NW >= 4, "row tiles per workgroup");
  constexpr float NEG_INF = -__builtin_huge_valf();
  constexpr float POS_INF = __builtin_huge_valf();

  // One LDS object per buffer: the waitcount pass can then tell that a tile's DMA (into
  // one buffer) and the fragment reads of the other buffer do not alias, and the objects'
  // addresses are link-time constants that fold into the reads' offset fields.
  // Two buffers per operand, each holding two consecutive 64-key tiles (slots 0 and 1).
  __shared__ __attribute__((aligned(1024))) unsigned char lds_k0[SLOTS * TILE], lds_k1[SLOTS * TILE],
      lds_v0[SLOTS * TILE], lds_v1[SLOTS * TILE];
  __shared__ float red[FUSED ? 2 * NW * BN : 1];  // [2][NW][BN] per-wave column sums

  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool dmaw = wv < 4;                      // waves 0-3 issue the tile DMA
  const int N = a.N;

  __shared__ int s_item, s_ready;
  // One work item; `return` ends it.
  auto run_item = [&](const int item) __attribute__((always_inline)) {
    const int lane = lane_now(), l32 = lane & 31, hh = lane >> 5;
    // The divisors of the item decode, taken opaquely: otherwise the compiler keeps their
    // reciprocals, computed once before the item loop, in registers across it.
    int BH = a.BH, G = a.G, Hkv = a.Hkv;
    asm volatile("" : "+s"(BH), "+s"(G), "+s"(Hkv));
    const int bh = (int)((unsigned)item % (unsigned)BH);
    const int wg = a.wg_bh - 1 - (int)((unsigned)item / (unsigned)BH);
    const int b = bh / Hkv, hkv = bh - b * Hkv;
    const int t_begin = wg * NW;
    const int t_end = min(a.tiles_bh, t_begin + NW);
    const int wg_q_hi = min(N, ((t_end - 1) / G + 1) * 32);
    const int kv_end = a.causal ? wg_q_hi : N;
    const int ntiles = (kv_end + BN - 1) / BN;

    // This wave's row tile: 32 query positions from q0 of query head `head`.
    const int t = t_begin + wv;
    const bool tv = t < t_end;
    const int tt = tv ? t : t_begin;
    const int q0 = (tt / G) * 32;
    const int head = hkv * G + (tt - (tt / G) * G);
    // last key this lane's query row may see (-1 for a padding tile); the smallest such limit
    // of the tile (tiles past it are masked) and the largest (tiles past it are skipped)
    const int qlim = !tv ? -1 : (a.causal ? min(q0 + l32, N - 1) : N - 1);
    const int lo_lim = !tv ? -1 : (a.causal ? min(q0, N - 1) : N - 1);
    const int wave_hi = !tv ? -1 : (a.causal ? min(q0 + 31, N - 1) : N - 1);

    // A negative scale runs as |scale| on -Q: the sign bits of Q flip at load, and
    // (-q).k = -(q.k) exactly in the FP32 accumulation, so the logits are those of scale * Q K^T
    const u32 qneg = a.neg_scale ? 0x80008000u : 0u;
    u32x4 qf[NDC];
    {
      const int qr = q0 + l32;
      const bool ok = tv && qr < N;
      const u16* qp = a.q + b * a.qs[0] + head * a.qs[1] + (long long)(ok ? qr : 0) * a.qs[2];
  #pragma unroll
      for (int c = 0; c < NDC; ++c) qf[c] = ok ? ((load8(qp, a.qs[3], 16 * c + 8 * hh, PARTIAL ? a.Dq : DP, a.qvec) & a.qmask) ^ qneg) : (u32x4){0u, 0u, 0u, 0u};
    }

    // Per-lane LDS byte offsets, one per operand, fixed for the kernel. The fragment, key
    // group, buffer and slot enter as instruction immediates.
    //   K tile: [chunk pair c][64 keys][32 B]. Fragment c of key 32s + l32 is chunk 2c + h
    //   (h = lane/32) at c*2048 + (32s + l32)*32 + 16*(h ^ key bit 3): the XOR puts keys k and
    //   k+8 in different halves of the 256-byte bank row, so the 16 lanes of a read phase hit
    //   every bank once.
    //   V tile: [channel tile dt][64 keys][64 B], unswizzled: four consecutive keys fill one
    //   256-byte bank row. The V^T fragment of channel tile dt, 16-key group c4, holds eight
    //   keys of channel 32dt + lane%32 in P^T slot order: slots 0-3 = keys 4h + 0..3 and slots
    //   4-7 = keys 8 + 4h + 0..3 (two transposing reads, + 512 B apart).
    const u32 koff = (u32)(l32 * 32 + ((hh ^ ((l32 >> 3) & 1)) << 4));
    u32 voff;
    {
      const int r = lane & 15, g = lane >> 4;
      voff = (u32)((4 * hh + (r >> 2)) * 64 + 32 * (g & 1) + 8 * (r & 3));
    }

    // Per-lane global offsets of the tile DMA (dma_tile_cm), the same for every block and
    // wave: K blocks are 32 keys x 2 chunks (lane l: key l/2, chunk l%2 XOR key bit 3, the
    // swizzle above), V blocks 16 keys x 4 chunks (lane l: key l/4, chunk l%4).
    const u32 krow = (u32)(a.ks[2] * 2), vrow = (u32)(a.vs[2] * 2);
    const u32 dk = (u32)(lane >> 1) * krow + (u32)(((lane & 1) ^ ((lane >> 4) & 1)) << 4);
    const u32 dv = (u32)(lane >> 2) * vrow + (u32)((lane & 3) << 4);
    const unsigned char* kg = (const unsigned char*)(a.k + b * a.ks[0] + hkv * a.ks[1]);
    const unsigned char* vg = (const unsigned char*)(a.v + b * a.vs[0] + hkv * a.vs[1]);
    // PARTIAL: the lanes' first channel within their K (16-channel) and V (32-channel) group
    const u32 dchk = (u32)(((lane & 1) ^ ((lane >> 4) & 1)) << 3), dchv = (u32)((lane & 3) << 3);
    auto dma_k = [&](int kb, unsigned char* ldst) { dma_tile_cm<DPW, 32, PARTIAL>(kg, krow, dk, kb, N, ldst, wv, a.D, dchk); };
    auto dma_v = [&](int kb, unsigned char* ldst) { dma_tile_cm<DPW, 64, PARTIAL>(vg, vrow, dv, kb, N, ldst, wv, a.D, dchv); };

    // K fragments of keys 32*s + l32 from buffer BUF, slot SLOT: chunk pairs h*NDC/KH .. +NDC/KH
    auto k_frags = [&](int BUF, int SLOT, int s, int h, u32x4(&kf)[NDC / KH]) __attribute__((always_inline)) {
      const unsigned char* kt = (BUF == 0 ? lds_k0 : lds_k1) + SLOT * TILE + s * 1024 + koff;
  #pragma unroll
      for (int c = 0; c < NDC / KH; ++c) kf[c] = *(const u32x4*)(kt + (h * (NDC / KH) + c) * 2048);
    };
    // V^T fragment of channel tile dt, 16-key group c4, buffer BUF, slot SLOT
    auto v_frag = [&](int BUF, int SLOT, int c4, int dt) __attribute__((always_inline)) -> u32x4 {
      const unsigned char* vt = (BUF == 0 ? lds_v0 : lds_v1) + SLOT * TILE + dt * 4096 + c4 * 1024 + voff;
      const s16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds_ptr_t)vt);
      const s16x4 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds_ptr_t)(vt + 512));
      const u32x2 ux = __builtin_bit_cast(u32x2, x), uy = __builtin_bit_cast(u32x2, y);
      return (u32x4){ux[0], ux[1], uy[0], uy[1]};
    };

    f32x16 o[NDT];
    float m_run = NEG_INF;                         // reference max of the row (log2 units)
    float l_run = 0.f;                             // FP32 sum of the probabilities (replay rows)
    float l_rnd = 0.f;                             // sum of the probabilities as rounded for P@V
    float nm = 0.f;                                // -m_run, or 0 while m_run is -inf
    bool fresh = true;                             // no tile of this row tile seen yet
    // Only rows the replay visits need the FP32 sum (their replay bias); it is wave-uniform.
    const bool exact_l = a.score && tv && q0 + 31 >= a.win_lo;
    u32 ones2;                                     // (1, 1) of the element type, for E::sum2
    asm volatile("s_mov_b32 %0, %1" : "=s"(ones2) : "i"(E::kOnes2));
  #pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[dt] = (f32x16){};

    // ---------------- traversal 1
    // Tiles are processed in pairs per barrier: buffer BUF holds tiles it and it+1 while the
    // DMA fills the other buffer with tiles it+2 and it+3.
    auto t1_sync = [&](int it, int BUF) __attribute__((always_inline)) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (dmaw) {
  #pragma unroll
        for (int sl = 0; sl < SLOTS; ++sl)
          if (it + SLOTS + sl < ntiles) {
            dma_k((it + SLOTS + sl) * BN, (BUF == 0 ? lds_k1 : lds_k0) + sl * TILE);
            dma_v((it + SLOTS + sl) * BN, (BUF == 0 ? lds_v1 : lds_v0) + sl * TILE);
          }
      }
    };
    // One 64-key tile: S^T = K Q^T (two 32-key accumulators; lanes hold queries), mask on
    // diagonal and ragged tiles, P = exp2(S*scale - m) rounded to the input dtype, O^T += V^T P^T.
    //
    // Reference max. The row's first tile sets m to its exact max, so that tile's largest
    // probability is exactly 1 and every row sum is at least 1. Later tiles keep m; their
    // probabilities may exceed 1 where the row's max has risen. The output is O divided by
    // l_rnd, the sum of the probabilities exactly as rounded for the P@V product, so a row
    // dominated by one key returns that key's value whatever m is (dividing by the unrounded
    // sum would leave that key's rounding error, up to 2^-8 relative in bf16, in the output).
    // The replay bias needs the FP32 sum of the unrounded probabilities (l_run, replay rows
    // only): b = m + log2 l_run does not depend on the choice of m. A tile some lane of which
    // sums to more than E::kMaxTileSum (inf included) takes a new reference (its exact max plus
    // E::kRescaleHeadroom), rescales O and both sums and recomputes its probabilities, which are
    // then at most 1. For random inputs that happens on a few percent of tiles, where following
    // the exact running max rescaled O on ~40% of them, and no tile spends instructions on a row
    // max.
    auto exact_max = [&](const f32x16(&sacc)[2]) __attribute__((always_inline)) -> float {
      // max over the 32 keys of this lane and the other half-wave: two chains of three-input
      // maxima (v_maximum3_f32, two new values each), 16 instructions for 32 values
      float mc[2];
  #pragma unroll
      for (int s = 0; s < 2; ++s) {
        mc[s] = vmax(vmax(sacc[s][0], sacc[s][1]), sacc[s][2]);
  #pragma unroll
        for (int i = 3; i < 15; i += 2) mc[s] = vmax(vmax(mc[s], sacc[s][i]), sacc[s][i + 1]);
      }
      return half_swap_maximum(vmax(vmax(mc[0], mc[1]), vmax(sacc[0][15], sacc[1][15]))) * a.abs_scale_log2;
    };
    // S^T of one tile into sacc, masked on diagonal and ragged tiles
    auto qk_tile = [&](int kb, int BUF, int SLOT, f32x16(&sacc)[2]) __attribute__((always_inline)) {
  #pragma unroll
      for (int s = 0; s < 2; ++s) {
  #pragma unroll
        for (int h = 0; h < KH; ++h) {
          u32x4 kf[NDC / KH];
          k_frags(BUF, SLOT, s, h, kf);
          FE_PRIO_HI();
  #pragma unroll
          for (int c = 0; c < NDC / KH; ++c) {
            const int cc = h * (NDC / KH) + c;
            sacc[s] = cc == 0 ? E::mfma(kf[c], qf[0], (f32x16){}) : E::mfma(kf[c], qf[cc], sacc[s]);
          }
          FE_PRIO_LO();
        }
      }
      if (kb + BN - 1 > lo_lim) {
        // key kb + 32s + 8(i/4) + 4h + i%4 is visible iff its offset within the tile is at most
        // rel: one subtraction per lane, then compares against inline constants
        const int rel = qlim - kb - 4 * hh;
  #pragma unroll
        for (int s = 0; s < 2; ++s)
  #pragma unroll
          for (int i = 0; i < 16; ++i)
            sacc[s][i] = 32 * s + 8 * (i >> 2) + (i & 3) <= rel ? sacc[s][i] : NEG_INF;
      }
    };
    // P = exp2(S*scale - m) packed to the input dtype, with per-lane partial sums of the
    // rounded probabilities (pr). The EXACT flavour (replay rows) also returns the lane's FP32
    // sum of the unrounded ones. The two flavours are separate code under a wave-uniform
    // branch: folded into one, the compiler turns the condition into a select per element.
    // S is consumed in place.
    auto probs = [&](auto exact_tag, f32x16(&sacc)[2], u32x4(&pb)[4], float(&pr)[4]) __attribute__((always_inline)) {
      constexpr bool EXACT = decltype(exact_tag)::value;
      float ps[4];
  #pragma unroll
      for (int s = 0; s < 2; ++s) {
        float p[16];
  #pragma unroll
        for (int i = 0; i < 16; ++i) {
          p[i] = fast_exp2(fmaf(sacc[s][i], a.abs_scale_log2, nm));
          if constexpr (EXACT) ps[i & 3] = s == 0 && i < 4 ? p[i] : ps[i & 3] + p[i];
        }
  #pragma unroll
        for (int c2 = 0; c2 < 2; ++c2)
          pb[2 * s + c2] = (u32x4){E::pack2(p[8 * c2 + 0], p[8 * c2 + 1]), E::pack2(p[8 * c2 + 2], p[8 * c2 + 3]),
                                   E::pack2(p[8 * c2 + 4], p[8 * c2 + 5]), E::pack2(p[8 * c2 + 6], p[8 * c2 + 7])};
      }
  #pragma unroll
      for (int j = 0; j < 4; ++j) {
        // zero-accumulator VOP3P form on the common path (see attn_rt2_kernel)
        pr[j] = EXACT ? E::sum2(pb[0][j], ones2, 0.f) : E::sum2_0(pb[0][j], ones2);
  #pragma unroll
        for (int c = 1; c < 4; ++c) pr[j] = E::sum2(pb[c][j], ones2, pr[j]);
      }
      if constexpr (EXACT)
        return (ps[0] + ps[1]) + (ps[2] + ps[3]);
      else
        return 0.f;
    };
    auto t1_step = [&](auto exact_tag, int it, int BUF, int SLOT) __attribute__((always_inline)) {
      const int kb = it * BN;
      if (kb > wave_hi) return;

      f32x16 sacc[2];
      qk_tile(kb, BUF, SLOT, sacc);
      if (fresh) {
        // first tile of the row tile (O and the sums are still zero): exact max, no rescale
        const float mt = exact_max(sacc);
        m_run = mt;
        nm = mt == NEG_INF ? 0.f : -mt;
        fresh = false;
      }
      u32x4 pb[4];
      float pr[4];
      float le = probs(exact_tag, sacc, pb, pr);
      // overflow guard on a lane's tile sum: the FP32 sum where it exists (ready right after the
      // exponentials), else the rounded one
      const float guard = decltype(exact_tag)::value ? le : (pr[0] + pr[1]) + (pr[2] + pr[3]);
      if (__any(guard > E::kMaxTileSum)) {
        // S again (the tile is still in LDS), the new reference (the exact max plus the type's
        // headroom), O and both sums rescaled, probabilities recomputed: now all at most 1
        qk_tile(kb, BUF, SLOT, sacc);
        const float mt = exact_max(sacc);
        const float mn = vmax(m_run, mt + E::kRescaleHeadroom);
        const float corr = mn > m_run ? fast_exp2(m_run - mn) : 1.f;
        l_run *= corr;
        l_rnd *= corr;
  #pragma unroll
        for (int dt = 0; dt < NDT; ++dt) o[dt] *= corr;
        m_run = mn;
        nm = mn == NEG_INF ? 0.f : -mn;
        le = probs(exact_tag, sacc, pb, pr);
      }
      l_rnd += (pr[0] + pr[1]) + (pr[2] + pr[3]);
      if constexpr (decltype(exact_tag)::value) l_run += le;

      if constexpr (NW > 8) {
        // three waves per SIMD cover the V read latency; no prefetch (16 fewer registers)
  #pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          u32x4 vf[4];
  #pragma unroll
          for (int c4 = 0; c4 < 4; ++c4) vf[c4] = v_frag(BUF, SLOT, c4, dt);
          FE_PRIO_HI();
  #pragma unroll
          for (int c4 = 0; c4 < 4; ++c4) o[dt] = E::mfma(vf[c4], pb[c4], o[dt]);
          FE_PRIO_LO();
        }
      } else {
        // V^T fragments of channel tile dt+1 are read while the MFMAs of tile dt run
        u32x4 vf[2][4];
  #pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) vf[0][c4] = v_frag(BUF, SLOT, c4, 0);
  #pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          if (dt + 1 < NDT) {
  #pragma unroll
            for (int c4 = 0; c4 < 4; ++c4) vf[(dt + 1) & 1][c4] = v_frag(BUF, SLOT, c4, dt + 1);
          }
          FE_PRIO_HI();
  #pragma unroll
          for (int c4 = 0; c4 < 4; ++c4) o[dt] = E::mfma(vf[dt & 1][c4], pb[c4], o[dt]);
          FE_PRIO_LO();
        }
      }
    };

    if (dmaw) {
  #pragma unroll
      for (int sl = 0; sl < SLOTS; ++sl)
        if (sl < ntiles) {
          dma_k(sl * BN, lds_k0 + sl * TILE);
          dma_v(sl * BN, lds_v0 + sl * TILE);
        }
    }
    // The tile loop is instantiated twice, with and without the FP32 sum of the replay rows,
    // and each wave runs one of them: the choice is made once per wave, not per tile.
    auto t1_loop = [&](auto exact_tag) __attribute__((always_inline)) {
      if constexpr (SLOTS == 2) {
        for (int it = 0; it < ntiles; it += 4) {
          t1_sync(it, 0);
          t1_step(exact_tag, it, 0, 0);
          if (it + 1 < ntiles) t1_step(exact_tag, it + 1, 0, 1);
          if (it + 2 < ntiles) {
            t1_sync(it + 2, 1);
            t1_step(exact_tag, it + 2, 1, 0);
            if (it + 3 < ntiles) t1_step(exact_tag, it + 3, 1, 1);
          }
        }
      } else {
        for (int it = 0; it < ntiles; it += 2) {
          t1_sync(it, 0);
          t1_step(exact_tag, it, 0, 0);
          if (it + 1 < ntiles) {
            t1_sync(it + 1, 1);
            t1_step(exact_tag, it + 1, 1, 0);
          }
        }
      }
    };
    if (exact_l)
      t1_loop(std::true_type{});
    else
      t1_loop(std::false_type{});

    // ---------------- finish rows
    const float l_tot = half_swap_sum(l_run);      // replay rows only
    {
      const int qi = q0 + l32;
      if (tv && qi < N) {
        const float inv = 1.f / half_swap_sum(l_rnd);
        u16* op = a.out + ((long long)(b * a.Hq + head) * N + qi) * (PARTIAL ? a.Dq : DP);
  #pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
  #pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const int d0 = 32 * dt + 8 * g4 + 4 * hh;
            if (PARTIAL && d0 >= a.Dq) continue;   // channels past Q's head dim are not stored
            const u32 w0 = E::pack2(o[dt][4 * g4 + 0] * inv, o[dt][4 * g4 + 1] * inv);
            const u32 w1 = E::pack2(o[dt][4 * g4 + 2] * inv, o[dt][4 * g4 + 3] * inv);
            store4<PARTIAL>(op, d0, a.Dq, w0, w1);
          }
        }
      }
    }

    // ---------------- traversal 2: replay
    if (!a.score) return;
    if (a.bias) {
      // Split schedule: hand the row's replay bias (see below) to replay_fast_kernel, or to the
      // replay items of this launch (agent-scope atomic store; after every wave's stores, one
      // lane sets the item's bit)
      const int qi = q0 + l32;
      const bool items = NW <= 8 && a.nattn < a.nitems;  // the launch makes none for 12 waves
      if (hh == 0 && tv && qi < N) {
        const bool live = qi >= a.win_lo;
        const float bv = live ? (m_run + fast_log2(l_tot) - a.decay_log2 * (float)(qi - (N - 1))) : POS_INF;
        float* bp = a.bias + (long long)(b * a.Hq + head) * N + qi;
        if (items)
          __hip_atomic_store(bp, bv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
          *bp = bv;
      }
      if (items && wg_q_hi - 1 >= a.win_lo) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (wv == 0 && lane_now() == 0)
          __hip_atomic_fetch_or(a.done + (item >> 5), 1u << (item & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      return;
    }
    if constexpr (FUSED) {
      if (wg_q_hi - 1 < a.win_lo) return;

      // p_qk * w_q / l_q = exp2(s*scale - b_q) with b_q = m_q + log2 l_q - decay*log2e*(q-N+1),
      // b_q = +inf for rows outside the window or past N. nb holds -b of the 16 rows of a lane.
      float nb[16];
      {
        const int qi = q0 + l32;
        const bool live = tv && qi < N && qi >= a.win_lo;
        const float br = live ? (m_run + fast_log2(l_tot) - a.decay_log2 * (float)(qi - (N - 1))) : POS_INF;
    #pragma unroll
        for (int i = 0; i < 16; ++i) nb[i] = -__shfl(br, 8 * (i >> 2) + 4 * hh + (i & 3));
      }
      const bool rin = tv && q0 + 31 >= a.win_lo;
      const int wave_hi_r = rin ? (a.causal ? min(q0 + 31, N - 1) : N - 1) : -1;
      float* imp_row = a.imp + (long long)bh * N;

      // Flush of the previous tile's per-wave column sums (written before the barrier that
      // precedes this call): one atomic per key per workgroup.
      auto flush = [&](int kb_prev, int buf_prev) {
        if (tid < BN) {
          const float* rr = red + buf_prev * NW * BN + tid;
          float sum = 0.f;
    #pragma unroll
          for (int w = 0; w < NW; w += 2) sum += rr[w * BN] + rr[(w + 1) * BN];
          const int key = kb_prev + tid;
          if (sum != 0.f && key < N) unsafeAtomicAdd(imp_row + key, sum);
        }
      };

      // One 64-key tile: S = Q K^T (lanes hold keys), causal mask on diagonal tiles, column
      // sums of exp2(S*scale - b_q) over this wave's 32 rows, written to LDS for the flush.
      auto t2_step = [&](int it, int BUF) __attribute__((always_inline)) {
        const int kb = it * BN;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (it > 0) flush(kb - BN, BUF ^ 1);
        if (dmaw && it + 1 < ntiles) dma_k(kb + BN, BUF == 0 ? lds_k1 : lds_k0);
        float cs[2] = {0.f, 0.f};
        if (kb <= wave_hi_r) {
          f32x16 sacc[2];
    #pragma unroll
          for (int s = 0; s < 2; ++s) {
    #pragma unroll
            for (int h = 0; h < KH; ++h) {
              u32x4 kf[NDC / KH];
              k_frags(BUF, 0, s, h, kf);
              FE_PRIO_HI();
    #pragma unroll
              for (int c = 0; c < NDC / KH; ++c) {
                const int cc = h * (NDC / KH) + c;
                sacc[s] = cc == 0 ? E::mfma(qf[0], kf[c], (f32x16){}) : E::mfma(qf[cc], kf[c], sacc[s]);
              }
              FE_PRIO_LO();
            }
          }
          if (a.causal && kb + BN - 1 > q0) {
    #pragma unroll
            for (int s = 0; s < 2; ++s) {
              // key kb + 32s + l32 against row q0 + 8(i/4) + 4h + i%4
              const int rel = kb + 32 * s + l32 - q0 - 4 * hh;
    #pragma unroll
              for (int i = 0; i < 16; ++i) sacc[s][i] = rel > 8 * (i >> 2) + (i & 3) ? NEG_INF : sacc[s][i];
            }
          }
    #pragma unroll
          for (int s = 0; s < 2; ++s) {
            float c4[4];
    #pragma unroll
            for (int i = 0; i < 16; ++i) {
              const float e = fast_exp2(fmaf(sacc[s][i], a.abs_scale_log2, nb[i]));
              if (i < 4)
                c4[i] = e;
              else
                c4[i & 3] += e;
            }
            cs[s] = (c4[0] + c4[1]) + (c4[2] + c4[3]);
          }
        }
        cs[0] = half_swap_sum(cs[0]);
        cs[1] = half_swap_sum(cs[1]);
        if (hh == 0) {
          float* rb = red + BUF * NW * BN + wv * BN;
          rb[l32] = cs[0];
          rb[32 + l32] = cs[1];
        }
      };

      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();  // every wave is done reading the traversal-1 tiles
      if (dmaw) dma_k(0, lds_k0);
      for (int it = 0; it < ntiles; it += 2) {
        t2_step(it, 0);
        if (it + 1 < ntiles) t2_step(it + 1, 1);
      }
      __syncthreads();
      flush((ntiles - 1) * BN, (ntiles - 1) & 1);
    }
  };
  // One replay item (split schedule with replay items; reference flash_evict/prefill.py:61-83):
  // the window rows of one attention item's NW row tiles (one per wave) against one key range,
  // the arithmetic of replay_fast_kernel with one row tile per wave: S = Q K^T with lanes holding
  // keys, exp2(s * scale*log2e - b_q) summed over the rows of each key in-lane and over the waves
  // in LDS (the V buffers, unused here), one FP32 atomic per key and tile. It first waits for
  // the attention item of its rows (same decode) to publish their biases, or runs that item.
  auto run_replay = [&](const int ritem) __attribute__((always_inline)) {
    const int lane = lane_now(), l32 = lane & 31, hh = lane >> 5;
    int BH = a.BH, G = a.G, Hkv = a.Hkv, rsplit = a.rsplit;
    asm volatile("" : "+s"(BH), "+s"(G), "+s"(Hkv), "+s"(rsplit));
    const int bh = (int)((unsigned)ritem % (unsigned)BH);
    const int rest = (int)((unsigned)ritem / (unsigned)BH);
    const int ks = rest % rsplit;
    const int wg = a.rwg0 >= 0 ? a.rwg0 + rest / rsplit : a.wg_bh - 1 - rest / rsplit;
    const int b = bh / Hkv, hkv = bh - b * Hkv;
    const int t_begin = wg * NW;
    const int t_end = min(a.tiles_bh, t_begin + NW);
    const int kv_end = a.causal ? min(N, ((t_end - 1) / G + 1) * 32) : N;
    const int ntiles_all = (kv_end + BN - 1) / BN;
    const int per = (ntiles_all + rsplit - 1) / rsplit;
    const int it_lo = ks * per, it_hi = min(ntiles_all, it_lo + per);
    const int dep = (a.wg_bh - 1 - wg) * BH + bh;
    if (wv == 0) {
      const bool ok = wait_item_done(a, dep, ntiles_all);
      if (lane_now() == 0) s_ready = ok ? 1 : 0;
    }
    __syncthreads();
    if (!__builtin_amdgcn_readfirstlane(s_ready)) {
      run_item(dep);
      __syncthreads();
    }
    if (it_lo >= it_hi) return;

    // this wave's row tile; nb: minus the biases of the 16 rows a lane holds (register i:
    // row 8(i/4) + 4h + i%4)
    const int t = t_begin + wv;
    const bool tv = t < t_end;
    const int tt = tv ? t : t_begin;
    const int q0 = (tt / G) * 32;
    const int head = hkv * G + (tt - (tt / G) * G);
    const bool rin = tv && q0 + 31 >= a.win_lo;
    const int wave_hi_r = rin ? (a.causal ? min(q0 + 31, N - 1) : N - 1) : -1;
    const u32 qneg = a.neg_scale ? 0x80008000u : 0u;
    u32x4 qf[NDC];
    float nb[16];
    {
      const int qr = q0 + l32;
      const bool ok = rin && qr < N;
      const u16* qp = a.q + b * a.qs[0] + head * a.qs[1] + (long long)(ok ? qr : 0) * a.qs[2];
  #pragma unroll
      for (int c = 0; c < NDC; ++c)
        qf[c] = ok ? ((load8(qp, a.qs[3], 16 * c + 8 * hh, PARTIAL ? a.Dq : DP, a.qvec) & a.qmask) ^ qneg)
                   : (u32x4){0u, 0u, 0u, 0u};
      const float br = ok ? __hip_atomic_load(a.bias + (long long)(b * a.Hq + head) * N + qr, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT)
                          : POS_INF;
  #pragma unroll
      for (int i = 0; i < 16; ++i) nb[i] = -__shfl(br, 8 * (i >> 2) + 4 * hh + (i & 3));
    }
    const u32 koff = (u32)(l32 * 32 + ((hh ^ ((l32 >> 3) & 1)) << 4));
    const u32 krow = (u32)(a.ks[2] * 2);
    const unsigned char* kg = (const unsigned char*)(a.k + b * a.ks[0] + hkv * a.ks[1]);
    float* imp_row = a.imp + (long long)bh * N;
    float* red_r = (float*)lds_v0;                 // [2][NW][BN] per-wave column sums
    auto r_dma = [&](int kb, unsigned char* ldst) {
      const int ln = lane_now();
      const u32 sw = (u32)((ln & 1) ^ ((ln >> 4) & 1));
      dma_tile_cm<DPW, 32, PARTIAL>(kg, krow, (u32)(ln >> 1) * krow + (sw << 4), kb, N, ldst, wv, a.D, sw << 3);
    };
    auto r_flush = [&](int kb_prev, int buf_prev) {
      if (wv == 0) {
        const int ln = lane_now();
        const float* rr = red_r + buf_prev * NW * BN + ln;
        float sum = 0.f;
  #pragma unroll
        for (int w = 0; w < NW; w += 2) sum += rr[w * BN] + rr[(w + 1) * BN];
        const int key = kb_prev + ln;
        if (sum != 0.f && key < N) unsafeAtomicAdd(imp_row + key, sum);
      }
    };
    auto r_step = [&](int it, int BUF) __attribute__((always_inline)) {
      const int kb = it * BN;
      if (dmaw) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (it > it_lo) r_flush(kb - BN, BUF ^ 1);
      if (dmaw && it + 1 < it_hi) r_dma(kb + BN, BUF == 0 ? lds_k1 : lds_k0);
      float cs[2] = {0.f, 0.f};
      if (kb <= wave_hi_r) {
        const unsigned char* kt = BUF == 0 ? lds_k0 : lds_k1;
  #pragma unroll
        for (int s = 0; s < 2; ++s) {
          f32x16 sacc = (f32x16){};
  #pragma unroll
          for (int c = 0; c < NDC; ++c) {
            const u32x4 kf = *(const u32x4*)(kt + c * 2048 + s * 1024 + koff);
            sacc = E::mfma(qf[c], kf, sacc);
          }
          // lanes hold key kb + 32s + l32; causal mask on diagonal halves
          if (a.causal && kb + 32 * s + 31 > q0) {
            const int rel = kb + 32 * s + l32 - q0 - 4 * hh;
  #pragma unroll
            for (int i = 0; i < 16; ++i) sacc[i] = rel > 8 * (i >> 2) + (i & 3) ? NEG_INF : sacc[i];
          }
          float c4[4];
  #pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float e = fast_exp2(fmaf(sacc[i], a.abs_scale_log2, nb[i]));
            if (i < 4)
              c4[i] = e;
            else
              c4[i & 3] += e;
          }
          cs[s] = (c4[0] + c4[1]) + (c4[2] + c4[3]);
        }
      }
      cs[0] = half_swap_sum(cs[0]);
      cs[1] = half_swap_sum(cs[1]);
      if (hh == 0) {
        float* rb = red_r + BUF * NW * BN + wv * BN;
        rb[l32] = cs[0];
        rb[32 + l32] = cs[1];
      }
    };
    if (dmaw) r_dma(it_lo * BN, lds_k0);
    for (int it = it_lo; it < it_hi; it += 2) {
      r_step(it, 0);
      if (it + 1 < it_hi) r_step(it + 1, 1);
    }
    __syncthreads();
    r_flush((it_hi - 1) * BN, (it_hi - 1 - it_lo) & 1);
  };

  if constexpr (FUSED) {
    // the kernel with the replay traversal (no workspace, so no queue) runs one item
    run_item((int)blockIdx.x);
  } else {
    const int item_end = a.queue ? a.nitems : (int)blockIdx.x + 1;
    for (int item = (int)blockIdx.x; item < item_end; item = a.queue ? next_item(a, &s_item, wv) : item_end) {
      if constexpr (NW <= 8) {
        if (item < a.nattn)
          run_item(item);
        else
          run_replay(item - a.nattn);
      } else {
        run_item(item);                            // no replay items (the launch does not make any)
      }
    }
  }
}



// Traversal 1 (reference flash_evict/prefill.py:37-60) with two row tiles per wave (attention
// only: the split schedule, or no importance), tile dims 96 and 128. Eight waves, two per SIMD, each holding the Q fragments
// and O accumulators of two row tiles, so every K and V^T fragment read from LDS feeds two
// MFMAs: half the LDS read traffic per MFMA of fused_fast_kernel, whose fragment reads cost
// more than its exponentials. A 64-key tile runs as two 32-key halves (QK^T, mask,
// probabilities, P@V of keys 32s .. 32s+31), which keeps S and P of both row tiles within
// the 256 registers of a wave at two waves per SIMD.
//
// Same mathematics as fused_fast_kernel. The reference max of a row is the exact max of its
// first 32 keys (instead of 64); the overflow guard, the rescale and the normalisation by the
// sum of the rounded probabilities are per row tile and per half. Each row tile also hands
// its replay bias to replay_fast_kernel, as fused_fast_kernel does.
//
// K fragments are read FE_RT2_KG at a time: two (250 registers, nothing spilled) and four
// (one value spilled outside the tile loop) measured the same.
#ifndef FE_RT2_KG
#define FE_RT2_KG 2
#endif
template <typename E, int DP, bool PARTIAL>
__global__ __launch_bounds__(512, 2) void attn_rt2_kernel(const AttnArgs a) {
  typedef FastTile<DP> T;
  constexpr int BN = T::BN, NDC = T::NDC, NDT = T::NDT, TILE = T::TILE;
  constexpr int DPW = T::DMA_PER_WAVE;
  constexpr int NW = 8, RT = 2;                  // waves per workgroup, row tiles per wave
  constexpr int SLOTS = 2;                       // 64-key tiles per LDS buffer
  constexpr int KG = NDC >= FE_RT2_KG ? FE_RT2_KG : NDC;   // K fragments per read group
  static_assert(DP >= 96 && DP <= 128 && NDC % KG == 0, "tile dims 96 and 128");
  constexpr float NEG_INF = -__builtin_huge_valf();
  constexpr float POS_INF = __builtin_huge_valf();

  __shared__ __attribute__((aligned(1024))) unsigned char lds_k0[SLOTS * TILE], lds_k1[SLOTS * TILE],
      lds_v0[SLOTS * TILE], lds_v1[SLOTS * TILE];
  // replay items: per-wave column sums of two buffers of two 64-key tiles, [buffer][slot][wave][key]
  __shared__ float red[2 * SLOTS * NW * BN];

  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool dmaw = wv < 4;                      // waves 0-3 issue the tile DMA
  const int N = a.N;

  __shared__ int s_item, s_ready;
  int item = (int)blockIdx.x;
  const int item_end = a.queue ? a.nitems : item + 1;
  // One attention item (traversal 1 of its 16 row tiles, the output, the replay biases).
  auto run_attention = [&](const int item) __attribute__((always_inline)) {
    const int lane = lane_now(), l32 = lane & 31, hh = lane >> 5;
    // The divisors of the item decode, taken opaquely: otherwise the compiler keeps their
    // reciprocals, computed once before the item loop, in registers across it.
    int BH = a.BH, G = a.G, Hkv = a.Hkv;
    asm volatile("" : "+s"(BH), "+s"(G), "+s"(Hkv));
    const int bh = (int)((unsigned)item % (unsigned)BH);
    const int wg = a.wg_bh - 1 - (int)((unsigned)item / (unsigned)BH);
    const int b = bh / Hkv, hkv = bh - b * Hkv;
    const int t_begin = wg * (NW * RT);
    const int t_end = min(a.tiles_bh, t_begin + NW * RT);
    const int wg_q_hi = min(N, ((t_end - 1) / G + 1) * 32);
    const int kv_end = a.causal ? wg_q_hi : N;
    const int ntiles = (kv_end + BN - 1) / BN;

    // This wave's row tiles j = 0, 1: 32 query positions from q0[j] of query head head[j].
    // lo_lim: below it no key of either tile is masked; wave_hi: past it every key of both tiles
    // is.
    int q0[RT], head[RT];
    bool tv[RT];
    int lo_lim = N, wave_hi = -1;
    bool in_win = false;
  #pragma unroll
    for (int j = 0; j < RT; ++j) {
      const int t = t_begin + RT * wv + j;
      tv[j] = t < t_end;
      const int tt = tv[j] ? t : t_begin;
      q0[j] = (tt / G) * 32;
      head[j] = hkv * G + (tt - (tt / G) * G);
      lo_lim = min(lo_lim, !tv[j] ? -1 : (a.causal ? min(q0[j], N - 1) : N - 1));
      wave_hi = max(wave_hi, !tv[j] ? -1 : (a.causal ? min(q0[j] + 31, N - 1) : N - 1));
      in_win = in_win || (tv[j] && q0[j] + 31 >= a.win_lo);
    }

    const u32 qneg = a.neg_scale ? 0x80008000u : 0u;   // a negative scale runs as |scale| on -Q
    u32x4 qf[RT][NDC];
  #pragma unroll
    for (int j = 0; j < RT; ++j) {
      const int qr = q0[j] + l32;
      const bool ok = tv[j] && qr < N;
      const u16* qp = a.q + b * a.qs[0] + head[j] * a.qs[1] + (long long)(ok ? qr : 0) * a.qs[2];
  #pragma unroll
      for (int c = 0; c < NDC; ++c)
        qf[j][c] = ok ? ((load8(qp, a.qs[3], 16 * c + 8 * hh, PARTIAL ? a.Dq : DP, a.qvec) & a.qmask) ^ qneg) : (u32x4){0u, 0u, 0u, 0u};
    }

    // LDS operand offsets and tile DMA: the layout of fused_fast_kernel
    const u32 koff = (u32)(l32 * 32 + ((hh ^ ((l32 >> 3) & 1)) << 4));
    u32 voff;
    {
      const int r = lane & 15, g = lane >> 4;
      voff = (u32)((4 * hh + (r >> 2)) * 64 + 32 * (g & 1) + 8 * (r & 3));
    }
    const u32 krow = (u32)(a.ks[2] * 2), vrow = (u32)(a.vs[2] * 2);
    const unsigned char* kg = (const unsigned char*)(a.k + b * a.ks[0] + hkv * a.ks[1]);
    const unsigned char* vg = (const unsigned char*)(a.v + b * a.vs[0] + hkv * a.vs[1]);
    // per-lane DMA offsets (see fused_fast_kernel), recomputed at each DMA: held across the
    // tile loop they would take registers the two row tiles need
    auto dma_k = [&](int kb, unsigned char* ldst) {
      const int ln = lane_now();
      const u32 sw = (u32)((ln & 1) ^ ((ln >> 4) & 1));
      dma_tile_cm<DPW, 32, PARTIAL>(kg, krow, (u32)(ln >> 1) * krow + (sw << 4), kb, N, ldst, wv, a.D, sw << 3);
    };
    auto dma_v = [&](int kb, unsigned char* ldst) {
      const int ln = lane_now();
      dma_tile_cm<DPW, 64, PARTIAL>(vg, vrow, (u32)(ln >> 2) * vrow + (u32)((ln & 3) << 4), kb, N, ldst, wv, a.D,
                                    (u32)((ln & 3) << 3));
    };

    // K fragments c0 .. c0+KG-1 of keys 32s + l32 (buffer BUF, slot SLOT)
    auto k_frags = [&](int BUF, int SLOT, int s, int c0, u32x4(&kf)[KG]) __attribute__((always_inline)) {
      const unsigned char* kt = (BUF == 0 ? lds_k0 : lds_k1) + SLOT * TILE + s * 1024 + koff;
  #pragma unroll
      for (int c = 0; c < KG; ++c) kf[c] = *(const u32x4*)(kt + (c0 + c) * 2048);
    };
    auto v_frag = [&](int BUF, int SLOT, int c4, int dt) __attribute__((always_inline)) -> u32x4 {
      const unsigned char* vt = (BUF == 0 ? lds_v0 : lds_v1) + SLOT * TILE + dt * 4096 + c4 * 1024 + voff;
      const s16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds_ptr_t)vt);
      const s16x4 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds_ptr_t)(vt + 512));
      const u32x2 ux = __builtin_bit_cast(u32x2, x), uy = __builtin_bit_cast(u32x2, y);
      return (u32x4){ux[0], ux[1], uy[0], uy[1]};
    };

    f32x16 o[RT][NDT];
    // nm: minus the row's reference max (log2 units); 0 while a padding tile has seen no key
    float l_run[RT], l_rnd[RT], nm[RT];
  #pragma unroll
    for (int j = 0; j < RT; ++j) {
      l_run[j] = 0.f;
      l_rnd[j] = 0.f;
      nm[j] = 0.f;
  #pragma unroll
      for (int dt = 0; dt < NDT; ++dt) o[j][dt] = (f32x16){};
    }
    bool fresh = true;                             // no key of this wave's tiles seen yet
    // Only rows the replay visits need the FP32 sum (their replay bias); wave-uniform.
    const bool exact_l = a.score && in_win;
    u32 ones2;
    asm volatile("s_mov_b32 %0, %1" : "=s"(ones2) : "i"(E::kOnes2));

    auto t1_sync = [&](int it, int BUF) __attribute__((always_inline)) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (dmaw) {
  #pragma unroll
        for (int sl = 0; sl < SLOTS; ++sl)
          if (it + SLOTS + sl < ntiles) {
            dma_k((it + SLOTS + sl) * BN, (BUF == 0 ? lds_k1 : lds_k0) + sl * TILE);
            dma_v((it + SLOTS + sl) * BN, (BUF == 0 ? lds_v1 : lds_v0) + sl * TILE);
          }
      }
    };
    // Key kh + 8(i/4) + 4h + i%4 (accumulator register i) is visible to the lane's query row of
    // tile j iff 8(i/4) + i%4 <= mask_rel(j, kh): the row's last visible key (-1 for a padding
    // tile) minus kh + 4h. Lane-derived, so recomputed here (diagonal and ragged halves only).
    auto mask_rel = [&](int j, int kh) __attribute__((always_inline)) -> int {
      const int ln = lane_now();
      const int ql = !tv[j] ? -1 : (a.causal ? min(q0[j] + (ln & 31), N - 1) : N - 1);
      return ql - kh - 4 * (ln >> 5);
    };
    // S^T of keys kh .. kh+31 for both row tiles (lanes hold queries; register i holds key
    // kh + 8(i/4) + 4h + i%4), masked on diagonal and ragged halves
    auto qk_half = [&](int kh, int BUF, int SLOT, int s, f32x16(&S)[RT]) __attribute__((always_inline)) {
  #pragma unroll
      for (int g = 0; g < NDC / KG; ++g) {
        u32x4 kf[KG];
        k_frags(BUF, SLOT, s, g * KG, kf);
        FE_PRIO_HI();
  #pragma unroll
        for (int c = 0; c < KG; ++c)
  #pragma unroll
          for (int j = 0; j < RT; ++j)
            S[j] = (g == 0 && c == 0) ? E::mfma(kf[0], qf[j][0], (f32x16){}) : E::mfma(kf[c], qf[j][g * KG + c], S[j]);
        FE_PRIO_LO();
      }
      if (kh + 31 > lo_lim) {
  #pragma unroll
        for (int j = 0; j < RT; ++j) {
          const int rel = mask_rel(j, kh);
  #pragma unroll
          for (int i = 0; i < 16; ++i) S[j][i] = 8 * (i >> 2) + (i & 3) <= rel ? S[j][i] : NEG_INF;
        }
      }
    };
    // the same for row tile J alone (the rare overflow recompute)
    auto qk_one = [&](auto jtag, int kh, int BUF, int SLOT, int s, f32x16& S) __attribute__((always_inline)) {
      constexpr int J = decltype(jtag)::value;
  #pragma unroll
      for (int g = 0; g < NDC / KG; ++g) {
        u32x4 kf[KG];
        k_frags(BUF, SLOT, s, g * KG, kf);
  #pragma unroll
        for (int c = 0; c < KG; ++c) S = (g == 0 && c == 0) ? E::mfma(kf[0], qf[J][0], (f32x16){}) : E::mfma(kf[c], qf[J][g * KG + c], S);
      }
      if (kh + 31 > lo_lim) {
        const int rel = mask_rel(J, kh);
  #pragma unroll
        for (int i = 0; i < 16; ++i) S[i] = 8 * (i >> 2) + (i & 3) <= rel ? S[i] : NEG_INF;
      }
    };
    // exact max (log2 units) of a row over the 32 keys of S: this lane's 16 and the other half-wave's
    auto exact_max = [&](const f32x16& S) __attribute__((always_inline)) -> float {
      float mc = vmax(vmax(S[0], S[1]), S[2]);
  #pragma unroll
      for (int i = 3; i < 15; i += 2) mc = vmax(vmax(mc, S[i]), S[i + 1]);
      return half_swap_maximum(vmax(mc, S[15])) * a.abs_scale_log2;
    };
    // P = exp2(S*scale - m) packed to the input dtype (pb[0]: keys 0-15 of the half, pb[1]:
    // 16-31), partial sums of the rounded probabilities (pr); EXACT also returns the lane's
    // FP32 sum of the unrounded ones
    // S is consumed in place (it holds the probabilities afterwards).
    auto probs = [&](auto exact_tag, f32x16& S, float nmj, u32x4(&pb)[2], float(&pr)[4]) __attribute__((always_inline)) {
      constexpr bool EXACT = decltype(exact_tag)::value;
      float ps[4];
  #pragma unroll
      for (int i = 0; i < 16; ++i) {
        S[i] = fast_exp2(fmaf(S[i], a.abs_scale_log2, nmj));
        if constexpr (EXACT) ps[i & 3] = i < 4 ? S[i] : ps[i & 3] + S[i];
      }
  #pragma unroll
      for (int c2 = 0; c2 < 2; ++c2)
        pb[c2] = (u32x4){E::pack2(S[8 * c2 + 0], S[8 * c2 + 1]), E::pack2(S[8 * c2 + 2], S[8 * c2 + 3]),
                         E::pack2(S[8 * c2 + 4], S[8 * c2 + 5]), E::pack2(S[8 * c2 + 6], S[8 * c2 + 7])};
  #pragma unroll
      for (int e = 0; e < 4; ++e) {
        // the zero-accumulator VOP3P form saves a v_mov per chain; measured 1-2% faster on the
        // common path, 1.5% slower in the replay-row variant (the compiler schedules it worse)
        const float first = EXACT ? E::sum2(pb[0][e], ones2, 0.f) : E::sum2_0(pb[0][e], ones2);
        pr[e] = E::sum2(pb[1][e], ones2, first);
      }
      if constexpr (EXACT)
        return (ps[0] + ps[1]) + (ps[2] + ps[3]);
      else
        return 0.f;
    };
    // overflow path of row tile J: S again, the new reference (the exact max plus the type's
    // headroom), O and both sums rescaled, probabilities recomputed (now at most 1)
    auto rescale_one = [&](auto exact_tag, auto jtag, int kh, int BUF, int SLOT, int s, u32x4(&pb)[2], float(&pr)[4])
                           __attribute__((always_inline)) -> float {
      constexpr int J = decltype(jtag)::value;
      f32x16 S;
      qk_one(jtag, kh, BUF, SLOT, s, S);
      // a row that overflows has a finite reference max (its tile is a real one)
      const float m_old = -nm[J];
      const float mn = vmax(m_old, exact_max(S) + E::kRescaleHeadroom);
      const float corr = mn > m_old ? fast_exp2(m_old - mn) : 1.f;
      l_run[J] *= corr;
      l_rnd[J] *= corr;
  #pragma unroll
      for (int dt = 0; dt < NDT; ++dt) o[J][dt] *= corr;
      nm[J] = -mn;
      return probs(exact_tag, S, nm[J], pb, pr);
    };
    // keys 32s .. 32s+31 of tile it (buffer BUF, slot SLOT)
    auto t1_half = [&](auto exact_tag, int it, int BUF, int SLOT, int s) __attribute__((always_inline)) {
      constexpr bool EXACT = decltype(exact_tag)::value;
      const int kh = it * BN + 32 * s;
      if (kh > wave_hi) return;

      f32x16 S[RT];
      qk_half(kh, BUF, SLOT, s, S);
      if (fresh) {
        // first keys of the row tiles (O and the sums are still zero): exact max, no rescale
  #pragma unroll
        for (int j = 0; j < RT; ++j) {
          const float mt = exact_max(S[j]);
          nm[j] = mt == NEG_INF ? 0.f : -mt;
        }
        fresh = false;
      }
      u32x4 pb[RT][2];
      float pr[RT][4], le[RT];
  #pragma unroll
      for (int j = 0; j < RT; ++j) le[j] = probs(exact_tag, S[j], nm[j], pb[j], pr[j]);
      {
        const float g0 = EXACT ? le[0] : (pr[0][0] + pr[0][1]) + (pr[0][2] + pr[0][3]);
        if (__any(g0 > E::kMaxTileSum)) le[0] = rescale_one(exact_tag, std::integral_constant<int, 0>{}, kh, BUF, SLOT, s, pb[0], pr[0]);
        const float g1 = EXACT ? le[1] : (pr[1][0] + pr[1][1]) + (pr[1][2] + pr[1][3]);
        if (__any(g1 > E::kMaxTileSum)) le[1] = rescale_one(exact_tag, std::integral_constant<int, 1>{}, kh, BUF, SLOT, s, pb[1], pr[1]);
      }
  #pragma unroll
      for (int j = 0; j < RT; ++j) {
        l_rnd[j] += (pr[j][0] + pr[j][1]) + (pr[j][2] + pr[j][3]);
        if constexpr (EXACT) l_run[j] += le[j];
      }
      // O^T += V^T P^T over the half's two 16-key groups; each V^T fragment feeds both row tiles
  #pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        u32x4 vf[2];
  #pragma unroll
        for (int c = 0; c < 2; ++c) vf[c] = v_frag(BUF, SLOT, 2 * s + c, dt);
        FE_PRIO_HI();
  #pragma unroll
        for (int c = 0; c < 2; ++c)
  #pragma unroll
          for (int j = 0; j < RT; ++j) o[j][dt] = E::mfma(vf[c], pb[j][c], o[j][dt]);
        FE_PRIO_LO();
      }
    };
    auto t1_step = [&](auto exact_tag, int it, int BUF, int SLOT) __attribute__((always_inline)) {
      t1_half(exact_tag, it, BUF, SLOT, 0);
      t1_half(exact_tag, it, BUF, SLOT, 1);
    };

    if (dmaw) {
  #pragma unroll
      for (int sl = 0; sl < SLOTS; ++sl)
        if (sl < ntiles) {
          dma_k(sl * BN, lds_k0 + sl * TILE);
          dma_v(sl * BN, lds_v0 + sl * TILE);
        }
    }
    auto t1_loop = [&](auto exact_tag) __attribute__((always_inline)) {
      for (int it = 0; it < ntiles; it += 4) {
        t1_sync(it, 0);
        t1_step(exact_tag, it, 0, 0);
        if (it + 1 < ntiles) t1_step(exact_tag, it + 1, 0, 1);
        if (it + 2 < ntiles) {
          t1_sync(it + 2, 1);
          t1_step(exact_tag, it + 2, 1, 0);
          if (it + 3 < ntiles) t1_step(exact_tag, it + 3, 1, 1);
        }
      }
    };
    if (exact_l)
      t1_loop(std::true_type{});
    else
      t1_loop(std::false_type{});

    // ---------------- finish rows: O / l_rnd, and the replay bias
  #pragma unroll
    for (int j = 0; j < RT; ++j) {
      const float l_tot = half_swap_sum(l_run[j]);
      const float inv = 1.f / half_swap_sum(l_rnd[j]);
      const int qi = q0[j] + l32;
      if (tv[j] && qi < N) {
        u16* op = a.out + ((long long)(b * a.Hq + head[j]) * N + qi) * (PARTIAL ? a.Dq : DP);
  #pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
  #pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const int d0 = 32 * dt + 8 * g4 + 4 * hh;
            if (PARTIAL && d0 >= a.Dq) continue;
            const u32 w0 = E::pack2(o[j][dt][4 * g4 + 0] * inv, o[j][dt][4 * g4 + 1] * inv);
            const u32 w1 = E::pack2(o[j][dt][4 * g4 + 2] * inv, o[j][dt][4 * g4 + 3] * inv);
            store4<PARTIAL>(op, d0, a.Dq, w0, w1);
          }
        }
        if (a.score && a.bias && hh == 0) {
          const bool live = qi >= a.win_lo;
          // agent-scope atomic store: replay items of this launch on other XCDs read it
          __hip_atomic_store(a.bias + (long long)(b * a.Hq + head[j]) * N + qi,
                             live ? (fast_log2(l_tot) - nm[j] - a.decay_log2 * (float)(qi - (N - 1))) : POS_INF,
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
    // replay items of this launch wait for the item's biases: every wave's stores complete,
    // then one lane sets the item's bit
    if (a.nattn < a.nitems && a.score && wg_q_hi - 1 >= a.win_lo) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (wv == 0 && lane_now() == 0)
        __hip_atomic_fetch_or(a.done + (item >> 5), 1u << (item & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };

  for (; item < item_end; item = a.queue ? next_item(a, &s_item, wv) : item_end) {
    if (item < a.nattn) {
      run_attention(item);
      continue;
    }
      // ---------------- replay item (reference flash_evict/prefill.py:61-83), short observation
      // windows: the window rows of one attention item's 16 row tiles against one key range.
      // S = Q K^T with lanes holding keys, exp2(s * scale*log2e - b_q) summed over the rows of
      // each key in-lane and over the waves in LDS, one FP32 atomic per key and tile: the
      // arithmetic of replay_fast_kernel, here in the attention kernel's workgroups, so the
      // replay fills the end of the attention launch instead of following it.
      const int ritem = item - a.nattn;
      const int lane = lane_now(), l32 = lane & 31, hh = lane >> 5;
      int BH = a.BH, G = a.G, Hkv = a.Hkv, rsplit = a.rsplit;
      asm volatile("" : "+s"(BH), "+s"(G), "+s"(Hkv), "+s"(rsplit));
      const int bh = (int)((unsigned)ritem % (unsigned)BH);
      const int rest = (int)((unsigned)ritem / (unsigned)BH);
      const int ks = rest % rsplit;
      const int wg = a.rwg0 >= 0 ? a.rwg0 + rest / rsplit : a.wg_bh - 1 - rest / rsplit;
      const int b = bh / Hkv, hkv = bh - b * Hkv;
      const int t_begin = wg * (NW * RT);
      const int t_end = min(a.tiles_bh, t_begin + NW * RT);
      const int kv_end = a.causal ? min(N, ((t_end - 1) / G + 1) * 32) : N;
      const int ntiles_all = (kv_end + BN - 1) / BN;
      const int per = (ntiles_all + rsplit - 1) / rsplit;
      const int it_lo = ks * per, it_hi = min(ntiles_all, it_lo + per);
      // the attention item of these rows (same decode) publishes their biases; if it has not
      // within the bound, this workgroup runs it
      const int dep = (a.wg_bh - 1 - wg) * BH + bh;
      if (wv == 0) {
        const bool ok = wait_item_done(a, dep, ntiles_all);
        if (lane_now() == 0) s_ready = ok ? 1 : 0;
      }
      __syncthreads();
      if (!__builtin_amdgcn_readfirstlane(s_ready)) {
        run_attention(dep);
        __syncthreads();
      }
      if (it_lo >= it_hi) continue;

      int q0[RT];
      bool tv[RT];
      u32x4 qf[RT][NDC];
      float nb[RT][16];
      int rwave_hi = -1;                       // last key this wave's window rows see
      const u32 qneg = a.neg_scale ? 0x80008000u : 0u;
  #pragma unroll
      for (int j = 0; j < RT; ++j) {
        const int t = t_begin + RT * wv + j;
        tv[j] = t < t_end;
        const int tt = tv[j] ? t : t_begin;
        q0[j] = (tt / G) * 32;
        const int head = hkv * G + (tt - (tt / G) * G);
        const bool rin = tv[j] && q0[j] + 31 >= a.win_lo;
        if (rin) rwave_hi = max(rwave_hi, a.causal ? min(q0[j] + 31, N - 1) : N - 1);
        const int qr = q0[j] + l32;
        const bool ok = rin && qr < N;
        const u16* qp = a.q + b * a.qs[0] + head * a.qs[1] + (long long)(ok ? qr : 0) * a.qs[2];
  #pragma unroll
        for (int c = 0; c < NDC; ++c)
          qf[j][c] = ok ? ((load8(qp, a.qs[3], 16 * c + 8 * hh, PARTIAL ? a.Dq : DP, a.qvec) & a.qmask) ^ qneg)
                        : (u32x4){0u, 0u, 0u, 0u};
        const float br = ok ? __hip_atomic_load(a.bias + (long long)(b * a.Hq + head) * N + qr, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT)
                            : POS_INF;
        // minus the biases of the 16 rows a lane holds (register i: row 8(i/4) + 4h + i%4)
  #pragma unroll
        for (int i = 0; i < 16; ++i) nb[j][i] = -__shfl(br, 8 * (i >> 2) + 4 * hh + (i & 3));
      }
      const u32 koff = (u32)(l32 * 32 + ((hh ^ ((l32 >> 3) & 1)) << 4));
      const u32 krow = (u32)(a.ks[2] * 2);
      const unsigned char* kg = (const unsigned char*)(a.k + b * a.ks[0] + hkv * a.ks[1]);
      float* imp_row = a.imp + (long long)bh * N;
      auto r_dma = [&](int kb, unsigned char* ldst) {
        const int ln = lane_now();
        const u32 sw = (u32)((ln & 1) ^ ((ln >> 4) & 1));
        dma_tile_cm<DPW, 32, PARTIAL>(kg, krow, (u32)(ln >> 1) * krow + (sw << 4), kb, N, ldst, wv, a.D, sw << 3);
      };
      // wave SLOT adds up slot SLOT of the pair from it0 in buffer BUF over the waves
      auto r_flush = [&](int it0, int BUF) __attribute__((always_inline)) {
        if (wv < SLOTS && it0 + wv < it_hi) {
          const int ln = lane_now();
          const float* rr = red + ((BUF * SLOTS + wv) * NW) * BN + ln;
          float sum = 0.f;
  #pragma unroll
          for (int w = 0; w < NW; w += 2) sum += rr[w * BN] + rr[(w + 1) * BN];
          const int key = (it0 + wv) * BN + ln;
          if (sum != 0.f && key < N) unsafeAtomicAdd(imp_row + key, sum);
        }
      };
      auto r_sync = [&](int it, int BUF) __attribute__((always_inline)) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (it > it_lo) r_flush(it - SLOTS, BUF ^ 1);
        if (dmaw) {
  #pragma unroll
          for (int sl = 0; sl < SLOTS; ++sl)
            if (it + SLOTS + sl < it_hi) r_dma((it + SLOTS + sl) * BN, (BUF == 0 ? lds_k1 : lds_k0) + sl * TILE);
        }
      };
      auto r_tile = [&](int it, int BUF, int SLOT) __attribute__((always_inline)) {
        const int kb = it * BN;
        float cs[2] = {0.f, 0.f};
        const unsigned char* kt = (BUF == 0 ? lds_k0 : lds_k1) + SLOT * TILE;
  #pragma unroll
        for (int s = 0; s < 2; ++s) {
          if (kb + 32 * s > rwave_hi) continue;
          f32x16 sacc[RT];
  #pragma unroll
          for (int j = 0; j < RT; ++j) sacc[j] = (f32x16){};
  #pragma unroll
          for (int c = 0; c < NDC; ++c) {
            const u32x4 kf = *(const u32x4*)(kt + c * 2048 + s * 1024 + koff);
  #pragma unroll
            for (int j = 0; j < RT; ++j) sacc[j] = E::mfma(qf[j][c], kf, sacc[j]);
          }
          float c4[4];
  #pragma unroll
          for (int j = 0; j < RT; ++j) {
            // lanes hold key kb + 32s + l32; causal mask on diagonal halves
            if (a.causal && kb + 32 * s + 31 > q0[j]) {
              const int ln = lane_now();
              const int rel = (ln & 31) - 4 * (ln >> 5) + (kb + 32 * s - q0[j]);
  #pragma unroll
              for (int i = 0; i < 16; ++i) sacc[j][i] = rel > 8 * (i >> 2) + (i & 3) ? NEG_INF : sacc[j][i];
            }
  #pragma unroll
            for (int i = 0; i < 16; ++i) {
              const float e = fast_exp2(fmaf(sacc[j][i], a.abs_scale_log2, nb[j][i]));
              if (j == 0 && i < 4)
                c4[i] = e;
              else
                c4[i & 3] += e;
            }
          }
          cs[s] = (c4[0] + c4[1]) + (c4[2] + c4[3]);
        }
        cs[0] = half_swap_sum(cs[0]);
        cs[1] = half_swap_sum(cs[1]);
        if (hh == 0) {
          float* rb = red + ((BUF * SLOTS + SLOT) * NW + wv) * BN;
          rb[l32] = cs[0];
          rb[32 + l32] = cs[1];
        }
      };
      if (dmaw) {
  #pragma unroll
        for (int sl = 0; sl < SLOTS; ++sl)
          if (it_lo + sl < it_hi) r_dma((it_lo + sl) * BN, lds_k0 + sl * TILE);
      }
      for (int it = it_lo; it < it_hi; it += 2 * SLOTS) {
        r_sync(it, 0);
        r_tile(it, 0, 0);
        if (it + 1 < it_hi) r_tile(it + 1, 0, 1);
        if (it + SLOTS < it_hi) {
          r_sync(it + SLOTS, 1);
          r_tile(it + SLOTS, 1, 0);
          if (it + SLOTS + 1 < it_hi) r_tile(it + SLOTS + 1, 1, 1);
        }
      }
      __syncthreads();
      const int last = it_lo + ((it_hi - 1 - it_lo) / SLOTS) * SLOTS;
      r_flush(last, ((last - it_lo) / SLOTS) & 1);
      continue;
  }
}

// Replay traversal of the split schedule. After fused_fast_kernel has written the bias
//   b_q = m_q + log2 l_q - decay*log2e*(q - N + 1)   (+inf outside the window or past N)
// of every query row, the importance is
//   I[b, j, k] += sum over the group's heads and rows q of exp2(s_qk * scale*log2e - b_q)
// (the value L1 norm is applied afterwards, as in the fused schedule). Without O, P and V
// this traversal needs far fewer registers than traversal 1. A workgroup holds 8 row tiles
// that share every K tile (one FP32 atomic per key and tile per workgroup), as 8/TPW waves
// of TPW row tiles each. TPW = 1 runs at four waves per SIMD. TPW = 2 (the default) runs at
// three (three workgroups per CU; 168 registers, none spilled, 1.5% faster than at two),
// with every K fragment read from LDS feeding two MFMAs: that halves the LDS read
// traffic, the co-bottleneck of this traversal next to the MFMAs, and measures about 3%
// faster than TPW = 1. The K tiles use the attention kernel's channel-group-major layout.

// Waves and row tiles of a replay workgroup: 8 row tiles as 8/TPW waves for TPW = 1 or 2;
// TPW = 3 runs 4 waves of three row tiles (12 per workgroup, two waves per SIMD). Above tile
// dim 128 (one row tile per wave) the Q fragments alone take up to 64 registers: two waves per
// SIMD.
template <int TPW, int DP>
struct ReplayShape {
  static constexpr int NW = TPW == 3 ? 4 : 8 / TPW;
  static constexpr int RT = NW * TPW;
  static constexpr int WAVES_PER_EU = TPW == 1 ? (DP > 128 ? 2 : 4) : (TPW == 2 ? 3 : 2);
};

template <typename E, int DP, int TPW, bool PARTIAL>
__global__ __launch_bounds__((64 * ReplayShape<TPW, DP>::NW), (ReplayShape<TPW, DP>::WAVES_PER_EU)) void replay_fast_kernel(
    const AttnArgs a) {
  typedef FastTile<DP> T;
  constexpr int BN = T::BN, NDC = T::NDC, TILE = T::TILE;
  constexpr int DPW = T::DMA_PER_WAVE;
  constexpr int NW = ReplayShape<TPW, DP>::NW;   // waves per workgroup
  constexpr int RT = ReplayShape<TPW, DP>::RT;   // row tiles per workgroup
  constexpr float NEG_INF = -__builtin_huge_valf();
  constexpr float POS_INF = __builtin_huge_valf();

  __shared__ __attribute__((aligned(1024))) unsigned char lds_k0[TILE], lds_k1[TILE];
  __shared__ float red[2 * NW * BN];              // [2][NW][BN] per-wave column sums

  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool dmaw = wv < 4;                      // waves 0-3 issue the tile DMA
  const int N = a.N;

  // Heaviest causal query blocks first; the grid covers only workgroups with window rows.
  // With few such workgroups (a short observation window) each one's keys are split over
  // a.rsplit blocks (block-uniform: an empty share exits before any barrier).
  __shared__ int s_item;
  const int item = block_item(a, &s_item, wv);
  if (item >= (a.queue ? a.nitems : (int)gridDim.x)) return;
  const int lane = lane_now(), l32 = lane & 31, hh = lane >> 5;
  const int BH = a.BH, G = a.G, Hkv = a.Hkv, rsplit = a.rsplit;
  const int bh = (int)((unsigned)item % (unsigned)BH);
  const int rest = (int)((unsigned)item / (unsigned)BH);
  const int ks = rest % rsplit;
  const int wg = a.wg_bh - 1 - rest / rsplit;
  const int b = bh / Hkv, hkv = bh - b * Hkv;
  const int t_begin = wg * RT;
  const int t_end = min(a.tiles_bh, t_begin + RT);
  const int wg_q_hi = min(N, ((t_end - 1) / G + 1) * 32);
  const int kv_end = a.causal ? wg_q_hi : N;
  const int ntiles_all = (kv_end + BN - 1) / BN;
  const int per = (ntiles_all + rsplit - 1) / rsplit;
  const int it_lo = ks * per;                     // this block's key tiles [it_lo, ntiles)
  const int ntiles = min(ntiles_all, it_lo + per);
  if (it_lo >= ntiles) return;

  // This wave's row tiles j: 32 query positions from q0[j] of query head head[j]. A operand:
  // query row q0 + l32, channels 16c + 8h .. +7; nb: minus the bias of the 16 rows a lane
  // holds in the accumulator (register i: row 8(i/4) + 4h + i%4).
  const u32 qneg = a.neg_scale ? 0x80008000u : 0u;   // a negative scale runs as |scale| on -Q
  int q0[TPW];
  u32x4 qf[TPW][NDC];
  float nb[TPW][16];
  int wave_hi = -1;
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int t = t_begin + TPW * wv + j;
    const bool tv = t < t_end;
    const int tt = tv ? t : t_begin;
    q0[j] = (tt / G) * 32;
    const int head = hkv * G + (tt - (tt / G) * G);
    const bool rin = tv && q0[j] + 31 >= a.win_lo;
    if (rin) wave_hi = max(wave_hi, a.causal ? min(q0[j] + 31, N - 1) : N - 1);
    const int qr = q0[j] + l32;
    const bool ok = rin && qr < N;
    const u16* qp = a.q + b * a.qs[0] + head * a.qs[1] + (long long)(ok ? qr : 0) * a.qs[2];
#pragma unroll
    for (int c = 0; c < NDC; ++c) qf[j][c] = ok ? ((load8(qp, a.qs[3], 16 * c + 8 * hh, PARTIAL ? a.Dq : DP, a.qvec) & a.qmask) ^ qneg) : (u32x4){0u, 0u, 0u, 0u};
    const float br = ok ? a.bias[(long long)(b * a.Hq + head) * N + qr] : POS_INF;
#pragma unroll
    for (int i = 0; i < 16; ++i) nb[j][i] = -__shfl(br, 8 * (i >> 2) + 4 * hh + (i & 3));
  }

  // K tiles in the attention kernel's channel-group-major layout: fragment c of key
  // 32s + l32 at c*2048 + s*1024 + koff; one DMA offset register (see dma_tile_cm)
  const u32 koff = (u32)(l32 * 32 + ((hh ^ ((l32 >> 3) & 1)) << 4));
  const u32 krow = (u32)(a.ks[2] * 2);
  const u32 dk = (u32)(lane >> 1) * krow + (u32)(((lane & 1) ^ ((lane >> 4) & 1)) << 4);
  // PARTIAL: the lane's first channel in its K group, recomputed at each DMA (held across
  // the loop it would be spilled at tile dim 128)
  auto dchk = [&]() {
    const int ln = lane_now();
    return (u32)(((ln & 1) ^ ((ln >> 4) & 1)) << 3);
  };
  const unsigned char* kg = (const unsigned char*)(a.k + b * a.ks[0] + hkv * a.ks[1]);
  float* imp_row = a.imp + (long long)bh * N;

  auto flush = [&](int kb_prev, int buf_prev) {
    if (wv == 0) {                               // BN = 64: wave 0 sums one key per lane
      const int ln = lane_now();
      const float* rr = red + buf_prev * NW * BN + ln;
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < NW; w += 2) sum += rr[w * BN] + rr[(w + 1) * BN];
      const int key = kb_prev + ln;
      if (sum != 0.f && key < N) unsafeAtomicAdd(imp_row + key, sum);
    }
  };

  auto step = [&](int it, int BUF) __attribute__((always_inline)) {
    const int kb = it * BN;
    if (dmaw) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (it > it_lo) flush(kb - BN, BUF ^ 1);
    if (dmaw && it + 1 < ntiles)
      dma_tile_cm<DPW, 32, PARTIAL>(kg, krow, dk, kb + BN, N, BUF == 0 ? lds_k1 : lds_k0, wv, a.D, PARTIAL ? dchk() : 0u);
    float cs[2] = {0.f, 0.f};
    if (kb <= wave_hi) {
      const unsigned char* kt = BUF == 0 ? lds_k0 : lds_k1;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        f32x16 sacc[TPW];
#pragma unroll
        for (int j = 0; j < TPW; ++j) sacc[j] = (f32x16){};
#pragma unroll
        for (int c = 0; c < NDC; ++c) {
          const u32x4 kf = *(const u32x4*)(kt + c * 2048 + s * 1024 + koff);
#pragma unroll
          for (int j = 0; j < TPW; ++j) sacc[j] = E::mfma(qf[j][c], kf, sacc[j]);
        }
        float c4[4];
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
          // lanes hold key kb + 32s + l32; causal mask on diagonal tiles
          if (a.causal && kb + BN - 1 > q0[j]) {
            const int ln = lane_now();
            const int rel = (ln & 31) - 4 * (ln >> 5) + (kb + 32 * s - q0[j]);
#pragma unroll
            for (int i = 0; i < 16; ++i) sacc[j][i] = rel > 8 * (i >> 2) + (i & 3) ? NEG_INF : sacc[j][i];
          }
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float e = fast_exp2(fmaf(sacc[j][i], a.abs_scale_log2, nb[j][i]));
            if (j == 0 && i < 4)
              c4[i] = e;
            else
              c4[i & 3] += e;
          }
        }
        cs[s] = (c4[0] + c4[1]) + (c4[2] + c4[3]);
      }
    }
    cs[0] = half_swap_sum(cs[0]);
    cs[1] = half_swap_sum(cs[1]);
    const int ln = lane_now();
    if (ln < 32) {
      float* rb = red + BUF * NW * BN + wv * BN;
      rb[ln] = cs[0];
      rb[32 + ln] = cs[1];
    }
  };

  if (dmaw) dma_tile_cm<DPW, 32, PARTIAL>(kg, krow, dk, it_lo * BN, N, lds_k0, wv, a.D, PARTIAL ? dchk() : 0u);
  for (int it = it_lo; it < ntiles; it += 2) {
    step(it, 0);
    if (it + 1 < ntiles) step(it + 1, 1);
  }
  __syncthreads();
  flush((ntiles - 1) * BN, (ntiles - 1 - it_lo) & 1);
}

namespace {

// Row tiles per replay wave (build options; two by default). Three at tile dim 128 (252
// registers, two waves per SIMD, each K fragment read from LDS feeding three MFMAs) replayed all
// rows of the headline shape 1.3% faster but the headline's 1050 rows 0.5% slower (fewer,
// larger workgroups); below 128 three were 3-13% slower.
#ifndef FE_REPLAY_TPW
#define FE_REPLAY_TPW 2
#endif
#ifndef FE_REPLAY_TPW128
#define FE_REPLAY_TPW128 2
#endif
template <typename E, int DP, bool PARTIAL>
ReplayPlan replay_entry(const char* name) {
  constexpr int TPW = DP > 128 ? 1 : (DP == 128 ? FE_REPLAY_TPW128 : FE_REPLAY_TPW);
  return ReplayPlan{(const void*)replay_fast_kernel<E, DP, TPW, PARTIAL>, ReplayShape<TPW, DP>::NW,
                    ReplayShape<TPW, DP>::RT, name};
}

// Tile dims of the fast kernels: multiples of 32 up to 256 (the tile DMA moves 32-channel
// multiples; above 128 each LDS buffer holds one tile instead of two). A head dim D (a multiple
// of 8, at most 256) runs on the tile dim DP = D rounded up to 32; when D < DP the PARTIAL
// instantiation reads zeros past channel D and stores only D channels.
constexpr int kFastDims = 8;
int fast_slot(int D) { return (D >= 8 && D <= 256 && D % 8 == 0) ? (D + 31) / 32 - 1 : -1; }

#define FE_REPLAY_PAIR(E, e, DP) \
  replay_entry<E, DP, false>("replay_fast<" e "," #DP ">"), replay_entry<E, DP, true>("replay_fast<" e "," #DP ",partial>")
#define FE_REPLAY_ENTRIES(E, e)                                                                                   \
  FE_REPLAY_PAIR(E, e, 32), FE_REPLAY_PAIR(E, e, 64), FE_REPLAY_PAIR(E, e, 96), FE_REPLAY_PAIR(E, e, 128),          \
      FE_REPLAY_PAIR(E, e, 160), FE_REPLAY_PAIR(E, e, 192), FE_REPLAY_PAIR(E, e, 224), FE_REPLAY_PAIR(E, e, 256)
// [dtype][tile dim][partial]
ReplayPlan g_replay[] = {FE_REPLAY_ENTRIES(F16, "f16"), FE_REPLAY_ENTRIES(BF16, "bf16")};

template <typename E, int DP, int NW, bool FUSED, bool PARTIAL>
FusedPlan fast_entry(const char* name) {
  return FusedPlan{(const void*)fused_fast_kernel<E, DP, NW, FUSED, PARTIAL>, 0, NW, NW, name};   // static LDS only
}

// Per (dtype, tile dim, partial): the attention-only kernel (split schedule, or no importance)
// and the fused kernel with the replay traversal (fe_prefill without a workspace). At tile dims
// 32 and 64 both stay at 8 waves: about 115 registers and 68 KiB of LDS at 64 already put two
// workgroups, four waves per SIMD, on a CU. 96 runs 12 waves like 128 (96 KiB of LDS: one
// workgroup per CU either way).
#define FE_FAST_PAIR(E, e, DP, NW, P, ps)                                                      \
  fast_entry<E, DP, NW, false, P>("attn_fast<" e "," #DP ps ">"),                               \
      fast_entry<E, DP, NW, true, P>("fused_fast<" e "," #DP ps ">")
#define FE_FAST_DIM(E, e, DP, NW) FE_FAST_PAIR(E, e, DP, NW, false, ""), FE_FAST_PAIR(E, e, DP, NW, true, ",partial")
#define FE_FAST_ENTRIES(E, e)                                                                                     \
  FE_FAST_DIM(E, e, 32, 8), FE_FAST_DIM(E, e, 64, 8), FE_FAST_DIM(E, e, 96, 12), FE_FAST_DIM(E, e, 128, 12),      \
      FE_FAST_DIM(E, e, 160, 8), FE_FAST_DIM(E, e, 192, 8), FE_FAST_DIM(E, e, 224, 4), FE_FAST_DIM(E, e, 256, 4)
// [dtype][tile dim][partial][fused]
FusedPlan g_fast[] = {FE_FAST_ENTRIES(F16, "f16"), FE_FAST_ENTRIES(BF16, "bf16")};
// Small grids at tile dims 32 and 64 (attention only): 4-wave workgroups of one row tile per
// wave, single-tile LDS buffers, four workgroups per CU, so twice the work items of the 8-wave
// kernel and each SIMD's four waves from four workgroups. Chosen by the launch when the 8-wave
// kernel's items would fill at most one round of its resident workgroups: the reference
// harness's Hq4/Hkv2 shape at 8K and 32K (a quarter and one round) measured 11% and 4.4% faster;
// at two rounds (B1 Hq32/Hkv8 N8192) 4-7% slower, at eight (N32768) 3% slower. At tile dims 96
// and 128 (two workgroups per CU) it stands in for attn_rt2_kernel up to 1.5 rounds of the latter's
// items (B2 Hq8/Hkv2 N4000: 30% faster).
#define FE_FAST_SMALL_DIM(E, e, DP) \
  fast_entry<E, DP, 4, false, false>("attn_fast4<" e "," #DP ">"), fast_entry<E, DP, 4, false, true>("attn_fast4<" e "," #DP ",partial>")
// [dtype][tile dim 32, 64, 96, 128][partial]
FusedPlan g_fast_small[] = {FE_FAST_SMALL_DIM(F16, "f16", 32), FE_FAST_SMALL_DIM(F16, "f16", 64),
                            FE_FAST_SMALL_DIM(F16, "f16", 96), FE_FAST_SMALL_DIM(F16, "f16", 128),
                            FE_FAST_SMALL_DIM(BF16, "bf16", 32), FE_FAST_SMALL_DIM(BF16, "bf16", 64),
                            FE_FAST_SMALL_DIM(BF16, "bf16", 96), FE_FAST_SMALL_DIM(BF16, "bf16", 128)};
// Attention-only traversal with two row tiles per wave at tile dims 96 and 128 (attn_rt2_kernel:
// 8 waves, 16 row tiles per workgroup), head dims below the tile dim included: 3-5% faster than
// fused_fast_kernel's 12 waves of one row tile on every measured configuration at D = 128, 3% at
// D = 80 and 96, 6% at D = 120 (B1 Hq32/Hkv8 N16384). At tile dim 64 (12 waves of two row tiles,
// 152 registers, three per SIMD) it was 16% slower than the 8-wave kernel that runs two
// workgroups per CU there, so 64 keeps that kernel. -D FE_ATTN_RT2=0 restores the 12-wave kernel
// everywhere. Bit s of FE_ATTN_RT2 selects tile dim 32(s+1) (s = 2, 3).
#ifndef FE_ATTN_RT2
#define FE_ATTN_RT2 12
#endif
#ifndef FE_ATTN_RT2_PARTIAL
#define FE_ATTN_RT2_PARTIAL 1
#endif
#define FE_RT2_ENTRY(E, e, DP, P, ps) FusedPlan{(const void*)attn_rt2_kernel<E, DP, P>, 0, 8, 16, "attn_rt2<" e "," #DP ps ">"}
#define FE_RT2_DIM(E, e, DP) FE_RT2_ENTRY(E, e, DP, false, ""), FE_RT2_ENTRY(E, e, DP, true, ",partial")
#define FE_RT2_ENTRIES(E, e) FE_RT2_DIM(E, e, 96), FE_RT2_DIM(E, e, 128)
// [dtype][tile dim 96, 128][partial]
FusedPlan g_rt2[] = {FE_RT2_ENTRIES(F16, "f16"), FE_RT2_ENTRIES(BF16, "bf16")};
static_assert(sizeof(g_replay) / sizeof(g_replay[0]) == 4 * kFastDims, "replay table");
static_assert(sizeof(g_fast) / sizeof(g_fast[0]) == 8 * kFastDims, "fast table");

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

bool kv_ok(const void* p, const long long* st, int N, int D) {
  if (st[3] != 1 || !aligned16(p) || st[0] % 8 || st[1] % 8 || st[2] % 8 || st[2] < D) return false;
  // byte offsets of rows up to N + 64 (one tile past the end) must fit the 32-bit range
  return (unsigned long long)(N + 64) * (unsigned long long)st[2] * 2ull < (1ull << 31);
}

}  // namespace

bool fast_layout(const AttnArgs& a) {
  return fast_slot(a.D) >= 0 && kv_ok(a.k, a.ks, a.N, a.D) && kv_ok(a.v, a.vs, a.N, a.D);
}

bool fast_plan(const AttnArgs& a, int dtype, FusedPlan& plan) {
  const int slot = fast_slot(a.D);
  if (slot < 0) return false;
  // Q is read once per row tile, element-wise when it is not 16-byte vectorisable (any
  // strides); K and V go through the tile DMA, which needs aligned unit-stride rows. The
  // scale must be positive here: the caller runs a negative one as |scale| on -Q and a zero
  // one with Q zeroed at load (AttnArgs::qmask).
  if (!(a.abs_scale_log2 > 0.f) || !fast_layout(a)) return false;
  const bool fused = a.score && !a.bias;
  // below the tile dim (the PARTIAL instantiation) when K/V or Q have fewer channels
  const int partial = (a.D != 32 * (slot + 1) || a.Dq != 32 * (slot + 1)) ? 1 : 0;
  if (!fused && (slot == 2 || slot == 3) && ((FE_ATTN_RT2 >> slot) & 1) && (!partial || FE_ATTN_RT2_PARTIAL)) {
    plan = g_rt2[2 * (2 * (dtype == 1 ? 1 : 0) + slot - 2) + partial];
    return true;
  }
  const int idx = 2 * (2 * ((dtype == 1 ? kFastDims : 0) + slot) + partial) + (fused ? 1 : 0);
  plan = g_fast[idx];
  return true;
}

bool fast_plan_small(const AttnArgs& a, int dtype, FusedPlan& plan) {
  const int slot = fast_slot(a.D);
  if (slot < 0 || slot > 3 || !(a.abs_scale_log2 > 0.f) || !fast_layout(a) || (a.score && !a.bias)) return false;
  const int partial = (a.D != 32 * (slot + 1) || a.Dq != 32 * (slot + 1)) ? 1 : 0;
  plan = g_fast_small[2 * (4 * (dtype == 1 ? 1 : 0) + slot) + partial];
  return true;
}

bool replay_plan(const AttnArgs& a, int dtype, ReplayPlan& plan) {
  FusedPlan fp;
  if (!fast_plan(a, dtype, fp)) return false;
  const int slot = fast_slot(a.D);
  plan = g_replay[2 * ((dtype == 1 ? kFastDims : 0) + slot) + ((a.D != 32 * (slot + 1) || a.Dq != 32 * (slot + 1)) ? 1 : 0)];
  return true;
}

void append_fast_resources(std::string& out) {
  for (const auto& e : g_replay) {
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
  auto plan_row = [&](const FusedPlan& e) {
    hipFuncAttributes attr;
    if (hipFuncGetAttributes(&attr, e.fn) != hipSuccess) return;
    char buf[512];
    snprintf(buf, sizeof(buf),
             "{\"kernel\":\"%s\",\"registers_per_thread\":%d,\"lds_static_bytes\":%zu,"
             "\"lds_dynamic_bytes\":%zu,\"scratch_bytes_per_thread\":%zu,\"max_threads_per_block\":%d},",
             e.name, attr.numRegs, (size_t)attr.sharedSizeBytes, e.lds, (size_t)attr.localSizeBytes,
             attr.maxThreadsPerBlock);
    out += buf;
  };
  for (const auto& e : g_fast) plan_row(e);
  for (const auto& e : g_fast_small) plan_row(e);
  for (const auto& e : g_rt2) plan_row(e);
}

}  // namespace fe
