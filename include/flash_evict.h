/*
 * flash_evict C ABI — MI355X (gfx950) prefill hot path.
 *
 * Every entry point is `extern "C"`, takes plain pointers, sizes and an opaque HIP
 * stream, returns 0 on success and a negative code on failure (the message is then
 * available from fe_last_error() on the calling thread). Nothing here throws, and
 * nothing synchronises the stream: work is enqueued and the call returns.
 *
 * Reference interfaces replaced (paths are in anishesg/flash-evict-prefill):
 *   fe_prefill        flash_evict/prefill.py:128-136  (importance zero-init + the Triton
 *                     `_prefill[(cdiv(N,BM), B*Hq)](...)` launch, kernel at :14-83)
 *   fe_prefill_ws     the same launch (prefill.py:128-136); the workspace carries the
 *                     per-row replay bias between the attention and replay kernels
 *   fe_zero_f32       flash_evict/prefill.py:129      (`torch.zeros` of the score array)
 *   fe_select         flash_evict/prefill.py:160-169  (avg_pool1d, topk, tail arange/cat,
 *                     sort, scatter_ of `select_tokens`), plus :180 (`~keep`) when invert=1
 *   fe_select_host    the same `select_tokens` body for CPU tensors (tests call it on CPU,
 *                     tests/test_prefill.py:77-84,149-159)
 *   fe_gather_rows    kv_distill.cache.gather_tokens as called at
 *                     flash_evict/kv_distill_adapter.py:38-39, streaming_adapter.py:86,
 *                     quality_adapter.py:109-110 (KV compaction by the kept indices)
 *   fe_snap_scores    flash_evict/baselines.py:15-27 (`snap_scores`, the SnapKV observation-
 *                     window scores of the baseline path; its selection, snap_select at
 *                     :30-40, is fe_select with recent = min(window, n, budget-1))
 *   fe_kernel_resources  scripts/benchmark.py:104-111 (`_prefill.device_caches` resource dump)
 */
#ifndef FLASH_EVICT_H_
#define FLASH_EVICT_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of q/k/v/out. */
enum { FE_DTYPE_F16 = 0, FE_DTYPE_BF16 = 1 };

/* Error codes. */
enum {
  FE_OK = 0,
  FE_ERR_INVALID = -1,     /* argument out of the supported range */
  FE_ERR_HIP = -2,         /* a HIP runtime call failed */
  FE_ERR_WORKSPACE = -3,   /* workspace missing or too small */
  FE_ERR_UNSUPPORTED = -4  /* shape/layout this build does not handle */
};

/*
 * Fused prefill: attention output plus exact replay importance.
 *
 * q: [B,Hq,N,D], k/v: [B,Hkv,N,D], any element strides (qs/ks/vs = {b,h,n,d} strides in
 * elements). out: contiguous [B,Hq,N,D] of the input dtype. importance: contiguous
 * [B,Hkv,N] float32 (may be NULL when score == 0).
 *
 *   out[b,h,q,:]   = softmax_k(scale * q.k, causal)[q,:] @ v           (P rounded to the
 *                    input dtype before P@V, FP32 accumulation)
 *   importance[b,j,k] = ||v[b,j,k,:]||_1 (if value_weighted) *
 *                    sum_{h in group j} sum_q w_q softmax(...)[b,h,q,k],
 *   w_q = exp(recency_decay * (q - (N-1))) for q >= N - window, else 0.
 *
 * `window` is the already-clamped observation window: min(N, observation_window or N).
 * The call zero-fills `importance` itself before accumulating into it.
 * The attention output does not depend on score/window/value_weighted (bitwise).
 */
int fe_prefill(const void* q, const void* k, const void* v, void* out, float* importance,
               int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
               const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
               int dtype, float scale, int causal, int value_weighted, int score,
               float recency_decay, int64_t window, void* hip_stream);

/*
 * Number of query rows the importance replay of fe_prefill visits: `window`, less the
 * oldest rows whose recency weight exp(-recency_decay*(N-1-q)) is exactly zero in FP32
 * (recency_decay*(N-1-q) >= 105), i.e. min(window, ceil(105/recency_decay)) when
 * recency_decay > 0. Those rows contribute exactly zero to every column in the reference
 * (flash_evict/prefill.py:66-67 weights them by an underflowed 0.0), so skipping them does
 * not change the importance. -1 for arguments fe_prefill would reject. No counterpart in
 * the reference (which replays every window row); for work accounting and tests.
 */
int64_t fe_replay_rows(int64_t N, int64_t window, float recency_decay);

/*
 * fe_prefill with a caller-provided workspace (same contract). fe_prefill_workspace_bytes()
 * is B*Hq*N floats of replay biases (score != 0; none otherwise), rounded up to 256 bytes,
 * plus 4 KiB of work-item counters. With the fast layouts (D a multiple of 8 up to 256,
 * nonzero scale, unit-stride 16-byte aligned K/V rows; Q of any strides):
 *   * the replay runs as a second kernel at higher occupancy: the attention kernel leaves the
 *     per-row replay bias m_q + log2 l_q - decay*log2(e)*(q-N+1) in the workspace;
 *   * with the whole workspace, the work items of the attention and replay kernels (groups of
 *     query rows, heaviest first) are taken from per-XCD queues in the counters as CUs free
 *     up (the call zeroes them first), instead of one per workgroup index. Each item is
 *     computed the same way whichever workgroup takes it: the output is bitwise that of the
 *     static schedule, the importance equal up to FP32 atomic order;
 *   * with the whole workspace and a short observation window (at most a quarter of the rows
 *     replayed) at head dims 8..64 and 72..128, in launches that fill the GPU, the replay runs
 *     as work items of the attention launch instead of a second kernel (same arithmetic:
 *     output bitwise equal, importance equal up to FP32 atomic order); each waits for its rows' attention item, and runs that item
 *     itself if the wait runs out (a GPU another kernel shares). With longer windows the
 *     heaviest 3% of the row groups replay that way, in the attention launch's tail, and the
 *     second kernel replays the other rows; causal launches at head dims up to 128 too small to
 *     fill the GPU replay every row as items, lightest rows first;
 *   * score == 0 uses the counters alone;
 *   * a zero scale runs on the fast kernels with Q zeroed at load (every logit exactly 0).
 * At head dims 72..128 (multiples of 8) the split schedule's attention kernel holds two row
 * tiles per wave and takes a row's reference max over its first 32 keys instead of 64: the
 * output then agrees with fe_prefill's to within two roundings of the probabilities, the
 * importance to FP32 summation order; at other head dims, and for launches of at most 1.5
 * rounds of that kernel's work items (which run one row tile per wave instead), the output
 * is bitwise equal and the importance equal up to FP32 atomic order. With room for the biases but not the counters
 * the schedule is static; with less workspace (or NULL) this is fe_prefill. Same reference
 * interface as fe_prefill.
 */
size_t fe_prefill_workspace_bytes(int64_t B, int64_t Hq, int64_t N, int score);
/*
 * fe_prefill_workspace_bytes plus, when the fast kernels cannot read K or V as laid out (rows
 * off 16-byte alignment, a channel stride other than 1, broadcast rows, a head dim that is not
 * a multiple of 8), room for both repacked into aligned rows of D rounded up to 8 channels
 * (2 * B*Hkv*N*ceil8(D) elements, each area 256-byte aligned). With that much workspace
 * fe_prefill_ws copies K and V there (an HBM-bound kernel) and runs the fast kernels instead of
 * the generic one; the output and importance are those of the same call on a contiguous copy.
 * The pointers are only inspected (alignment), never dereferenced. No counterpart in the
 * reference, whose Triton kernel reads any strides in place (prefill.py:131-136).
 */
size_t fe_prefill_workspace_bytes_kv(int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D, int score,
                                     const void* k, const int64_t* k_strides, const void* v,
                                     const int64_t* v_strides);
int fe_prefill_ws(const void* q, const void* k, const void* v, void* out, float* importance,
                  int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                  const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                  int dtype, float scale, int causal, int value_weighted, int score,
                  float recency_decay, int64_t window, void* workspace, size_t workspace_bytes,
                  void* hip_stream);

/*
 * fe_prefill_ws with the replay-bias workspace taken from a fixed device buffer inside the
 * library, so the call allocates nothing: no hipMalloc/hipFree and no allocating library
 * routine (and no timing events: fe_fused_timing_enable does not apply to it). No
 * counterpart in the reference; it is for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The buffer holds FE_STATIC_BIAS_ROWS floats and the work-item counters (16 MiB + 4 KiB) on
 * every GPU this entry point has run on, from its first call there until the process ends
 * (processes that never call it do not hold the buffer). A scoring call needs
 * B*Hq*N <= FE_STATIC_BIAS_ROWS and otherwise fails with FE_ERR_WORKSPACE before launching
 * anything. Every call on one GPU shares that GPU's buffer: calls that overlap on one GPU
 * (concurrent streams or threads) race, so the caller must order them. Results: those of
 * fe_prefill_ws with its whole workspace (bitwise output, importance up to FP32 atomic order).
 */
#define FE_STATIC_BIAS_ROWS 4194304
int fe_prefill_static(const void* q, const void* k, const void* v, void* out, float* importance,
                      int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                      const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                      int dtype, float scale, int causal, int value_weighted, int score,
                      float recency_decay, int64_t window, void* hip_stream);

/* Zero-fill n floats with a fill kernel (graph-capture safe: no hipMemset node). */
int fe_zero_f32(float* p, int64_t n, void* hip_stream);

/*
 * Token selection over `rows` score rows of length n (row r starts at
 * scores + r * row_stride, unit element stride, float32).
 *   past = row[:n-recent]; if pool_kernel > 1 and budget > recent, past is replaced by
 *   avg_pool1d(past, pool_kernel, stride 1, pad pool_kernel/2, count_include_pad);
 *   the (budget - recent) largest entries of past are kept (ties: lower index first),
 *   together with the suffix [n-recent, n).
 * indices_out: [rows, budget] int64, ascending. mask_out: [rows, n] bytes (0/1), the keep
 * mask, or the eviction mask (1 = evict) when invert != 0. Either output may be NULL.
 * workspace: device memory of at least fe_select_workspace_bytes(...) bytes (may be NULL
 * when that is 0): rows*(n-recent) floats of pooled scores when pooling, none otherwise.
 */
size_t fe_select_workspace_bytes(int64_t rows, int64_t n, int64_t budget, int64_t recent,
                                 int pool_kernel);
int fe_select(const float* scores, int64_t rows, int64_t n, int64_t row_stride,
              int64_t budget, int64_t recent, int pool_kernel,
              int64_t* indices_out, uint8_t* mask_out, int invert,
              void* workspace, size_t workspace_bytes, void* hip_stream);

/* The same selection on host memory (CPU tensors); identical results to fe_select. */
int fe_select_host(const float* scores, int64_t rows, int64_t n, int64_t row_stride,
                   int64_t budget, int64_t recent, int pool_kernel,
                   int64_t* indices_out, uint8_t* mask_out, int invert);

/*
 * KV compaction gather: out[b,h,j,:] = x[b,h,indices[b,h,j],:].
 * x: [B,H,N,D] elements of elem_bytes (1, 2, 4 or 8) bytes with element strides
 * x_strides = {b,h,n,d} (nonnegative); indices: [B,H,K] int64 with element strides
 * index_strides = {b,h,j} (zero strides broadcast); out: contiguous [B,H,K,D].
 * An index outside [0, N) yields a zero row. Rows move as 16-byte chunks when the
 * channel stride is 1 and rows, strides and pointers are 16-byte aligned.
 */
int fe_gather_rows(const void* x, const int64_t* indices, void* out,
                   int64_t B, int64_t H, int64_t N, int64_t D, int64_t K,
                   const int64_t* x_strides, const int64_t* index_strides, int elem_bytes,
                   void* hip_stream);

/*
 * SnapKV observation-window scores (baseline path). With W = min(window, N) and
 * G = Hq/Hkv, for every query head h of group j the last W query positions t give
 *   p[h,t,:] = softmax_FP32(float(round_dtype(q[b,h,t,:] . k[b,j,n,:])) * D^-0.5,
 *                           causal: n <= t)
 *   scores[b,j,n] = (1/G) * sum_{h in group j} sum_t p[h,t,n]
 * q: [B,Hq,N,D], k: [B,Hkv,N,D] with element strides {b,h,n,d}; scores: contiguous
 * [B,Hkv,N] float32, every element written. workspace: device memory of at least
 * fe_snap_scores_workspace_bytes(...) bytes. window >= 1.
 */
size_t fe_snap_scores_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t window);
int fe_snap_scores(const void* q, const void* k, float* scores, int64_t B, int64_t Hq, int64_t Hkv,
                   int64_t N, int64_t D, const int64_t* q_strides, const int64_t* k_strides,
                   int dtype, int64_t window, void* workspace, size_t workspace_bytes,
                   void* hip_stream);

/*
 * Timing of the attention + importance kernels alone (the fused kernel, or the attention
 * and replay kernels of the split schedule): when enabled, fe_prefill / fe_prefill_ws
 * record a HIP event pair around them on the caller's stream. The switch and the record
 * are per calling thread: a thread times only its own calls and reads only its own
 * events. fe_fused_timing_read waits for the recorded events (not for the stream),
 * returns the number of timed launches and their total duration in milliseconds, and
 * clears the thread's record. No counterpart in the reference (benchmark support).
 */
int fe_fused_timing_enable(int enable);
int fe_fused_timing_read(int64_t* launches, double* total_ms);

/* JSON description of the device kernels (registers, LDS, scratch), written to buf. */
int fe_kernel_resources(char* buf, size_t cap);

/*
 * Names of the attention (+ replay) kernels the calling thread's last fe_prefill,
 * fe_prefill_ws or fe_prefill_static launched, e.g. "attn_rt2<bf16,128> + replay_fast<bf16,128>"
 * ("" before any such call), written to buf with its terminating zero. No counterpart in the
 * reference (benchmark support: which kernels a timing covers). FE_ERR_INVALID when cap is
 * too small.
 */
int fe_last_plan(char* buf, size_t cap);

/* Message of the last failing call on this thread ("" if none). */
const char* fe_last_error(void);

/* ABI version (incremented on incompatible changes). */
int fe_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FLASH_EVICT_H_ */
