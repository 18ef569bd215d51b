"""CPU oracle for the flash_evict prefill hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithm of the reference's evict() path so the
HIP kernels can be checked against it. Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import it, and only as the checker; the product package
(flash_evict) never imports or calls anything here.

Modules and the reference code each one restates (anishesg/flash-evict-prefill):
  attention.materialized   flash_evict/reference.py:5-25 (dense FP32 ground truth)
  attention.chunked        the same mathematics, streamed over query blocks so that the
                           N x N matrix is never materialised (row softmax is
                           independent per query, so the chunking is exact)
  select.select_tokens     flash_evict/prefill.py:140-170 (pool, top-k, tail, sort, mask)
  select.snap_select       flash_evict/baselines.py:28-40
  select.avg_pool          torch avg_pool1d(k, stride 1, pad k//2, count_include_pad)
  brute                    pure-Python loops over the same definitions (tiny inputs only)
  snap.snap_scores         flash_evict/baselines.py:15-27 (SnapKV observation-window scores)
  gather.gather_tokens     kv_distill.cache.gather_tokens as called at
                           flash_evict/kv_distill_adapter.py:38-39 (KV compaction)
  analytic                 closed forms used by tests/test_prefill.py:87-102,134-146

How each function is pinned (checked against something other than itself):
  materialized  golden known answers of the reference tests and notes
                (tests/test_prefill.py:62-74, RESEARCH_NOTES.md:47-52), closed forms for
                Q=K=0 (analytic), invariants (sum_k mass = G*sum_q w_q), brute-force loops
                in float64 on tiny inputs, and the textbook attention of
                torch.nn.functional.scaled_dot_product_attention for the output.
  chunked       equality with materialized on every shape the dense form fits, plus the
                closed forms at long N.
  select_tokens golden known answers (tests/test_prefill.py:77-84), torch.topk /
                torch.sort / F.avg_pool1d on tie-free inputs, brute-force selection, and
                the snap_select equivalence of tests/test_prefill.py:149-155.
  snap_select   torch.topk-based restatement on tie-free inputs.
  snap_scores   the reference's own check (tests/test_baselines.py:19-20: a full window
                gives the H2O mass of `materialized` / G), mass conservation (each key row
                sums to W), the q = 0 closed form (uniform causal rows) and float64 loops.
  gather_tokens torch.gather on in-range indices, brute-force loops, and the call-site
                identities (arange(N) gives the cache, the uniform_recent arange gives the
                suffix slice, quality_adapter.py:41-43).
Tie order among equal scores is parity unpinned by design: the reference leaves it to
torch.topk (flash_evict/prefill.py:144); this build keeps the lower index.
"""
