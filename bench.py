"""Benchmark of the flash_evict prefill hot path on one MI355X.

A step is one full `evict()` layer (zero-init, fused attention + replay-score kernel,
value-norm scaling, radix top-k + mask) over resident synthetic bf16 inputs at the
headline shape B=1, Hq=32, Hkv=8, N=32768, D=128, causal, budget 1024, recency_decay 0.1,
reserved_recent 64, all-query replay (observation_window 0).

Prints one JSON line on stdout:
  value        = the layer's algorithmic attention+score TFLOP / measured layer time
  ms_per_step  = ms per layer (the metric's first half)
  roofline     = the fused kernel alone: the TFLOP it executes / its mean duration, timed
                 with HIP events recorded by the library on the kernel's own stream
  cpu_baseline = the CPU oracle (oracle/attention.chunked) on one query head of the same
                 workload, extrapolated to the layer (reported only)
Algorithmic work of a layer (the metric's definition): 4*D*P_attn + 2*D*P_replay with
P_attn = B*Hq*N(N+1)/2 (causal) and P_replay the query-key pairs of the last W query rows
(W = the observation window, all rows when 0). The library replays only the last
R = fe_replay_rows(N, W, recency_decay) of them: rows whose recency weight
exp(-decay*(N-1-q)) is exactly zero in FP32 (decay*(N-1-q) >= 105) add exactly nothing to the
importance. The roofline counts the work executed (R rows), so its fraction of peak is the
MFMA utilisation; `config` lists both counts.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "flash-evict-prefill_amd"), ROOT]

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA (published)

CONFIGS = {
    # name: (B, Hq, Hkv, N, D, evict kwargs)
    "headline": (1, 32, 8, 32768, 128, dict(budget=1024, recency_decay=0.1, reserved_recent=64,
                                            observation_window=0, pool_kernel=1)),
    "headline_b10": (1, 32, 8, 32768, 128, dict(budget=3277, recency_decay=0.0, reserved_recent=0,
                                                observation_window=0, pool_kernel=1)),
    "llama8k": (1, 32, 8, 8192, 128, dict(budget=1024, recency_decay=0.1, reserved_recent=64,
                                          observation_window=0, pool_kernel=1)),
    "qwen32k_w128": (1, 28, 4, 32768, 128, dict(budget=2048, recency_decay=0.0, reserved_recent=64,
                                                observation_window=128, pool_kernel=5)),
    "long131k": (1, 32, 8, 131072, 128, dict(budget=1024, recency_decay=0.1, reserved_recent=64,
                                             observation_window=0, pool_kernel=1)),
}


def log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


def replay_rows(n, window, recency_decay):
    """Query rows the library's replay visits (fe_replay_rows)."""
    from flash_evict import _lib
    rows = _lib.lib().fe_replay_rows(n, min(n, window or n), float(recency_decay))
    if rows < 1:
        raise ValueError("fe_replay_rows rejected n=%d window=%d decay=%g" % (n, window, recency_decay))
    return rows


def algorithmic_flop(b, hq, n, d, window, recency_decay=0.0, causal=True, effective=True):
    w = replay_rows(n, window, recency_decay) if effective else min(n, window or n)
    if causal:
        p_attn = b * hq * n * (n + 1) // 2
        # sum_{q=n-w}^{n-1} (q+1)
        p_replay = b * hq * (w * (2 * n - w + 1) // 2)
    else:
        p_attn = b * hq * n * n
        p_replay = b * hq * w * n
    return 4 * d * p_attn + 2 * d * p_replay


def cpu_baseline(q, k, v, kw, threads, sample_heads=8):
    """Time the CPU oracle on `sample_heads` query heads (all N queries, their KV heads) and
    extrapolate to the layer; also time the library's host selection on the layer's scores."""
    import ctypes
    import torch
    from oracle.attention import chunked
    from flash_evict import _lib
    torch.set_num_threads(threads)
    b, hq, n, d = q.shape
    hk = k.shape[1]
    g = hq // hk
    sample_heads = min(sample_heads, hq)
    kv_needed = (sample_heads + g - 1) // g
    qc, kc, vc = q[:1, :sample_heads].cpu(), k[:1, :kv_needed].cpu(), v[:1, :kv_needed].cpu()
    args = dict(causal=True, value_weighted=True, recency_decay=kw["recency_decay"],
                observation_window=kw["observation_window"], block=1024)
    t0 = time.perf_counter()
    _, imp = chunked(qc, kc, vc, **args)
    dt = time.perf_counter() - t0
    layer_s = dt * (b * hq) / sample_heads
    flop = algorithmic_flop(b, hq, n, d, kw["observation_window"], kw["recency_decay"], effective=False)
    # host selection (fe_select_host) on a [B*Hkv, N] score array of the layer's size
    scores = imp[0, :1].expand(b * hk, n).contiguous()
    idx = torch.empty((b * hk, kw["budget"]), dtype=torch.int64)
    mask = torch.empty((b * hk, n), dtype=torch.bool)
    L = _lib.lib()
    t1 = time.perf_counter()
    _lib.check(L.fe_select_host(scores.data_ptr(), b * hk, n, n, kw["budget"], kw["reserved_recent"],
                                kw["pool_kernel"], idx.data_ptr(), mask.data_ptr(), 0), "fe_select_host")
    sel_ms = (time.perf_counter() - t1) * 1e3
    cpu_model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(flop / layer_s / 1e12, 4),
        "unit": "TFLOP/s",
        "ms_per_layer": round(layer_s * 1e3 + sel_ms, 1),
        "cores": threads,
        "kind": "port",
        "select_host_ms": round(sel_ms, 2),
        "sample": "oracle/attention.chunked (FP32 torch CPU, 1024-query blocks) on %d of %d query heads "
                  "(all %d queries), %.2f s measured, x%g extrapolated; selection: fe_select_host on "
                  "%d x %d scores (1 thread); CPU %s" % (sample_heads, b * hq, n, dt, (b * hq) / sample_heads,
                                                          b * hk, n, cpu_model),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="headline", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--traffic-json", default=os.path.join(ROOT, "profiles", "fused_attn_score_headline_traffic.json"),
                    help="rocprofv3 PMC summary giving HBM bytes per fused launch (optional)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (the path shards by (batch, KV head) with "
              "no exchange; multi-GPU runs are not part of it). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import flash_evict
    from flash_evict import _lib

    b, hq, hk, n, d, kw = CONFIGS[args.config]
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log("config %s: B=%d Hq=%d Hkv=%d N=%d D=%d %s" % (args.config, b, hq, hk, n, d, kw))
    gen = torch.Generator(device=dev).manual_seed(20260910)
    q = torch.randn((b, hq, n, d), device=dev, dtype=torch.bfloat16, generator=gen)
    k = torch.randn((b, hk, n, d), device=dev, dtype=torch.bfloat16, generator=gen)
    v = torch.randn((b, hk, n, d), device=dev, dtype=torch.bfloat16, generator=gen)
    torch.cuda.synchronize()

    def step():
        return flash_evict.evict(q, k, v, kw["budget"], reserved_recent=kw["reserved_recent"],
                                 pool_kernel=kw["pool_kernel"], recency_decay=kw["recency_decay"],
                                 observation_window=kw["observation_window"])

    with torch.inference_mode():
        for i in range(args.warmup):
            step()
            torch.cuda.synchronize()
            log("warmup %d/%d done" % (i + 1, args.warmup))
        L = _lib.lib()
        _lib.check(L.fe_fused_timing_read(None, None), "fe_fused_timing_read")
        _lib.check(L.fe_fused_timing_enable(1), "fe_fused_timing_enable")
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        _lib.check(L.fe_fused_timing_enable(0), "fe_fused_timing_enable")
        import ctypes
        launches = ctypes.c_int64(0)
        fused_ms = ctypes.c_double(0.0)
        _lib.check(L.fe_fused_timing_read(ctypes.byref(launches), ctypes.byref(fused_ms)),
                   "fe_fused_timing_read")
    ms = elapsed * 1e3 / args.steps
    log("timed %d steps: %.3f ms/layer" % (args.steps, ms))
    flop = algorithmic_flop(b, hq, n, d, kw["observation_window"], kw["recency_decay"], effective=False)
    executed = algorithmic_flop(b, hq, n, d, kw["observation_window"], kw["recency_decay"])
    fused_avg_ms = fused_ms.value / max(1, launches.value)
    achieved = executed / (fused_avg_ms * 1e-3) / 1e12
    traffic = None
    if os.path.exists(args.traffic_json):
        try:
            with open(args.traffic_json) as f:
                tj = json.load(f)
            if tj.get("config") == args.config:
                traffic = tj.get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    record = {
        "metric": "ms/layer + fused attn+score TFLOP/s (% MFMA peak), N=32K Hq32/Hkv8 D128 bf16",
        "value": round(flop / (ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v resident in HBM)",
        "config": {"workload": "evict() layer, %s" % args.config, "B": b, "Hq": hq, "Hkv": hk, "N": n, "D": d,
                   "causal": True, **kw, "algorithmic_tflop": round(flop / 1e12, 4),
                   "replay_rows": replay_rows(n, kw["observation_window"], kw["recency_decay"]),
                   "executed_tflop": round(executed / 1e12, 4)},
        "roofline": {"bound": "mfma", "kernel": "fused_attn_score", "achieved": round(achieved, 2),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic, "mean_ms": round(fused_avg_ms, 4), "launches": launches.value},
        "fused_share_of_layer": round(fused_avg_ms / ms, 4),
    }
    if not args.no_cpu_baseline:
        threads = max(1, min(16, len(os.sched_getaffinity(0))))
        log("cpu baseline on %d threads ..." % threads)
        record["cpu_baseline"] = cpu_baseline(q, k, v, kw, threads)
    else:
        record["cpu_baseline"] = None
    print(json.dumps(record), flush=True)


if __name__ == "__main__":
    main()
