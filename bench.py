"""Benchmark of the flash_evict prefill hot path on one MI355X.

A step is one full `evict()` layer (zero-init, attention kernel + replay kernel, value-norm
scaling, radix top-k + mask) over resident synthetic inputs. The default is the headline shape
B=1, Hq=32, Hkv=8, N=32768, D=128, bf16, causal, budget 1024, recency_decay 0.1,
reserved_recent 64, all-query window (observation_window 0); --config selects the other
BASELINE configs (tiny and edge in fp16, llama8k, qwen32k_w128, long131k), the headline in
fp16, the reference harness's default shape (ref8k, ref32k, ref128k) and D=64 at the headline
head counts (d64_b10).

Work counts. The metric's definition of a layer's work is 4*D*P_attn + 2*D*P_replay with
P_attn = B*Hq*N(N+1)/2 (causal) and P_replay the query-key pairs of the last W query rows
(W = the observation window, all rows when 0): 13.19 TFLOP at the headline. The library
replays only the last R = fe_replay_rows(N, W, recency_decay) of them, because rows whose
recency weight exp(-decay*(N-1-q)) is exactly zero in FP32 (decay*(N-1-q) >= 105) add exactly
nothing to the importance: 9.07 TFLOP executed at the headline (R = 1050).

Prints one JSON line on stdout:
  value              = TFLOP the kernels execute per layer / measured layer time
  value_defined_work = the metric's defined TFLOP per layer / measured layer time
  ms_per_step        = ms per layer (the metric's first half), timed without instrumentation
  roofline           = the attention + replay kernels alone: executed TFLOP / their mean
                       duration, timed with HIP events the library records on the kernels'
                       own stream over as many further layers; frac = fraction of dense bf16
                       MFMA peak
  full_replay        = the same inputs with recency_decay 0 (every one of the 32768 rows
                       replayed, so executed = defined work): layer ms and the attention +
                       replay kernels' ms, TFLOP/s and fraction of peak, from the same run
  cpu_baseline       = the CPU oracle (oracle/attention.chunked, FP32 torch) on a sample of
                       the same workload's query heads, on the box's usable host cores
                       (reported only)
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "flash-evict-prefill_amd"), ROOT]

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 (and fp16) MFMA (published)

# name: shape, element type, input recipe and evict() arguments. The first five after the
# headline are the BASELINE.json configs (tiny and edge in fp16); headline_f16 is the headline
# in fp16; ref8k/ref32k/ref131k are the reference harness's default shape (scripts/benchmark.py:
# Hq4/Hkv2/D64 bf16, budget ceil(0.1 N), default scoring: every row replayed); d64_b10 is D=64
# at the headline head counts with every row replayed.
_HL = dict(B=1, Hq=32, Hkv=8, N=32768, D=128)
_HL_EVICT = dict(budget=1024, recency_decay=0.1, reserved_recent=64, observation_window=0, pool_kernel=1)
CONFIGS = {
    "headline": dict(_HL, dtype="bf16", evict=_HL_EVICT),
    "tiny": dict(B=1, Hq=4, Hkv=4, N=512, D=64, dtype="f16",
                 evict=dict(budget=64, recency_decay=0.0, reserved_recent=0, observation_window=0, pool_kernel=1)),
    "edge": dict(B=2, Hq=8, Hkv=2, N=4000, D=128, dtype="f16", causal=False, value_weighted=False, qk_scale=30.0,
                 transposed=True, zero_v_rows=0.1,
                 evict=dict(budget=400, recency_decay=0.0, reserved_recent=0, observation_window=0, pool_kernel=1)),
    "llama8k": dict(B=1, Hq=32, Hkv=8, N=8192, D=128, dtype="bf16", outlier_channels=4,
                    evict=dict(budget=1024, recency_decay=0.1, reserved_recent=64, observation_window=0, pool_kernel=1)),
    "qwen32k_w128": dict(B=1, Hq=28, Hkv=4, N=32768, D=128, dtype="bf16",
                         evict=dict(budget=2048, recency_decay=0.0, reserved_recent=64, observation_window=128,
                                    pool_kernel=5)),
    "long131k": dict(B=1, Hq=32, Hkv=8, N=131072, D=128, dtype="bf16",
                     evict=dict(budget=1024, recency_decay=0.1, reserved_recent=64, observation_window=0, pool_kernel=1)),
    "headline_f16": dict(_HL, dtype="f16", evict=_HL_EVICT),
    "headline_b10": dict(_HL, dtype="bf16", evict=dict(budget=3277, recency_decay=0.0, reserved_recent=0,
                                                        observation_window=0, pool_kernel=1)),
    "d64_b10": dict(B=1, Hq=32, Hkv=8, N=32768, D=64, dtype="bf16",
                    evict=dict(budget=3277, recency_decay=0.0, reserved_recent=0, observation_window=0, pool_kernel=1)),
}
for _n in (8192, 32768, 131072):
    CONFIGS["ref%dk" % (_n // 1024)] = dict(B=1, Hq=4, Hkv=2, N=_n, D=64, dtype="bf16",
                                           evict=dict(budget=-(-_n // 10), recency_decay=0.0, reserved_recent=0,
                                                      observation_window=0, pool_kernel=1))


def last_plan():
    """Kernels of this thread's last prefill launch, as the library names them (fe_last_plan):
    the attention kernel, and the replay kernel when the split schedule ran."""
    import ctypes
    from flash_evict import _lib
    buf = ctypes.create_string_buffer(512)
    _lib.check(_lib.lib().fe_last_plan(buf, len(buf)), "fe_last_plan")
    return buf.value.decode()


def make_inputs(cfg, dev):
    """Seeded synthetic q, k, v of the config, resident on `dev` (drawn on the device)."""
    import torch
    dt = torch.bfloat16 if cfg["dtype"] == "bf16" else torch.float16
    b, hq, hk, n, d = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["N"], cfg["D"]
    gen = torch.Generator(device=dev).manual_seed(20260910)
    if cfg.get("transposed"):
        q = torch.randn((b, n, hq, d), device=dev, generator=gen).transpose(1, 2)
        k = torch.randn((b, n, hk, d), device=dev, generator=gen).transpose(1, 2)
        v = torch.randn((b, n, hk, d), device=dev, generator=gen).transpose(1, 2)
    else:
        q = torch.randn((b, hq, n, d), device=dev, generator=gen)
        k = torch.randn((b, hk, n, d), device=dev, generator=gen)
        v = torch.randn((b, hk, n, d), device=dev, generator=gen)
    s = cfg.get("qk_scale", 1.0)
    q, k = q * s, k * s
    if cfg.get("outlier_channels"):
        ch = torch.randperm(d, generator=gen, device=dev)[: cfg["outlier_channels"]]
        q[..., ch] *= 8
        k[..., ch] *= 8
    if cfg.get("zero_v_rows"):
        rows = torch.randperm(n, generator=gen, device=dev)[: int(n * cfg["zero_v_rows"])]
        v[:, :, rows] = 0
    return q.to(dt), k.to(dt), v.to(dt)


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


def _usable_cores():
    """Host cores this process may use: its affinity set, capped by a cgroup CPU quota when
    one is set (containers often pin many cores but grant a smaller share)."""
    affinity = len(os.sched_getaffinity(0))
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()[:2]
        if q != "max":
            quota = int(q) / int(period)
    except (OSError, ValueError):
        quota = None
    cores = affinity if quota is None else max(1, min(affinity, int(quota + 0.999)))
    return cores, affinity, quota


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(q, k, v, kw, executed_flop, sample_heads=8):
    """The reference's CPU-capable path restated (oracle/attention.chunked: FP32 softmax
    attention and importance, then the library's host selection) on the host cores.

    Times `sample_heads` query heads over all N queries after one untimed warm-up, and
    reports the rate on the same work count as the GPU line's `value` (the per-head work is
    uniform, so the sample's rate is the layer's rate); ms_per_layer scales the sample time
    by the head count."""
    import torch
    from oracle.attention import chunked
    from flash_evict import _lib
    cores, affinity, quota = _usable_cores()
    torch.set_num_threads(cores)
    b, hq, n, d = q.shape
    hk = k.shape[1]
    g = hq // hk
    sample_heads = min(sample_heads, hq)
    kv_needed = (sample_heads + g - 1) // g
    qc, kc, vc = q[:1, :sample_heads].cpu(), k[:1, :kv_needed].cpu(), v[:1, :kv_needed].cpu()
    args = dict(causal=kw.get("causal", True), value_weighted=kw.get("value_weighted", True),
                recency_decay=kw["recency_decay"], observation_window=kw["observation_window"], block=1024)
    chunked(qc, kc, vc, heads=[(0, 0)], query_rows=[(0, 2048)], **args)        # warm-up
    t0 = time.perf_counter()
    _, imp = chunked(qc, kc, vc, **args)
    dt = time.perf_counter() - t0
    layer_s = dt * (b * hq) / sample_heads
    # host selection (fe_select_host, one thread) on a [B*Hkv, N] score array of the layer's size
    scores = imp[0, :1].expand(b * hk, n).contiguous()
    idx = torch.empty((b * hk, kw["budget"]), dtype=torch.int64)
    mask = torch.empty((b * hk, n), dtype=torch.bool)
    L = _lib.lib()
    t1 = time.perf_counter()
    _lib.check(L.fe_select_host(scores.data_ptr(), b * hk, n, n, kw["budget"], kw["reserved_recent"],
                                kw["pool_kernel"], idx.data_ptr(), mask.data_ptr(), 0), "fe_select_host")
    sel_ms = (time.perf_counter() - t1) * 1e3
    return {
        "value": round(executed_flop / layer_s / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": "oracle chunked FP32, %d of %d q-heads x %d rows, %.1f s" % (sample_heads, b * hq, n, dt),
        "ms_per_layer": round(layer_s * 1e3 + sel_ms, 1),
        "select_host_ms": round(sel_ms, 2),
        "affinity_cores": affinity,
        "cgroup_cpu_quota": quota,
        "torch_threads": torch.get_num_threads(),
        "cpu_model": _cpu_model(),
        "note": "rate on the GPU line's executed-work count; ms_per_layer = sample time x %g + host selection "
                "(1 thread); one untimed warm-up" % ((b * hq) / sample_heads),
    }


def _timed_layers(step, steps, warmup, tag, warmup_ms=0.0):
    """Run at least `warmup` untimed layers, continuing back to back until `warmup_ms` of
    warm-up have passed, then `steps` timed layers, then `steps` more with the library's HIP
    events around the attention + replay kernels; return (ms per layer, those kernels' ms per
    launch, launches, warm-up layers run).

    The minimum warm-up time is there for the GPU's power management: after a change of load
    the part first runs these kernels at a clock well below the one it then holds (measured on
    the llama8k layer: about 1.85 GHz for the first layers, 1.55-1.65 GHz from the third to
    the tenth, 1.93 GHz steady from about the sixtieth layer, 35 ms in), so a few warm-up
    layers time the controller's transient instead of the kernels."""
    import ctypes
    import torch
    from flash_evict import _lib
    L = _lib.lib()
    t_start = time.perf_counter()
    for i in range(warmup):
        step()
        torch.cuda.synchronize()
        log("%s warmup %d/%d done" % (tag, i + 1, warmup))
    done, t_log = warmup, time.perf_counter()
    while (time.perf_counter() - t_start) * 1e3 < warmup_ms:
        for _ in range(8):
            step()
        torch.cuda.synchronize()
        done += 8
        if time.perf_counter() - t_log > 0.5:
            t_log = time.perf_counter()
            log("%s warmup: %d layers, %.2f s" % (tag, done, t_log - t_start))
    # the timed layers run without the library's timing events (each event record costs the
    # stream about 6 us, 1.7% of a llama8k layer); the same number of layers follows with the
    # events on, for the attention + replay kernels' own duration (roofline)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    _lib.check(L.fe_fused_timing_read(None, None), "fe_fused_timing_read")
    _lib.check(L.fe_fused_timing_enable(1), "fe_fused_timing_enable")
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    _lib.check(L.fe_fused_timing_enable(0), "fe_fused_timing_enable")
    launches = ctypes.c_int64(0)
    fused_ms = ctypes.c_double(0.0)
    _lib.check(L.fe_fused_timing_read(ctypes.byref(launches), ctypes.byref(fused_ms)), "fe_fused_timing_read")
    ms = elapsed * 1e3 / steps
    log("%s timed %d steps after %d warm-up layers (%.2f s): %.3f ms/layer" % (
        tag, steps, done, t0 - t_start, ms))
    return ms, fused_ms.value / max(1, launches.value), launches.value, done


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--warmup-ms", type=float, default=1500.0,
                    help="minimum warm-up time per measured phase (untimed layers run back to back)")
    ap.add_argument("--config", default="headline", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-full-replay", action="store_true")
    ap.add_argument("--traffic-json", default=os.path.join(ROOT, "profiles", "attn_replay_headline_traffic.json"),
                    help="rocprofv3 PMC summary giving HBM bytes per fused launch (optional)")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (the path shards by (batch, KV head) with "
              "no exchange; multi-GPU runs are not part of it). Use --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import flash_evict

    cfg = CONFIGS[args.config]
    b, hq, hk, n, d = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["N"], cfg["D"]
    causal, weighted = cfg.get("causal", True), cfg.get("value_weighted", True)
    kw = dict(cfg["evict"], causal=causal, value_weighted=weighted)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    log("config %s: B=%d Hq=%d Hkv=%d N=%d D=%d %s %s" % (args.config, b, hq, hk, n, d, cfg["dtype"], kw))
    q, k, v = make_inputs(cfg, dev)
    torch.cuda.synchronize()

    def make_step(decay):
        def step():
            return flash_evict.evict(q, k, v, kw["budget"], reserved_recent=kw["reserved_recent"],
                                     pool_kernel=kw["pool_kernel"], recency_decay=decay,
                                     observation_window=kw["observation_window"], causal=causal,
                                     value_weighted=weighted)
        return step

    def flops(decay, effective=True):
        return algorithmic_flop(b, hq, n, d, kw["observation_window"], decay, causal=causal, effective=effective)

    with torch.inference_mode():
        ms, fused_avg_ms, launches, warm_run = _timed_layers(make_step(kw["recency_decay"]), args.steps,
                                                             args.warmup, args.config, args.warmup_ms)
        plan_name = last_plan()
        full = None
        if kw["recency_decay"] > 0 and not args.no_full_replay:
            fsteps = max(3, args.steps // 2)
            f_ms, f_fused, f_launches, f_warm = _timed_layers(make_step(0.0), fsteps, min(2, args.warmup),
                                                              "full-replay", args.warmup_ms)
            f_flop = flops(0.0)
            f_ach = f_flop / (f_fused * 1e-3) / 1e12
            full = {"recency_decay": 0.0, "replay_rows": replay_rows(n, kw["observation_window"], 0.0),
                    "executed_tflop": round(f_flop / 1e12, 4), "ms_per_layer": round(f_ms, 4),
                    "fused_mean_ms": round(f_fused, 4), "fused_achieved_tflops": round(f_ach, 2),
                    "fused_frac": round(f_ach / PEAK_BF16_TFLOPS, 4), "launches": f_launches,
                    "steps": fsteps, "warmup_layers_run": f_warm}
    flop = flops(kw["recency_decay"], effective=False)
    executed = flops(kw["recency_decay"])
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
        "value": round(executed / (ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_layers_run": warm_run,
        "warmup_min_ms": args.warmup_ms,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": cfg["dtype"],
        "data": "synthetic (seeded normal q/k/v resident in HBM%s)" % (
            "; q,k x%g, %s" % (cfg.get("qk_scale", 1.0), ", ".join(x for x in (
                "transposed [B,N,H,D] views" if cfg.get("transposed") else "",
                "%d%% zero v rows" % int(100 * cfg["zero_v_rows"]) if cfg.get("zero_v_rows") else "",
                "%d outlier channels x8" % cfg["outlier_channels"] if cfg.get("outlier_channels") else "") if x))
            if any(cfg.get(x) for x in ("transposed", "zero_v_rows", "outlier_channels", "qk_scale")) else ""),
        "config": {"workload": "evict() layer, %s" % args.config, "B": b, "Hq": hq, "Hkv": hk, "N": n, "D": d,
                   **kw, "algorithmic_tflop": round(flop / 1e12, 4),
                   "replay_rows": replay_rows(n, kw["observation_window"], kw["recency_decay"]),
                   "executed_tflop": round(executed / 1e12, 4)},
        "value_defined_work": round(flop / (ms * 1e-3) / 1e12, 2),
        "roofline": {"bound": "mfma", "kernel": plan_name,
                     "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                     "mean_ms": round(fused_avg_ms, 4), "launches": launches},
        "fused_share_of_layer": round(fused_avg_ms / ms, 4),
        "full_replay": full,
    }
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        record["cpu_baseline"] = cpu_baseline(q, k, v, kw, executed)
    else:
        record["cpu_baseline"] = None
    print(json.dumps(record), flush=True)


if __name__ == "__main__":
    main()
