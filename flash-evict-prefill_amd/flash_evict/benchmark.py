"""Latency and PyTorch-allocator peak measurements of one attention layer.

Same protocol as the reference's scripts/benchmark.py:18-126 (anishesg/flash-evict-prefill):
per method two warm-up calls, `--repeats` calls timed with HIP events (median reported),
then one more call with the allocator statistics reset around it; methods run in an
order shuffled by a seeded RNG per sequence length; the report also lists the device
kernels' registers, LDS and scratch (`kernel_resources`, standing in for the Triton
`device_caches` dump at :104-111). Methods, for q [1,H,N,D], k/v [1,Hkv,N,D] bf16 and
budget ceil(0.1 N):

  torch_flash            torch's fused SDPA (the reference's baseline attention)
  hip_attention_only     prefill(score=False)      (reference: triton_attention_only)
  fused_replay_scores    prefill()
  fused_replay_topk      evict(budget)
  flash_snap_w32/_w128   flash_snap(budget, window)
  gather_kv              gather_tokens of K and V by evict's kept indices (the adapters'
                         compaction step; not a method of the reference script)

Run as `python -m flash_evict.benchmark --lengths 8192 32768 --heads 28 --kv-heads 4
--dim 128 --output benchmark.json` with flash-evict-prefill_amd/ on PYTHONPATH.

`--kernels` instead times the HBM-bound kernels on scaled synthetics (the headline's score
array is only 1 MiB, where they are launch-latency bound) and reports achieved GB/s against
algorithmic bytes (each input byte read once, each output byte written once).

`--policies` runs the protocol of the reference's scripts/benchmark_policies.py:26-96: for
every length, torch_flash and hip_attention_only once, then per budget flash_snap at windows
32 and 128 and `evict(budget, **policy)` for every scoring policy (a JSON list of
{name, recency_decay, observation_window, value_weighted, reserved_recent, pool_kernel} via
`--policy-file`, else DEFAULT_POLICIES, the reference's published rows), in a seeded
shuffled order, appending to an existing report with the same arguments (resumable).
"""
import argparse
import gc
import hashlib
import json
import math
import os
import random
import statistics
import subprocess
from pathlib import Path

import torch

from . import evict, gather_tokens, kernel_resources, prefill
from . import _lib
from .baselines import flash_attention, flash_snap


@torch.inference_mode()
def measure(fn, repeats):
    """Median of `repeats` event-timed calls after two warm-ups, then allocator peaks of
    one more call (scripts/benchmark.py:18-49)."""
    for _ in range(2):
        result = fn()
        del result
    torch.cuda.synchronize()
    times = []
    for _ in range(repeats):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        result = fn()
        end.record()
        end.synchronize()
        times.append(start.elapsed_time(end))
        del result
    gc.collect()
    torch.cuda.empty_cache()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    before = torch.cuda.memory_stats()
    free_before, total = torch.cuda.mem_get_info()
    result = fn()
    torch.cuda.synchronize()
    after = torch.cuda.memory_stats()
    record = {"median_ms": statistics.median(times), "samples_ms": times,
              "allocated_before_bytes": before["allocated_bytes.all.current"],
              "peak_allocated_bytes": after["allocated_bytes.all.peak"],
              "peak_increment_bytes": after["allocated_bytes.all.peak"] - before["allocated_bytes.all.current"],
              "peak_reserved_bytes": after["reserved_bytes.all.peak"],
              "free_device_bytes_before": free_before, "total_device_bytes": total}
    del result
    return record


def _tool_output(cmd):
    """Text output of a diagnostic tool, or a note when it is unavailable."""
    try:
        return subprocess.run(cmd, capture_output=True, text=True, timeout=20).stdout
    except (OSError, subprocess.SubprocessError) as e:
        return "unavailable: %s" % e


def _git_revision():
    try:
        return subprocess.check_output(["git", "rev-parse", "HEAD"], text=True, stderr=subprocess.DEVNULL,
                                       cwd=os.path.dirname(os.path.abspath(__file__))).strip()
    except (OSError, subprocess.SubprocessError):
        return None


def _sources():
    here = Path(__file__).resolve().parent
    files = [here / "prefill.py", here / "baselines.py", here / "cache.py", Path(_lib.LIB_PATH)]
    return {f.name: hashlib.sha256(f.read_bytes()).hexdigest() for f in files if f.exists()}


def methods_for(q, k, v, budget):
    """The timed callables of one sequence length."""
    kept = {}

    def gather_kv():
        if "idx" not in kept:   # kept indices of one evict() call, made in the first warm-up
            kept["idx"] = evict(q, k, v, budget)[2]
        return gather_tokens(k, kept["idx"]), gather_tokens(v, kept["idx"])
    return {
        "torch_flash": lambda: flash_attention(q, k, v),
        "hip_attention_only": lambda: prefill(q, k, v, score=False),
        "fused_replay_scores": lambda: prefill(q, k, v),
        "fused_replay_topk": lambda: evict(q, k, v, budget),
        "flash_snap_w32": lambda: flash_snap(q, k, v, budget, 32),
        "flash_snap_w128": lambda: flash_snap(q, k, v, budget, 128),
        "gather_kv": gather_kv,
    }


# Scoring policies of the reference's published policy benchmark (results/policy_benchmark.json
# rows d01_r0 and d0.1_w128_*), plus the decay-1 and window-128 policies of its sweep.
DEFAULT_POLICIES = [
    dict(name="d01_r0", recency_decay=.1, observation_window=0, value_weighted=True, reserved_recent=0, pool_kernel=1),
    dict(name="d0.1_w128_r0", recency_decay=.1, observation_window=128, value_weighted=True, reserved_recent=0,
         pool_kernel=1),
    dict(name="d0.1_w128_r64", recency_decay=.1, observation_window=128, value_weighted=True, reserved_recent=64,
         pool_kernel=1),
    dict(name="w128_r64", recency_decay=0., observation_window=128, value_weighted=True, reserved_recent=64,
         pool_kernel=1),
    dict(name="d1_r64", recency_decay=1., observation_window=0, value_weighted=True, reserved_recent=64,
         pool_kernel=1),
]


def policy_methods(q, k, v, budgets, policies):
    """(name, budget, callable) of one length (scripts/benchmark_policies.py:58-67)."""
    methods = [("torch_flash", None, lambda: flash_attention(q, k, v)),
               ("hip_attention_only", None, lambda: prefill(q, k, v, score=False))]
    for budget in budgets:
        for window in (32, 128):
            methods.append(("snap_w%d" % window, budget, lambda b=budget, w=window: flash_snap(q, k, v, b, w)))
        for policy in policies:
            kw = {key: val for key, val in policy.items() if key != "name"}
            methods.append((policy["name"], budget, lambda b=budget, kw=kw: evict(q, k, v, b, **kw)))
    return methods


def run_policies(args):
    policies = DEFAULT_POLICIES
    if args.policy_file:
        policies = json.loads(Path(args.policy_file).read_text())
    torch.manual_seed(20260910)
    dest = Path(args.output)
    dest.parent.mkdir(parents=True, exist_ok=True)
    run_args = {"lengths": args.lengths, "budgets": args.budgets, "repeats": args.repeats, "heads": args.heads,
                "kv_heads": args.kv_heads, "dim": args.dim}
    report = {"args": run_args, "policies": policies, "gpu": torch.cuda.get_device_name(), "torch": torch.__version__,
              "hip": torch.version.hip, "dtype": "bfloat16", "batch": 1, "git_revision": _git_revision(),
              "source_sha256": _sources(),
              "scope": "one layer; incremental allocations, inputs excluded; output, scores, selection included",
              "rows": []}
    if dest.exists():
        old = json.loads(dest.read_text())
        for key in ("args", "policies"):
            if old.get(key) != report[key]:
                raise ValueError("existing report %s was made with other %s" % (dest, key))
        report = old
    done = {(r["n"], r["method"], r["budget"]) for r in report["rows"]}
    for n in args.lengths:
        q = torch.randn((1, args.heads, n, args.dim), device="cuda", dtype=torch.bfloat16)
        k = torch.randn((1, args.kv_heads, n, args.dim), device="cuda", dtype=q.dtype)
        v = torch.randn_like(k)
        methods = policy_methods(q, k, v, args.budgets, policies)
        random.Random(n).shuffle(methods)
        for name, budget, fn in methods:
            if (n, name, budget) in done:
                continue
            try:
                row = {"n": n, "method": name, "budget": budget, **measure(fn, args.repeats)}
            except torch.OutOfMemoryError as e:
                row = {"n": n, "method": name, "budget": budget, "error": "OOM", "detail": str(e)}
                gc.collect()
                torch.cuda.empty_cache()
            report["rows"].append(row)
            done.add((n, name, budget))
            report["kernel_resources"] = kernel_resources()
            dest.write_text(json.dumps(report, indent=2) + "\n")
            print(json.dumps({key: val for key, val in row.items() if key != "samples_ms"}), flush=True)
        del q, k, v
        gc.collect()
        torch.cuda.empty_cache()
    expected = len(args.lengths) * (2 + len(args.budgets) * (2 + len(policies)))
    report["complete"] = len(done) == expected
    dest.write_text(json.dumps(report, indent=2) + "\n")


def _event_ms(fn, repeats):
    """Median HIP-event time of `fn` (on torch's current stream) after two warm-ups."""
    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    times = []
    for _ in range(repeats):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        fn()
        end.record()
        end.synchronize()
        times.append(start.elapsed_time(end))
    return statistics.median(times)


@torch.inference_mode()
def kernel_rows(repeats):
    """Scaled-synthetic timings of the zero-fill, selection and gather kernels."""
    from .prefill import _select
    rows, n, budget, recent = 256, 131072, 1024, 64
    g = torch.Generator(device="cuda").manual_seed(20260910)
    scores = torch.rand((rows, n), device="cuda", generator=g)
    out = []

    def row(name, fn, nbytes, shape):
        ms = _event_ms(fn, repeats)
        out.append({"kernel": name, "shape": shape, "median_ms": ms, "algorithmic_bytes": nbytes,
                    "GB/s": nbytes / (ms * 1e-3) / 1e9, "frac_of_8TB/s": nbytes / (ms * 1e-3) / 8e12})
        print(json.dumps(out[-1]), flush=True)

    zbuf = torch.empty(rows * n, dtype=torch.float32, device="cuda")
    L = _lib.lib()

    def zero():
        _lib.check(L.fe_zero_f32(zbuf.data_ptr(), zbuf.numel(), torch.cuda.current_stream().cuda_stream), "fe_zero_f32")
    row("zero_f32", zero, rows * n * 4, "%d x %d float32" % (rows, n))
    sel_bytes = rows * n * 4 + rows * n + rows * budget * 8
    row("select (top-k + mask + indices)", lambda: _select(scores, budget, recent, 1, False), sel_bytes,
        "%d rows x %d, budget %d, recent %d" % (rows, n, budget, recent))
    pool_bytes = sel_bytes + 2 * rows * (n - recent) * 4
    row("select with pool 5", lambda: _select(scores, budget, recent, 5, False), pool_bytes,
        "%d rows x %d, budget %d, recent %d, pool 5 (pooled scores written and read once)" % (rows, n, budget, recent))
    h, keys, d, keep = 8, 131072, 128, 65536
    cache = torch.randn((1, keys, h, d), device="cuda", generator=g).to(torch.bfloat16).transpose(1, 2)
    idx = torch.sort(torch.randperm(keys, device="cuda", generator=g)[:keep]).values.expand(1, h, keep).contiguous()
    gbytes = 2 * h * keep * d * 2 + h * keep * 8
    row("gather_tokens", lambda: gather_tokens(cache, idx), gbytes,
        "%d heads x %d of %d rows x %d bf16 (transposed view)" % (h, keep, keys, d))
    return out


def main(argv=None):
    p = argparse.ArgumentParser()
    p.add_argument("--lengths", type=int, nargs="+", default=[8192, 32768, 131072])
    p.add_argument("--heads", type=int, default=4)
    p.add_argument("--kv-heads", type=int, default=2)
    p.add_argument("--dim", type=int, default=64)
    p.add_argument("--repeats", type=int, default=5)
    p.add_argument("--methods", nargs="+", default=None, help="subset of the method names")
    p.add_argument("--output", default="benchmark.json")
    p.add_argument("--kernels", action="store_true", help="time the HBM-bound kernels on scaled synthetics")
    p.add_argument("--policies", action="store_true", help="policy latency at fixed budgets")
    p.add_argument("--budgets", type=int, nargs="+", default=[256, 1024])
    p.add_argument("--policy-file", default=None, help="JSON list of scoring policies (--policies)")
    args = p.parse_args(argv)
    if args.policies:
        run_policies(args)
        return
    if args.kernels:
        report = {"gpu": torch.cuda.get_device_name(), "torch": torch.__version__, "hip": torch.version.hip,
                  "rows": kernel_rows(args.repeats)}
        Path(args.output).write_text(json.dumps(report, indent=2) + "\n")
        return
    torch.manual_seed(20260910)
    output = Path(args.output)
    output.parent.mkdir(parents=True, exist_ok=True)
    report = {"args": vars(args), "gpu": torch.cuda.get_device_name(), "torch": torch.__version__,
              "hip": torch.version.hip, "dtype": "bfloat16", "batch": 1, "git_revision": _git_revision(),
              "source_sha256": _sources(), "rocm_smi_before": _tool_output(["rocm-smi"]),
              "scope": "single attention layer; allocations include output and selection, exclude inputs",
              "rows": []}
    for n in args.lengths:
        q = torch.randn((1, args.heads, n, args.dim), device="cuda", dtype=torch.bfloat16)
        k = torch.randn((1, args.kv_heads, n, args.dim), device="cuda", dtype=q.dtype)
        v = torch.randn_like(k)
        budget = math.ceil(n * .1)
        methods = methods_for(q, k, v, budget)
        if args.methods:
            methods = {name: fn for name, fn in methods.items() if name in args.methods}
        # Seeded order reduces a systematic warm-up/temperature ordering effect.
        items = list(methods.items())
        random.Random(n).shuffle(items)
        for name, fn in items:
            try:
                row = {"n": n, "method": name, "budget": budget, **measure(fn, args.repeats)}
            except torch.OutOfMemoryError as e:
                row = {"n": n, "method": name, "error": "OOM", "detail": str(e)}
                gc.collect()
                torch.cuda.empty_cache()
            report["rows"].append(row)
            report["kernel_resources"] = kernel_resources()
            output.write_text(json.dumps(report, indent=2) + "\n")
            print(json.dumps({key: val for key, val in row.items() if key != "samples_ms"}), flush=True)
        del q, k, v
        gc.collect()
        torch.cuda.empty_cache()


if __name__ == "__main__":
    main()
