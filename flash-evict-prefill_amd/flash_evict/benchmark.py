"""Latency and PyTorch-allocator peak measurements of one attention layer on MI355X.

Protocol and report format of the reference's harnesses (scripts/benchmark.py:18-126 and
scripts/benchmark_policies.py:26-96 in anishesg/flash-evict-prefill): each measured call gets
two untimed warm-ups, then `--repeats` samples timed with HIP events (the median is reported),
then one more call with the allocator's peak statistics reset around it. Within a sequence
length the cases run in an order shuffled by a seeded RNG, the report is rewritten after
every row, and `--require-idle` refuses to report a row while another process holds the GPU.

Modes (q [1,H,N,D], k/v [1,Hkv,N,D] bf16):

  default      per length, budget ceil(0.1 N), the methods
                 torch_flash          torch's flash SDPA (the reference's baseline attention)
                 hip_attention_only   prefill(score=False)    (reference: triton_attention_only)
                 fused_replay_scores  prefill()
                 fused_replay_topk    evict(budget)
                 flash_snap_w32/_w128 flash_snap(budget, window)
                 gather_kv            gather_tokens of K and V by evict's kept indices (the
                                      adapters' compaction step; not in the reference script)
  --policies   per length torch_flash and hip_attention_only, then per budget flash_snap at
               windows 32 and 128 and evict(budget, **policy) for every scoring policy (a
               JSON list of {name, recency_decay, observation_window, value_weighted,
               reserved_recent, pool_kernel} from --policy-file, else DEFAULT_POLICIES);
               an existing report made with the same arguments is resumed
  --kernels    the HBM-bound kernels on scaled synthetics (the headline's score array is
               only 1 MiB, where they are launch-latency bound): achieved GB/s of
               algorithmic bytes (each input byte read once, each output byte written once)
  --generic    prefill on the shapes, scales and layouts the fast kernels do not read in
               place (head dims that are not a multiple of 8 and K/V rows off 16-byte
               alignment, which prefill() repacks into its workspace; a zero scale, run with Q
               zeroed at load), and the first two through the workspace-free entry point (the
               generic kernel), next to the fast path at D = 32, 64, 80, 96, 128, 192 and 256
               (and at D = 128 with a negative scale and with a channel-strided q, which it
               reads element-wise): attention only, and with every row replayed; TFLOP/s of the
               work the caller asked for (at D = 80 the kernels compute on 96-channel tiles)

Run as `python -m flash_evict.benchmark --lengths 8192 32768 --heads 28 --kv-heads 4
--dim 128 --output benchmark.json` with flash-evict-prefill_amd/ on PYTHONPATH.
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

SEED = 20260910

# Report keys of one measured row (the reference's format).
_ALLOC_KEYS = ("allocated_before_bytes", "peak_allocated_bytes", "peak_increment_bytes", "peak_reserved_bytes",
               "free_device_bytes_before", "total_device_bytes")


# ---------------------------------------------------------------- measurement primitives

def event_samples(fn, repeats, warmup=2):
    """GPU milliseconds of `repeats` calls of `fn`, each bracketed by its own pair of HIP
    events on the current stream, after `warmup` untimed calls. The events are read back
    once, after the last sample."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(repeats)]
    for begin, end in marks:
        begin.record()
        fn()
        end.record()
    torch.cuda.synchronize()
    return [begin.elapsed_time(end) for begin, end in marks]


def allocator_peaks(fn):
    """Allocator statistics of one call of `fn`, made with the caching allocator emptied
    and its peak counters reset: what the call allocates beyond its inputs."""
    gc.collect()
    torch.cuda.empty_cache()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    held = torch.cuda.memory_allocated()
    free, total = torch.cuda.mem_get_info()
    keep = fn()
    torch.cuda.synchronize()
    stats = torch.cuda.memory_stats()
    del keep
    peak = stats["allocated_bytes.all.peak"]
    values = (held, peak, peak - held, stats["reserved_bytes.all.peak"], free, total)
    return dict(zip(_ALLOC_KEYS, values))


@torch.inference_mode()
def measure(fn, repeats):
    """Median latency (and every sample) plus the allocator peaks of one call."""
    samples = event_samples(fn, repeats)
    return {"median_ms": statistics.median(samples), "samples_ms": samples, **allocator_peaks(fn)}


# ---------------------------------------------------------------- environment records

def _tool_output(cmd, timeout=20):
    try:
        return subprocess.run(cmd, capture_output=True, text=True, timeout=timeout).stdout
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
    files = [here / "prefill.py", here / "baselines.py", here / "cache.py", here / "benchmark.py", Path(_lib.LIB_PATH)]
    return {f.name: hashlib.sha256(f.read_bytes()).hexdigest() for f in files if f.exists()}


def parse_gpu_pids(text):
    """PIDs named in the JSON or table output of `amd-smi process` / `rocm-smi --showpids`."""
    pids = set()
    try:
        data = json.loads(text)
    except ValueError:
        data = None
    if data is not None:
        stack = [data]
        while stack:
            x = stack.pop()
            if isinstance(x, dict):
                for key, val in x.items():
                    tag = key.strip().upper()
                    if tag == "PID" and isinstance(val, (int, str)) and str(val).strip().isdigit():
                        pids.add(int(val))
                    elif tag.startswith("PID") and tag[3:].isdigit():
                        pids.add(int(tag[3:]))   # rocm-smi --showpids --json: {"PID1234": "name, ..."}
                    stack.append(val)
            elif isinstance(x, list):
                stack.extend(x)
        return sorted(pids)
    for line in text.splitlines():
        head = line.strip().split()
        if head and head[0].isdigit() and len(head) > 1:
            pids.add(int(head[0]))
    return sorted(pids)


class ContentionGuard:
    """Records the processes holding the GPU around each row (the reference's contention
    check, scripts/benchmark.py:60,90-115, on AMD's process queries) and, with
    `require_idle`, refuses to report a row measured while another process was present.
    The raw query output is kept in each row: inside a container whose PID namespace hides
    the KFD process directory, amd-smi reports "No running processes detected" even for
    this process, and the guard can then see no contention at all."""

    QUERIES = (["amd-smi", "process", "--json"], ["rocm-smi", "--showpids", "--json"])

    def __init__(self, require_idle):
        self.require_idle = require_idle
        self.query = None
        for cmd in self.QUERIES:
            out = _tool_output(cmd)
            if not out.startswith("unavailable") and out.strip():
                self.query = cmd
                break

    def snapshot(self):
        """(raw tool output, PIDs other than this process)."""
        if self.query is None:
            return "unavailable: no amd-smi/rocm-smi process query", []
        raw = _tool_output(self.query)
        return raw, [p for p in parse_gpu_pids(raw) if p != os.getpid()]

    def check(self, others, when):
        if self.require_idle and others:
            raise RuntimeError("other GPU processes %s %s the measurement; refusing an uncontended timing claim"
                               % (others, when))


# ---------------------------------------------------------------- cases

class Case:
    """One measured call: a sequence length, a method name, an optional budget."""

    def __init__(self, n, method, budget, fn):
        self.n, self.method, self.budget, self.fn = n, method, budget, fn

    @property
    def key(self):
        return (self.n, self.method, self.budget)


def layer_cases(q, k, v, n, names=None):
    """Methods of the default mode at budget ceil(0.1 N)."""
    budget = math.ceil(0.1 * n)
    kept = []

    def gather_kv():
        if not kept:            # the kept indices of one evict(), made in the first warm-up
            kept.append(evict(q, k, v, budget)[2])
        return gather_tokens(k, kept[0]), gather_tokens(v, kept[0])

    table = [("torch_flash", lambda: flash_attention(q, k, v)),
             ("hip_attention_only", lambda: prefill(q, k, v, score=False)),
             ("fused_replay_scores", lambda: prefill(q, k, v)),
             ("fused_replay_topk", lambda: evict(q, k, v, budget)),
             ("flash_snap_w32", lambda: flash_snap(q, k, v, budget, 32)),
             ("flash_snap_w128", lambda: flash_snap(q, k, v, budget, 128)),
             ("gather_kv", gather_kv)]
    return [Case(n, name, budget, fn) for name, fn in table if names is None or name in names]


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


def _evict_with(q, k, v, budget, policy):
    options = {key: val for key, val in policy.items() if key != "name"}
    return lambda: evict(q, k, v, budget, **options)


def policy_cases(q, k, v, n, budgets, policies):
    """Cases of the policy mode: the two attention baselines once, then per budget the two
    SnapKV windows and every scoring policy."""
    cases = [Case(n, "torch_flash", None, lambda: flash_attention(q, k, v)),
             Case(n, "hip_attention_only", None, lambda: prefill(q, k, v, score=False))]
    for budget in budgets:
        cases += [Case(n, "snap_w%d" % w, budget, (lambda b=budget, w=w: flash_snap(q, k, v, b, w))) for w in (32, 128)]
        cases += [Case(n, p["name"], budget, _evict_with(q, k, v, budget, p)) for p in policies]
    return cases


# ---------------------------------------------------------------- runner

class Report:
    """The JSON report: header fields, rows, resumable by (n, method, budget)."""

    def __init__(self, path, header, resume_keys=()):
        self.path = Path(path)
        self.path.parent.mkdir(parents=True, exist_ok=True)
        self.data = dict(header, rows=[])
        if resume_keys and self.path.exists():
            old = json.loads(self.path.read_text())
            for key in resume_keys:
                if old.get(key) != header[key]:
                    raise ValueError("existing report %s was made with other %s" % (self.path, key))
            self.data = old
        self.done = {(r["n"], r["method"], r["budget"]) for r in self.data["rows"]}

    def add(self, row):
        self.data["rows"].append(row)
        self.done.add((row["n"], row["method"], row["budget"]))
        self.data["kernel_resources"] = kernel_resources()
        self.save()

    def save(self):
        self.path.write_text(json.dumps(self.data, indent=2) + "\n")


def _measure_case(case, repeats, guard):
    raw_before, others_before = guard.snapshot()
    guard.check(others_before, "preceded")
    row = {"n": case.n, "method": case.method, "budget": case.budget}
    try:
        row.update(measure(case.fn, repeats))
    except torch.OutOfMemoryError as e:
        row.update(error="OOM", detail=str(e))
        gc.collect()
        torch.cuda.empty_cache()
    raw_after, others_after = guard.snapshot()
    row.update(compute_processes_before=raw_before, compute_processes_after=raw_after,
               other_compute_pids=sorted(set(others_before) | set(others_after)))
    guard.check(others_after, "overlapped")
    return row


def run(report, lengths, heads, kv_heads, dim, make_cases, repeats, guard):
    """Measure every case of every length not yet in the report, in a seeded shuffled
    order per length (ordering effects of warm-up and temperature average out)."""
    for n in lengths:
        q = torch.randn((1, heads, n, dim), device="cuda", dtype=torch.bfloat16)
        k = torch.randn((1, kv_heads, n, dim), device="cuda", dtype=torch.bfloat16)
        v = torch.randn_like(k)
        todo = [c for c in make_cases(q, k, v, n) if c.key not in report.done]
        random.Random(n).shuffle(todo)
        for case in todo:
            row = _measure_case(case, repeats, guard)
            report.add(row)
            print(json.dumps({key: val for key, val in row.items()
                              if key not in ("samples_ms", "compute_processes_before", "compute_processes_after")}),
                  flush=True)
        del q, k, v
        gc.collect()
        torch.cuda.empty_cache()


def _header(args, extra):
    return dict(args=extra.pop("args"), gpu=torch.cuda.get_device_name(), torch=torch.__version__,
                hip=torch.version.hip, dtype="bfloat16", batch=1, git_revision=_git_revision(),
                source_sha256=_sources(), **extra)


# ---------------------------------------------------------------- scaled-synthetic kernels

@torch.inference_mode()
def kernel_rows(repeats):
    """Scaled-synthetic timings of the zero-fill, selection, pooling and gather kernels."""
    from .prefill import _select
    rows, n, budget, recent = 256, 131072, 1024, 64
    g = torch.Generator(device="cuda").manual_seed(SEED)
    scores = torch.rand((rows, n), device="cuda", generator=g)
    out = []

    def row(name, fn, nbytes, shape):
        ms = statistics.median(event_samples(fn, repeats))
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
    for r2, n2 in ((8, 32768), (256, 32768)):       # the headline's rows; rows staged whole in LDS
        s2 = torch.rand((r2, n2), device="cuda", generator=g)
        b2 = r2 * n2 * 4 + r2 * n2 + r2 * budget * 8
        row("select %d x %d" % (r2, n2), lambda s2=s2: _select(s2, budget, recent, 1, True), b2,
            "%d rows x %d, budget %d, recent %d (evict mask)" % (r2, n2, budget, recent))
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


# ---------------------------------------------------------------- generic attention path

def _attention_flop(hq, n, d, replay):
    """Causal attention FLOP of one layer (B = 1): QK^T and P@V over the n(n+1)/2 visible
    pairs, plus the replay's QK^T recomputation when every row is replayed."""
    pairs = n * (n + 1) // 2
    return (4 + (2 if replay else 0)) * pairs * d * hq


def _workspace_free(q, k, v, scale, replay):
    """fe_prefill (no workspace) on q, k, v: the fused kernel, or the generic one where the fast
    kernels cannot read K/V in place or the scale is zero."""
    from . import _lib
    from .prefill import _DTYPES
    b, h, n, d = q.shape
    hk = k.shape[1]
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    imp = torch.empty((b, hk, n), dtype=torch.float32, device=q.device)
    L = _lib.lib()
    args = (q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), imp.data_ptr() if replay else None, b, h, hk,
            n, d, _lib.strides(q), _lib.strides(k), _lib.strides(v), _DTYPES[q.dtype],
            d ** -0.5 if scale is None else scale, 1, 1, int(replay), 0.0, n)

    def fn():
        _lib.check(L.fe_prefill(*args, torch.cuda.current_stream().cuda_stream), "fe_prefill")
    return fn


@torch.inference_mode()
def generic_rows(repeats, n=8192, hq=32, hk=8):
    """Attention (and attention with every row replayed) on the layouts and scales the fast
    kernels do not read in place: through prefill() (repacked K/V, zero scale on the fast
    kernels) and through the workspace-free entry point (the generic kernel), next to the fast
    path on ordinary layouts."""
    g = torch.Generator(device="cuda").manual_seed(SEED)

    def inputs(d):
        q = torch.randn((1, hq, n, d), device="cuda", generator=g, dtype=torch.bfloat16)
        k = torch.randn((1, hk, n, d), device="cuda", generator=g, dtype=torch.bfloat16)
        v = torch.randn((1, hk, n, d), device="cuda", generator=g, dtype=torch.bfloat16)
        return q, k, v

    def strided_q(d):
        q2 = torch.randn((1, hq, n, 2 * d), device="cuda", generator=g, dtype=torch.bfloat16)
        _, k, v = inputs(d)
        return q2[..., ::2], k, v                  # channel stride 2

    def offset_kv(d):
        q, _, _ = inputs(d)
        size = hk * n * d
        flat = torch.randn(2 * size + 1, device="cuda", generator=g, dtype=torch.bfloat16)
        k = flat[1:1 + size].view(1, hk, n, d)      # rows 2 bytes off 16-byte alignment
        v = flat[1 + size:1 + 2 * size].view(1, hk, n, d)
        return q, k, v

    # path "fast": prefill() on the fast kernels as laid out; "repacked": prefill() copies K/V the
    # fast kernels cannot read into its workspace first; "zero scale": fast kernels with Q zeroed
    # at load (with or without a workspace); "generic": the workspace-free entry point fe_prefill,
    # whose only kernel for these layouts is the generic one (nowhere to repack)
    cases = [("D=128", "fast", 128, lambda: inputs(128), None),
             ("D=64", "fast", 64, lambda: inputs(64), None),
             ("D=96", "fast", 96, lambda: inputs(96), None),
             ("D=32", "fast", 32, lambda: inputs(32), None),
             ("D=80", "fast", 80, lambda: inputs(80), None),
             ("D=192", "fast", 192, lambda: inputs(192), None),
             ("D=256", "fast", 256, lambda: inputs(256), None),
             ("D=100", "repacked", 100, lambda: inputs(100), None),
             ("D=100", "generic", 100, lambda: inputs(100), None),
             ("D=256 zero scale", "zero scale", 256, lambda: inputs(256), 0.0),
             ("D=128 negative scale", "fast", 128, lambda: inputs(128), -(128 ** -0.5)),
             ("D=128 zero scale", "zero scale", 128, lambda: inputs(128), 0.0),
             ("D=128 q channel stride 2", "fast", 128, lambda: strided_q(128), None),
             ("D=128 K/V rows misaligned", "repacked", 128, lambda: offset_kv(128), None),
             ("D=128 K/V rows misaligned", "generic", 128, lambda: offset_kv(128), None)]
    out = []
    for name, path, d, make, scale in cases:
        q, k, v = make()
        for replay in (False, True):
            if path == "generic":
                fn = _workspace_free(q, k, v, scale, replay)
            else:
                fn = (lambda: prefill(q, k, v, scale=scale, recency_decay=0.0)) if replay else \
                     (lambda: prefill(q, k, v, scale=scale, score=False))
            # ten warm-ups: the part runs the first launches of a fast-path case at a higher
            # clock than it holds once its power draw has built up
            ms = statistics.median(event_samples(fn, repeats, warmup=10))
            flop = _attention_flop(hq, n, d, replay)
            out.append({"case": name, "path": path, "work": "attention + full replay" if replay else "attention only",
                        "shape": "B1 Hq%d Hkv%d N%d D%d bf16 causal" % (hq, hk, n, d), "median_ms": ms,
                        "executed_tflop": flop / 1e12, "TFLOP/s": flop / (ms * 1e-3) / 1e12,
                        "frac_of_2.5PFLOP/s": flop / (ms * 1e-3) / 2.5e15})
            print(json.dumps(out[-1]), flush=True)
        del q, k, v
    return out


# ---------------------------------------------------------------- command line

def main(argv=None):
    p = argparse.ArgumentParser()
    p.add_argument("--lengths", type=int, nargs="+", default=[8192, 32768, 131072])
    p.add_argument("--heads", type=int, default=4)
    p.add_argument("--kv-heads", type=int, default=2)
    p.add_argument("--dim", type=int, default=64)
    p.add_argument("--repeats", type=int, default=5)
    p.add_argument("--methods", nargs="+", default=None, help="subset of the method names")
    p.add_argument("--output", default="benchmark.json")
    p.add_argument("--require-idle", action="store_true", help="refuse rows measured while another process holds the GPU")
    p.add_argument("--kernels", action="store_true", help="time the HBM-bound kernels on scaled synthetics")
    p.add_argument("--generic", action="store_true", help="prefill on the generic kernel's shapes and layouts")
    p.add_argument("--policies", action="store_true", help="policy latency at fixed budgets")
    p.add_argument("--budgets", type=int, nargs="+", default=[256, 1024])
    p.add_argument("--policy-file", default=None, help="JSON list of scoring policies (--policies)")
    args = p.parse_args(argv)

    if args.kernels or args.generic:
        data = {"gpu": torch.cuda.get_device_name(), "torch": torch.__version__, "hip": torch.version.hip,
                "rows": kernel_rows(args.repeats) if args.kernels else generic_rows(args.repeats)}
        Path(args.output).write_text(json.dumps(data, indent=2) + "\n")
        return

    torch.manual_seed(SEED)
    guard = ContentionGuard(args.require_idle)
    shape = (args.lengths, args.heads, args.kv_heads, args.dim)
    if args.policies:
        policies = json.loads(Path(args.policy_file).read_text()) if args.policy_file else DEFAULT_POLICIES
        run_args = {"lengths": args.lengths, "budgets": args.budgets, "repeats": args.repeats, "heads": args.heads,
                    "kv_heads": args.kv_heads, "dim": args.dim}
        report = Report(args.output, _header(args, dict(
            args=run_args, policies=policies,
            scope="one layer; incremental allocations, inputs excluded; output, scores, selection included")),
            resume_keys=("args", "policies"))
        run(report, *shape, lambda q, k, v, n: policy_cases(q, k, v, n, args.budgets, policies), args.repeats, guard)
        expected = len(args.lengths) * (2 + len(args.budgets) * (2 + len(policies)))
        report.data["complete"] = len(report.done) == expected
        report.save()
        return

    report = Report(args.output, _header(args, dict(
        args=vars(args), rocm_smi_before=_tool_output(["rocm-smi"]),
        scope="single attention layer; allocations include output and selection, exclude inputs")))
    run(report, *shape, lambda q, k, v, n: layer_cases(q, k, v, n, args.methods), args.repeats, guard)


if __name__ == "__main__":
    main()
