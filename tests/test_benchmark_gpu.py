"""The benchmark harness (flash_evict.benchmark, the protocol of the reference's
scripts/benchmark.py:18-126) on a tiny problem: every method runs, rows carry the
reference's fields, and the kernel resource dump is attached."""
import json

import pytest

from flash_evict import benchmark

pytestmark = pytest.mark.gpu

FIELDS = {"n", "method", "budget", "median_ms", "samples_ms", "allocated_before_bytes", "peak_allocated_bytes",
          "peak_increment_bytes", "peak_reserved_bytes", "free_device_bytes_before", "total_device_bytes"}


def test_harness_runs_every_method(tmp_path):
    out = tmp_path / "bench.json"
    benchmark.main(["--lengths", "256", "300", "--heads", "4", "--kv-heads", "2", "--dim", "64",
                    "--repeats", "2", "--output", str(out)])
    report = json.loads(out.read_text())
    rows = report["rows"]
    names = {"torch_flash", "hip_attention_only", "fused_replay_scores", "fused_replay_topk", "flash_snap_w32",
             "flash_snap_w128", "gather_kv"}
    assert {(r["n"], r["method"]) for r in rows} == {(n, m) for n in (256, 300) for m in names}
    for r in rows:
        assert FIELDS <= set(r), r
        assert len(r["samples_ms"]) == 2 and r["median_ms"] > 0
        assert r["budget"] == (26 if r["n"] == 256 else 30)
    kernels = {e["kernel"] for e in report["kernel_resources"]}
    assert any(k.startswith("fused_fast") for k in kernels) and "gather_rows16_kernel" in kernels


def test_kernel_mode(tmp_path):
    out = tmp_path / "k.json"
    benchmark.main(["--kernels", "--repeats", "2", "--output", str(out)])
    rows = json.loads(out.read_text())["rows"]
    assert [r["kernel"] for r in rows] == ["zero_f32", "select (top-k + mask + indices)", "select 8 x 32768",
                                          "select 256 x 32768", "select with pool 5", "gather_tokens"]
    assert all(r["median_ms"] > 0 and r["GB/s"] > 0 for r in rows)


def test_policy_mode_resumes(tmp_path):
    out = tmp_path / "p.json"
    argv = ["--policies", "--lengths", "256", "--budgets", "64", "128", "--heads", "4", "--kv-heads", "2",
            "--dim", "64", "--repeats", "2", "--output", str(out)]
    benchmark.main(argv)
    report = json.loads(out.read_text())
    rows = report["rows"]
    expected = {("torch_flash", None), ("hip_attention_only", None)}
    expected |= {(m, b) for b in (64, 128) for m in ["snap_w32", "snap_w128"] + [p["name"] for p in
                                                                               benchmark.DEFAULT_POLICIES]}
    assert {(r["method"], r["budget"]) for r in rows} == expected
    assert report["complete"] and all(FIELDS <= set(r) for r in rows)
    benchmark.main(argv)   # resumes: nothing left to measure
    assert len(json.loads(out.read_text())["rows"]) == len(rows)
