"""Host-side pieces of the benchmark harness (no GPU): the process-query parser of the
contention guard and the refusal rule of --require-idle."""
import os

import pytest

from flash_evict import benchmark


def test_parse_amd_smi_process_json():
    text = ('[{"gpu": 0, "process_list": [{"process_info": {"name": "python3", "pid": 4242, '
            '"memory_usage": {"vram_mem": {"value": 1, "unit": "B"}}}}, '
            '{"process_info": {"name": "other", "pid": "77"}}]}, {"gpu": 1, "process_list": []}]')
    assert benchmark.parse_gpu_pids(text) == [77, 4242]


def test_parse_rocm_smi_showpids_json_and_tables():
    assert benchmark.parse_gpu_pids('{"system": {"PID1234": "python3, 1, 0, 0, 0", "PID99": "x, 1, 0, 0, 0"}}') \
        == [99, 1234]
    table = "PID   PROCESS NAME  GPU(s)  VRAM USED\n5150  python3       1       1024\n"
    assert benchmark.parse_gpu_pids(table) == [5150]
    assert benchmark.parse_gpu_pids('{"system": {}}') == []
    assert benchmark.parse_gpu_pids("No KFD PIDs currently running") == []


def test_guard_refuses_only_when_required():
    g = benchmark.ContentionGuard.__new__(benchmark.ContentionGuard)
    g.query = None
    g.require_idle = False
    g.check([123], "preceded")                  # recorded, not refused
    g.require_idle = True
    g.check([], "preceded")
    with pytest.raises(RuntimeError, match="uncontended"):
        g.check([123], "overlapped")
    raw, others = g.snapshot()
    assert raw.startswith("unavailable") and others == []
    assert os.getpid() > 0
