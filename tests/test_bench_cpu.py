"""bench.py's host-side parts on the CPU: the CPU baseline (the oracle timed
on a bounded sample and extrapolated, one thread and all cores) on the small
Tied workload, and the GPU-count guard."""
import os
import subprocess
import sys

import bench


def test_cpu_baseline_fields(monkeypatch):
    monkeypatch.setenv("OMP_NUM_THREADS", "2")
    r = bench.cpu_baseline(bench.WORKLOADS["tied-256x512x8192-f32"])
    assert r["kind"] == "port" and r["cores"] == 1 and r["unit"] == "rows/s"
    assert r["value"] > 0 and "one chunk of 2, 4, 6 rows" in r["sample"]
    model, cores = bench.cpu_info()
    assert r["cpu"] == model and r["host_cores"] == cores
    if cores > 1:
        a = r["all_cores"]
        assert a["cores"] == 2 and a["value"] > 0 and a["unit"] == "rows/s"


def test_more_than_one_gpu_is_refused():
    p = subprocess.run([sys.executable, os.path.join(bench.ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert p.returncode != 0
    assert "one GPU" in (p.stdout + p.stderr)
