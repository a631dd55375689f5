"""bench.py's host-side parts on the CPU: the CPU baseline (the oracle timed
on a bounded sample and extrapolated, one thread and all cores) on the small
Tied workload, the GPU-count guard, and the algorithmic work the roofline
fractions divide by."""
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


def test_algorithmic_work_per_step():
    """The flops and bytes the bench's roofline fractions divide by, restated
    per workload from the shapes: each GEMM 2·rows·V·H flops (Tied with
    teacher CE: student and teacher rows), the row pass's logits read and
    gradients written plus the statistics entries it reads."""
    w = bench.work_per_step(bench.WORKLOADS["tied-8192x4096x131072-bf16-int8"], None)
    bt, h, v, nst = 8192, 4096, 131072, 512
    assert w["gemm_logits"] == ("mfma", 2 * (2 * bt) * h * v)
    assert w["gemm_grad_hidden"] == w["gemm_grad_weight"] == ("mfma", 2 * (2 * bt) * v * h)
    # bf16 rows of both logits read, both gradients written; per row pair the
    # two rows' tile statistics, the pair's two KL sums, the label logits,
    # both rows' half-tile maxima
    assert w["row_pass"] == ("hbm", 2 * bt * v * 2 + 2 * bt * v * 2 +
                             bt * (2 * nst * 16 + nst * 8 + 8) + bt * nst * 8 * 2)
    assert w["quant"] == ("hbm", v * h * 8)
    # bf16 inputs beside fp32 Precomputed logits: the student's bf16 row and
    # the teacher's fp32 row read, the student's gradient written; the
    # teacher's statistics per 256-column tile (from the GEMM), the KL sums,
    # the student's half-tile maxima
    w = bench.work_per_step(bench.WORKLOADS["precomputed-4096x4096x65536-bf16"], None)
    bt, h, v, nst = 4096, 4096, 65536, 256
    assert w["gemm_logits"] == ("mfma", 2 * bt * h * v)
    assert w["row_pass"] == ("hbm", bt * v * (2 + 4) + bt * v * 2 +
                             bt * (2 * nst * 16 + nst * 8 + 8) + bt * nst * 8)
    # fp32 Precomputed: both fp32 rows read, the student's fp32 gradient
    # written; the teacher's statistics per 8192-column segment
    w = bench.work_per_step(bench.WORKLOADS["precomputed-4096x4096x65536-f32"], None)
    assert w["row_pass"] == ("hbm", 2 * bt * v * 4 + bt * v * 4 + bt * (nst * 16 + 8 * 16 + 8))
