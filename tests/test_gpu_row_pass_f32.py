"""GPU parity of the chunked row pass over fp32 logits, against the oracle.

Groups of at least 20·2^20 logits per logits block (rows x V) take the
three-launch fp32 row pass: per-row constants, the gradient over (row,
256-column) blocks with each block's share of the row's KL sums, then each
row's KL from those shares. These cases sit just above that size with a small
hidden width, so that the oracle's products stay cheap (run on the host's
cores; results bitwise the same as one thread):
* V not a multiple of the 256-column block, labels forced into the last,
  partial block and into the first column, every 7th row ignored;
* every teacher mode: Tied (teacher CE gradient in place), Separate (own
  teacher weight), Precomputed logits read in place, also at a pitch wider
  than V;
* bf16 inputs whose KL term needs fp32 logits (Separate, Precomputed): the
  gradient rows then go to a separate bf16 buffer;
* two staging groups in one call, which reuse the per-block KL buffer.
Tolerances as in tests/parity.py (loss terms 1e-4 relative; gradients 1e-3
for fp32 inputs, 2e-2 for bf16 inputs with the oracle fed the rounded values).
"""
import os

import numpy as np
import pytest

import oracle as O
from helpers import bf16_round, normal, uniform_labels
from parity import check_output

import orda_hip as H
from orda_hip import LossOptions, Teacher

pytestmark = pytest.mark.gpu

BLOCK = 256            # columns per gradient block of the fp32 pass
THRESHOLD = 20 << 20   # rows x V from which the fp32 pass is chunked


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    assert H.is_available(), "liborda_hip.so does not see a gfx950 device"
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    O.set_threads(threads)
    yield torch, torch.device("cuda:0")
    O.set_threads(1)


def edge_labels(bt, v, seed, ignore_every=7):
    y = uniform_labels(bt, v, seed)
    last0 = (v - 1) // BLOCK * BLOCK          # first column of the partial block
    y[1::11] = last0 + (np.arange(len(y[1::11])) % (v - last0))
    y[2::13] = 0
    y[::ignore_every] = -100
    return y


CASES = {
    # name: (mode, dtype, bt, h, ht, v, options)
    "tied-f32": ("tied", "f32", 320, 16, 16, 110000,
                 dict(kd_weight=0.5, temperature=1.5, label_smoothing=0.1, teacher_ce_weight=0.7)),
    "separate-f32": ("separate", "f32", 300, 24, 40, 120000,
                     dict(kd_weight=0.5, temperature=2.0, label_smoothing=0.1,
                          teacher_ce_weight=1.0)),
    "separate-bf16": ("separate", "bf16", 300, 24, 40, 120000,
                      dict(kd_weight=0.5, temperature=2.0, label_smoothing=0.0,
                           teacher_ce_weight=1.0)),
    "precomputed-f32": ("precomputed", "f32", 256, 32, 0, 131072,
                        dict(kd_weight=0.7, temperature=1.0)),
    "precomputed-f32-wide-pitch": ("precomputed", "f32", 256, 32, 0, 131072,
                                   dict(kd_weight=0.7, temperature=1.5, label_smoothing=0.1)),
    "precomputed-bf16": ("precomputed", "bf16", 264, 24, 0, 130000,
                         dict(kd_weight=0.4, temperature=1.5)),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_f32_row_pass_against_oracle(torch_dev, name):
    torch, dev = torch_dev
    mode, dtype, bt, h, ht, v, kw = CASES[name]
    assert bt * v >= THRESHOLD
    s = normal((bt, h), 1)
    w = normal((v, h), 2, 0.2)
    y = edge_labels(bt, v, 3)
    opts = LossOptions(student_ce_weight=1.0, **kw)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    if dtype == "bf16":
        s, w = bf16_round(s), bf16_round(w)

    def dev_t(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(tdt)

    if mode == "tied":
        th = normal((bt, h), 4)
        if dtype == "bf16":
            th = bf16_round(th)
        t_ref, t_gpu = Teacher.Tied(th), Teacher.Tied(dev_t(th))
    elif mode == "separate":
        th, tw = normal((bt, ht), 4), normal((v, ht), 5, 0.15)
        if dtype == "bf16":
            th, tw = bf16_round(th), bf16_round(tw)
        t_ref, t_gpu = Teacher.Separate(th, tw), Teacher.Separate(dev_t(th), dev_t(tw))
    else:
        tl = normal((bt, v), 6, 2.0)
        tl[np.arange(bt), np.clip(y, 0, v - 1)] += 8.0
        t_ref = Teacher.Precomputed(tl)
        if name.endswith("wide-pitch"):
            wide = torch.zeros((bt, v + 24), device=dev, dtype=torch.float32)
            wide[:, :v] = torch.from_numpy(tl).to(dev)
            t_gpu = Teacher.Precomputed(wide[:, :v])
        else:
            t_gpu = Teacher.Precomputed(torch.from_numpy(tl).to(dev))
    got = H.distillation_loss(dev_t(s), dev_t(w), torch.from_numpy(y).to(dev), t_gpu, opts)
    ref = O.distillation_loss(s, w, y, t_ref, opts)
    check_output(got, ref, kind="bf16" if dtype == "bf16" else "f32")


@pytest.mark.parametrize("teacher_ce", [True, False])
def test_f32_row_pass_two_staging_groups(torch_dev, teacher_ce):
    """Two staging groups of 256 rows (256 x 131072 logits per block, the
    chunked fp32 pass in each): the per-block KL shares are reused from one
    group to the next, and every row's KL, NLLs and gradients must still
    match the oracle's, with the reference's per-chunk KL rounding."""
    torch, dev = torch_dev
    bt, h, v = 512, 16, 131072
    s, th = normal((bt, h), 11), normal((bt, h), 12)
    w = normal((v, h), 13, 0.2)
    y = edge_labels(bt, v, 14, ignore_every=5)
    opts = LossOptions(kd_weight=0.6, temperature=1.5, label_smoothing=0.1,
                       teacher_ce_weight=0.5 if teacher_ce else 0.0,
                       chunk_size=H.ChunkSize.Fixed(256))
    ctx = H.Context(0)
    ctx.set_staging_budget(1)   # one chunk per group
    ctx.set_timing(True)
    dt = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    got = H.distillation_loss(dt(s), dt(w), dt(y), Teacher.Tied(dt(th)), opts, ctx=ctx)
    _, n = ctx.kernel_time("gemm_logits")
    assert n == 2, f"expected two logits launches (two groups), got {n}"
    ref = O.distillation_loss(s, w, y, Teacher.Tied(th), opts)
    check_output(got, ref)
    ctx.close()
