"""GPU parity of GEMM launch paths that the other cases reach only at large
shapes, against the oracle:

* grad_W as whole rounds plus a tail with K split (a Store/Accum product
  whose last round would hold fewer than 192 workgroups runs its whole
  rounds in one launch and the remaining columns as a second product that
  splits K): H = 64 gives grad_W one M-tile and V = 76900 301 column tiles,
  one whole round and a 45-tile tail; two staging groups of 256 rows make the
  second group's grad_W accumulate (the Accum epilogue through both launches
  and the split reduction), with K = 512 per group.

* grad_hidden in shared raster rounds at 12 N-tiles (H = 3072: blocks of
  5 M x 6 N tiles per XCD, bands of 20 M-tiles) with a grouped tail: BT =
  2860 gives 24 M-tiles over the student and teacher problems, one band and
  4 M-tiles after it.

* grad_hidden as whole rounds over its first rows plus a tail of rows with
  K split: H = 512 (2 N-tiles) and BT = 17000 give 67 M-tiles per problem,
  268 tiles over student and teacher rows, one round over the first 16384
  rows and a 12-tile tail (V = 320: K split in two).

fp32 (the oracle's tolerance 1e-3 on gradients) and bf16 inputs (2e-2, the
oracle fed the same bf16-rounded values).
"""
import os

import numpy as np
import pytest

import oracle as O
from helpers import bf16_round, normal, uniform_labels
from parity import check_output

import orda_hip as H
from orda_hip import ChunkSize, LossOptions, Teacher

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    assert H.is_available(), "liborda_hip.so does not see a gfx950 device"
    O.set_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    yield torch, torch.device("cuda:0")
    O.set_threads(1)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_grad_w_tail_split_accumulated_over_groups(torch_dev, dtype):
    torch, dev = torch_dev
    bt, h, v = 512, 64, 76900
    s, th = normal((bt, h), 81), normal((bt, h), 82)
    w = normal((v, h), 83, 0.15)
    y = uniform_labels(bt, v, 84)
    y[::9] = -100
    if dtype == "bf16":
        s, th, w = bf16_round(s), bf16_round(th), bf16_round(w)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    dt = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(tdt)
    opts = LossOptions(kd_weight=0.5, temperature=1.5, label_smoothing=0.1,
                       chunk_size=ChunkSize.Fixed(256))
    ctx = H.Context(0)
    ctx.set_staging_budget(1)   # one chunk per group: two groups
    ctx.set_timing(True)
    got = H.distillation_loss(dt(s), dt(w), torch.from_numpy(y).to(dev), Teacher.Tied(dt(th)),
                              opts, ctx=ctx)
    _, n = ctx.kernel_time("gemm_logits")
    ctx.close()
    assert n == 2, f"expected two staging groups, got {n} logits launches"
    ref = O.distillation_loss(s, w, y, Teacher.Tied(th), opts)
    check_output(got, ref, kind=dtype)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_grad_hidden_shared_rounds_twelve_column_tiles(torch_dev, dtype):
    torch, dev = torch_dev
    bt, h, v = 2860, 3072, 301
    s, th = normal((bt, h), 91), normal((bt, h), 92)
    w = normal((v, h), 93, 0.02)   # logits spread ~1.1
    y = uniform_labels(bt, v, 94)
    y[::8] = -100
    if dtype == "bf16":
        s, th, w = bf16_round(s), bf16_round(th), bf16_round(w)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    dt = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(tdt)
    opts = LossOptions(kd_weight=0.4, temperature=1.5, label_smoothing=0.1)
    got = H.distillation_loss(dt(s), dt(w), torch.from_numpy(y).to(dev), Teacher.Tied(dt(th)), opts)
    ref = O.distillation_loss(s, w, y, Teacher.Tied(th), opts)
    check_output(got, ref, kind=dtype)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_grad_hidden_tail_rows_split(torch_dev, dtype):
    torch, dev = torch_dev
    bt, h, v = 17000, 512, 320
    s, th = normal((bt, h), 101), normal((bt, h), 102)
    w = normal((v, h), 103, 0.05)
    y = uniform_labels(bt, v, 104)
    y[::10] = -100
    if dtype == "bf16":
        s, th, w = bf16_round(s), bf16_round(th), bf16_round(w)
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    dt = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(tdt)
    opts = LossOptions(kd_weight=0.4, temperature=2.0, label_smoothing=0.1,
                       chunk_size=ChunkSize.Fixed(bt))
    got = H.distillation_loss(dt(s), dt(w), torch.from_numpy(y).to(dev), Teacher.Tied(dt(th)), opts)
    ref = O.distillation_loss(s, w, y, Teacher.Tied(th), opts)
    check_output(got, ref, kind=dtype)
