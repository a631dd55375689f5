"""Run-to-run determinism of the GPU path: the same call gives bitwise the
same outputs every time, on the same context (workspace reused) and on a new
one. Nothing in the library sums in an order that depends on timing: the
split-K partials are reduced in split order, and the row statistics, row
losses and per-chunk sums are reduced in fixed orders, with no
floating-point atomics.

The cases reach the paths whose reductions could differ: split K in both
backward GEMMs (small shapes), grad_hidden in shared raster rounds with a
grouped tail, grad_hidden as one whole round plus a tail of rows with K
split, the paired bf16 row pass with INT8 grad_W (deterministic and
stochastic rounding), several staging groups accumulating into grad_W, a
Separate teacher (bf16: its fp32 logits read in the student logits GEMM's
epilogue), Precomputed logits through the chunked fp32 row pass and beside
bf16 inputs (read in the epilogue), and the fp32 inputs under Profile.Fast.
"""
import numpy as np
import pytest

from helpers import normal, uniform_labels

import orda_hip as H
from orda_hip import ChunkSize, KernelConfig, LossOptions, Profile, Teacher

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    assert H.is_available(), "liborda_hip.so does not see a gfx950 device"
    return torch, torch.device("cuda:0")


CASES = {
    # name: (mode, dtype, bt, h, ht, v, weight scale, options)
    "tied-bf16-int8": ("tied", "bf16", 1024, 512, 512, 30000, 0.04,
                       dict(kd_weight=0.4, temperature=1.5, label_smoothing=0.1,
                            config=KernelConfig(quantize_grad_weight=True))),
    "tied-bf16-int8-stochastic-groups": (
        "tied", "bf16", 1024, 256, 256, 20000, 0.05,
        dict(kd_weight=0.4, temperature=2.0, chunk_size=ChunkSize.Fixed(128),
             config=KernelConfig(quantize_grad_weight=True, stochastic_rounding=True,
                                 stochastic_seed=7))),
    "tied-f32-split-k": ("tied", "f32", 256, 512, 512, 8192, 0.04,
                         dict(kd_weight=0.4, temperature=1.5)),
    "tied-bf16-shared-rounds": ("tied", "bf16", 8492, 800, 800, 301, 0.04,
                                dict(kd_weight=0.5, temperature=1.5, label_smoothing=0.1)),
    # grad_hidden: 20 x 16 tiles, one whole round of 256 and a tail of rows
    # 4096-4999 with K split
    "tied-bf16-tail-split": ("tied", "bf16", 5000, 4096, 4096, 1024, 0.04,
                             dict(kd_weight=0.4, temperature=1.5)),
    "separate-bf16": ("separate", "bf16", 500, 256, 384, 20000, 0.05,
                      dict(kd_weight=0.5, temperature=2.0, teacher_ce_weight=0.3)),
    "precomputed-f32-chunked": ("precomputed", "f32", 300, 64, 0, 120000, 0.1,
                                dict(kd_weight=0.7, temperature=1.5)),
    "precomputed-bf16-epilogue": ("precomputed", "bf16", 700, 256, 0, 30000, 0.05,
                                  dict(kd_weight=0.7, temperature=1.5, label_smoothing=0.1,
                                       chunk_size=ChunkSize.Fixed(256))),
    "tied-f32-fast": ("tied", "f32", 512, 384, 384, 16000, 0.05,
                      dict(kd_weight=0.4, temperature=1.5,
                           config=KernelConfig.from_profile(Profile.Fast))),
}


def _inputs(torch, dev, mode, dtype, bt, h, ht, v, wscale):
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(tdt)
    s = t(normal((bt, h), 61))
    w = t(normal((v, h), 62, wscale))
    y = uniform_labels(bt, v, 63)
    y[::7] = -100
    y = torch.from_numpy(y).to(dev)
    if mode == "tied":
        teacher = Teacher.Tied(t(normal((bt, h), 64)))
    elif mode == "separate":
        teacher = Teacher.Separate(t(normal((bt, ht), 64)), t(normal((v, ht), 65, wscale)))
    else:   # fp32 logits beside either input dtype
        teacher = Teacher.Precomputed(torch.from_numpy(normal((bt, v), 64, 2.0)).to(dev))
    return s, w, y, teacher


def _outputs(out):
    """Every output of one call, as (name, value) pairs."""
    items = [("loss", out.loss), ("student_ce", out.student_ce), ("teacher_ce", out.teacher_ce),
             ("kl", out.kl), ("chunk_plan", (out.chunk_plan.chunk_size, out.chunk_plan.num_chunks))]
    for name in ("grad_student_hidden", "grad_weight", "grad_teacher_hidden", "grad_teacher_weight",
                 "row_nll_student", "row_nll_teacher", "row_kl", "quant_codes", "quant_scales"):
        items.append((name, getattr(out, name)))
    return items


@pytest.mark.parametrize("name", sorted(CASES))
def test_same_call_same_bits(torch_dev, name):
    torch, dev = torch_dev
    mode, dtype, bt, h, ht, v, wscale, kw = CASES[name]
    s, w, y, teacher = _inputs(torch, dev, mode, dtype, bt, h, ht, v, wscale)
    opts = LossOptions(**kw)
    quant = opts.config.quantize_grad_weight
    ctx = H.Context(0)
    runs = [H.distillation_loss(s, w, y, teacher, opts, ctx=ctx, rows=True, quant_codes=quant)
            for _ in range(2)]
    ctx.close()
    fresh = H.Context(0)
    runs.append(H.distillation_loss(s, w, y, teacher, opts, ctx=fresh, rows=True,
                                    quant_codes=quant))
    fresh.close()
    first = _outputs(runs[0])
    for k, other in enumerate(runs[1:], 1):
        for (name_a, a), (_, b) in zip(first, _outputs(other)):
            if a is None or b is None:
                assert a is None and b is None, (name, name_a, k)
            elif isinstance(a, torch.Tensor):
                assert torch.equal(a, b), f"{name}: {name_a} differs on run {k}"
            else:
                assert a == b, f"{name}: {name_a} differs on run {k}: {a} != {b}"
