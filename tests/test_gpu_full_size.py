"""Parity at the full benchmark shape: Tied teacher, BT=8192, H=4096,
V=131072, bf16 inputs, kd 0.4, T 1.5, label smoothing 0.1, INT8 grad_W
(Auto plan: 16 chunks x 512 rows), every 13th label ignored.

The CPU oracle cannot run this shape in test time, so the reference is the
row-chunked float32/float64 torch restatement (tests/torch_reference.py,
pinned to the oracle at small sizes on the CPU) run on the same GPU.
Tolerances as in tests/parity.py (loss terms 1e-4, bf16 gradients 2e-2).
Size-independent properties of the INT8 result are checked besides: codes
within ±127, every non-target row reaching ±127 at its largest element, and
non-target rows of the returned grad_W equal to code x scale exactly. The
INT8 step itself is pinned end to end: the same call with quantization off
gives the fp32 grad_W that the quantized call quantized, and quantizing it
with orda_quant_rows_int8 (bit-exact against the oracle's quantizer) must
give identical codes, scales and dequantized rows (src/api.rs:380-399).

Also at full shape against the same restatement: the three fp32 workloads
(Tied 2048x4096x32000, Separate 4096x(2048, 4096)x32000, Precomputed
4096x4096x65536), and the Separate and Precomputed shapes with bf16 inputs.
"""
import pytest

from parity import (check_grad_device, check_quant_of_own_gradient,
                    check_quantized_vs_reference_device, check_scalar)
from torch_reference import loss_tied_chunked

import orda_hip as H
from orda_hip import KernelConfig, LossOptions, Teacher

pytestmark = pytest.mark.gpu


def test_tied_bf16_int8_full_benchmark_shape():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    assert H.is_available(), "liborda_hip.so does not see a gfx950 device"
    torch.backends.cuda.matmul.allow_tf32 = False
    dev = torch.device("cuda:0")
    bt, h, v = 8192, 4096, 131072
    g = torch.Generator(device=dev)
    g.manual_seed(20261201)
    hs = torch.randn(bt, h, generator=g, device=dev).to(torch.bfloat16)
    ht = torch.randn(bt, h, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(v, h, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    y = torch.randint(0, v, (bt,), generator=g, device=dev)
    y[::13] = -100
    opts = LossOptions(kd_weight=0.4, temperature=1.5, label_smoothing=0.1,
                       config=KernelConfig(quantize_grad_weight=True))
    got = H.distillation_loss(hs, w, y, Teacher.Tied(ht), opts, quant_codes=True)
    assert (got.chunk_plan.chunk_size, got.chunk_plan.num_chunks) == (512, 16)

    ref = loss_tied_chunked(hs, ht, w, y, kd=0.4, T=1.5, alpha=0.1)
    rel = {}
    for k in ("loss", "student_ce", "teacher_ce", "kl"):
        check_scalar(k, getattr(got, k), ref[k])
        rel[k] = abs(getattr(got, k) - ref[k]) / abs(ref[k])
    rel["grad_student_hidden"] = check_grad_device(
        "grad_student_hidden", got.grad_student_hidden, ref["grad_student_hidden"], "bf16")
    rel["grad_teacher_hidden"] = check_grad_device(
        "grad_teacher_hidden", got.grad_teacher_hidden, ref["grad_teacher_hidden"], "bf16")
    rel["grad_weight"] = check_grad_device("grad_weight (dequantized)", got.grad_weight,
                                           ref["grad_weight"], "bf16")
    print("relative errors:", {k: f"{e:.2e}" for k, e in rel.items()})
    del ref

    codes, scales = got.quant_codes, got.quant_scales.reshape(-1)
    target = torch.zeros(v, dtype=torch.bool, device=dev)
    target[y[y != -100]] = True
    other = ~target
    assert int(codes.abs().max()) <= 127
    assert bool((codes[other].abs().amax(1) == 127).all())
    assert torch.equal(got.grad_weight[other], codes[other].float() * scales[other, None])

    print("quantization off: same call", flush=True)
    plain_opts = LossOptions(kd_weight=0.4, temperature=1.5, label_smoothing=0.1)
    plain = H.distillation_loss(hs, w, y, Teacher.Tied(ht), plain_opts)
    check_quant_of_own_gradient(
        got, plain.grad_weight, y,
        quant=lambda m, t: H.quant_rows_int8(m, t, -100, False, 0))


FP32_WORKLOADS = ["tied-2048x4096x32000-f32", "separate-4096x2048x4096x32000-f32",
                  "precomputed-4096x4096x65536-f32"]


@pytest.mark.parametrize("name", FP32_WORKLOADS)
def test_fp32_workloads_full_shape(name):
    """The fp32 workloads at their full shapes, on bench.py's own inputs (its
    seeded generator), every 17th label ignored, against loss_chunked run on
    the same GPU: loss terms to 1e-4, fp32 gradients to 1e-3."""
    import torch
    import bench
    from torch_reference import loss_chunked
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    assert H.is_available(), "liborda_hip.so does not see a gfx950 device"
    torch.backends.cuda.matmul.allow_tf32 = False
    wl = bench.WORKLOADS[name]
    mode, bt, h, ht, v, dt, kd, T, alpha, w_t, _ = wl
    dev = torch.device("cuda:0")
    s, w, y, t = bench.make_inputs(torch, wl, dev, seed=7)
    y[::17] = -100
    opts = bench.options(H, wl)
    print(f"case {name}", flush=True)
    got = H.distillation_loss(s, w, y, bench.teacher_obj(H, t), opts)
    th = t[1] if mode in ("tied", "separate") else None
    tw = t[2] if mode == "separate" else None
    tl = t[1] if mode == "precomputed" else None
    ref = loss_chunked(s, w, y, mode, th, tw, tl, kd=kd, T=T, alpha=alpha,
                       w_t=opts.teacher_ce_weight)
    rel = {}
    for k in ("loss", "student_ce", "teacher_ce", "kl"):
        check_scalar(k, getattr(got, k), ref[k])
        rel[k] = abs(getattr(got, k) - ref[k]) / max(abs(ref[k]), 1e-2)
    for k in ("grad_student_hidden", "grad_weight", "grad_teacher_hidden", "grad_teacher_weight"):
        g, r = getattr(got, k), ref[k]
        assert (g is None) == (r is None), f"{k}: presence differs"
        if r is not None:
            rel[k] = check_grad_device(k, g, r, "f32")
    print("relative errors:", {k: f"{e:.2e}" for k, e in rel.items()})
    if mode == "tied":
        # The INT8 clause of the gate at this fp32 shape: the quantized call
        # quantizes its own fp32 grad_W exactly, and its codes and scales
        # meet the gate against the reference's fp32 grad_W quantized by
        # orda_quant_rows_int8 (bit-exact against the oracle's quantizer).
        import dataclasses
        qopts = dataclasses.replace(opts, config=dataclasses.replace(opts.config,
                                                                      quantize_grad_weight=True))
        print("quantized call", flush=True)
        q = H.distillation_loss(s, w, y, bench.teacher_obj(H, t), qopts, quant_codes=True)

        def quant(m, tg):
            return H.quant_rows_int8(m, tg, -100, False, 0)
        check_quant_of_own_gradient(q, got.grad_weight, y, quant=quant)
        _, rq, rs = quant(ref["grad_weight"], y)
        flips = check_quantized_vs_reference_device(q, got.grad_weight, ref["grad_weight"], rq, rs)
        print(f"INT8 codes differing at rounding boundaries: {flips} of {v * h}")


@pytest.mark.parametrize("name", ["separate-4096x2048x4096x32000-bf16",
                                  "precomputed-4096x4096x65536-bf16"])
def test_bf16_inputs_beside_fp32_teacher_logits_full_shape(name):
    """The Separate and Precomputed workloads' full shapes with bf16 hidden
    rows and weights (Precomputed logits stay fp32): the student's logits
    GEMM reads the teacher's fp32 logits in its epilogue (a Separate
    teacher's from its own GEMM, with teacher CE and its gradient), the
    student logits are stored in bf16. Against loss_chunked on the same
    bf16-rounded values on the same GPU: loss terms to 1e-4, bf16 gradients
    to 2e-2."""
    import torch
    import bench
    from torch_reference import loss_chunked
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    assert H.is_available(), "liborda_hip.so does not see a gfx950 device"
    torch.backends.cuda.matmul.allow_tf32 = False
    wl = bench.WORKLOADS[name]
    mode, bt, h, ht, v, dt, kd, T, alpha, w_t, _ = wl
    assert dt == "bf16"
    dev = torch.device("cuda:0")
    s, w, y, t = bench.make_inputs(torch, wl, dev, seed=11)
    y[::17] = -100
    opts = bench.options(H, wl)
    print(f"case {name}", flush=True)
    got = H.distillation_loss(s, w, y, bench.teacher_obj(H, t), opts)
    th = t[1] if mode == "separate" else None
    tw = t[2] if mode == "separate" else None
    tl = t[1] if mode == "precomputed" else None
    ref = loss_chunked(s, w, y, mode, th, tw, tl, kd=kd, T=T, alpha=alpha,
                       w_t=opts.teacher_ce_weight)
    rel = {}
    for k in ("loss", "student_ce", "teacher_ce", "kl"):
        check_scalar(k, getattr(got, k), ref[k])
        rel[k] = abs(getattr(got, k) - ref[k]) / max(abs(ref[k]), 1e-2)
    for k in ("grad_student_hidden", "grad_weight", "grad_teacher_hidden", "grad_teacher_weight"):
        g, r = getattr(got, k), ref[k]
        assert (g is None) == (r is None), f"{k}: presence differs"
        if r is not None:
            rel[k] = check_grad_device(k, g, r, "bf16")
    print("relative errors:", {k: f"{e:.2e}" for k, e in rel.items()})


WIDE = [("tied", "bf16", 1024, 8192, 8192, 50257), ("tied", "bf16", 1024, 16384, 16384, 50257),
        ("separate", "bf16", 1024, 8192, 16384, 50257), ("tied", "f32", 1024, 8192, 8192, 50257),
        ("tied", "bf16", 6400, 8192, 8192, 16000)]


@pytest.mark.parametrize("case", WIDE, ids=[f"{m}-{d}-bt{bt}-h{h}-ht{ht}-v{v}"
                                            for m, d, bt, h, ht, v in WIDE])
def test_wide_hidden(case):
    """Model widths of the largest decoders (H = 8192 and 16384; a Separate
    teacher twice the student's width) at a ragged V, kd 0.5, T 2, label
    smoothing 0.1, teacher CE, every 13th label ignored: the logits GEMM's K,
    grad_hidden's N and grad_W's N at their widest, against loss_chunked on
    the same (bf16-rounded) values on the same GPU; loss terms to 1e-4,
    gradients to the input dtype's gate. The last shape puts 50 M-tiles of
    8192-wide bf16 student and teacher rows (200 MB) into the logits GEMM,
    which then walks them in a band of 32 M-tiles and the 18 M-tiles past it
    in the grouped raster."""
    import torch
    from torch_reference import loss_chunked
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    assert H.is_available(), "liborda_hip.so does not see a gfx950 device"
    torch.backends.cuda.matmul.allow_tf32 = False
    mode, dt, bt, h, ht, v = case
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(h + ht)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32
    s = torch.randn(bt, h, generator=g, device=dev).to(tdt)
    w = (torch.randn(v, h, generator=g, device=dev) * (0.5 / h ** 0.5)).to(tdt)
    th = torch.randn(bt, ht, generator=g, device=dev).to(tdt)
    tw = (torch.randn(v, ht, generator=g, device=dev) * (0.5 / ht ** 0.5)).to(tdt) \
        if mode == "separate" else None
    y = torch.randint(0, v, (bt,), generator=g, device=dev)
    y[::13] = -100
    opts = LossOptions(kd_weight=0.5, temperature=2.0, label_smoothing=0.1, teacher_ce_weight=1.0)
    teacher = Teacher.Tied(th) if mode == "tied" else Teacher.Separate(th, tw)
    print(f"case {mode}-{dt}-bt{bt}-h{h}-ht{ht}-v{v}", flush=True)
    got = H.distillation_loss(s, w, y, teacher, opts)
    ref = loss_chunked(s, w, y, mode, th, tw, None, kd=0.5, T=2.0, alpha=0.1, w_t=1.0)
    for k in ("loss", "student_ce", "teacher_ce", "kl"):
        check_scalar(k, getattr(got, k), ref[k])
    for k in ("grad_student_hidden", "grad_weight", "grad_teacher_hidden", "grad_teacher_weight"):
        gk, rk = getattr(got, k), ref[k]
        assert (gk is None) == (rk is None), f"{k}: presence differs"
        if rk is not None:
            check_grad_device(k, gk, rk, dt)
