"""GPU tests of the torch autograd op (orda_hip.autograd): loss.backward()
through the HIP path must deliver the float64 torch-autograd gradients
(tests/torch_reference.py, itself pinned to the oracle on the CPU), scaled by
the incoming gradient, in each input's dtype, only to the inputs the
reference differentiates (src/api.rs:244-258). Tolerances as in tests/parity.py;
bf16 cases feed the reference the same bf16-rounded values.
"""
import numpy as np
import pytest

from helpers import bf16_round, normal, uniform_labels
from parity import check_grad, check_scalar
from torch_reference import loss_f64

import orda_hip as H
from orda_hip import LossOptions, Reduction, Teacher
from orda_hip.autograd import distillation_loss_autograd

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    assert H.is_available(), "liborda_hip.so does not see a gfx950 device"
    return torch, torch.device("cuda:0")


CASES = {
    # name: (mode, bt, h, ht, v, options, dtype)
    "tied_tce_smooth": ("tied", 96, 64, 64, 1000,
                        dict(kd_weight=0.4, temperature=1.5, label_smoothing=0.1), "f32"),
    "tied_bf16": ("tied", 128, 96, 96, 1500,
                  dict(kd_weight=0.4, temperature=1.5, label_smoothing=0.1), "bf16"),
    "separate_tce_sum": ("separate", 80, 48, 96, 900,
                         dict(kd_weight=0.5, temperature=2.0, teacher_ce_weight=1.0,
                              reduction=Reduction.Sum), "f32"),
    "separate_no_tce": ("separate", 64, 32, 64, 700,
                        dict(kd_weight=0.5, temperature=2.0), "f32"),
    "precomputed": ("precomputed", 72, 64, 64, 1100, dict(kd_weight=0.7, temperature=1.0), "f32"),
    "pure_student_bf16": ("tied", 100, 64, 64, 800, dict(teacher_ce_weight=0.0), "bf16"),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_autograd_op_gradients(torch_dev, name):
    torch, dev = torch_dev
    mode, bt, h, ht, v, o, dt = CASES[name]
    s = normal((bt, h), 1)
    w = normal((v, h), 2, 0.05)
    y = uniform_labels(bt, v, 3)
    y[::7] = -100
    th = tw = tl = None
    if mode in ("tied", "separate"):
        th = normal((bt, ht), 4)
    if mode == "separate":
        tw = normal((v, ht), 5, 0.04)
    if mode == "precomputed":
        tl = normal((bt, v), 6, 2.0)
    if dt == "bf16":
        s, w = bf16_round(s), bf16_round(w)
        th = None if th is None else bf16_round(th)
        tw = None if tw is None else bf16_round(tw)
    tdt = torch.bfloat16 if dt == "bf16" else torch.float32

    def leaf(a):
        if a is None:
            return None
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(tdt).requires_grad_(True)
    S, W, TH, TW = leaf(s), leaf(w), leaf(th), leaf(tw)
    Y = torch.from_numpy(y).to(dev)
    if mode == "tied":
        teacher = Teacher.Tied(TH)
    elif mode == "separate":
        teacher = Teacher.Separate(TH, TW)
    else:
        teacher = Teacher.Precomputed(torch.from_numpy(tl).to(dev))
    opts = LossOptions(**o)
    loss, comps = distillation_loss_autograd(S, W, Y, teacher, opts)
    (2.5 * loss).backward()

    ref = loss_f64(s, w, y, mode, th, tw, tl, w_s=opts.student_ce_weight,
                   w_t=opts.teacher_ce_weight, kd=opts.kd_weight, T=opts.temperature,
                   alpha=opts.label_smoothing, ignore=opts.ignore_index,
                   mean=opts.reduction == Reduction.Mean)
    check_scalar("loss", loss.item(), ref["loss"])
    for i, k in enumerate(("student_ce", "teacher_ce", "kl")):
        check_scalar(k, comps[i].item(), ref[k])
    assert not comps.requires_grad
    for t, k in ((S, "grad_student_hidden"), (W, "grad_weight"), (TH, "grad_teacher_hidden"),
                 (TW, "grad_teacher_weight")):
        if t is None:
            continue
        r = ref[k]
        if r is None:
            assert t.grad is None, f"{k}: the reference has no such gradient"
            continue
        assert t.grad is not None and t.grad.dtype == tdt, f"{k}: missing or wrong dtype"
        check_grad(k, t.grad, 2.5 * r, dt)


def test_autograd_op_in_a_training_step(torch_dev):
    """Drop-in use: the op inside an optimizer step lowers the loss."""
    torch, dev = torch_dev
    bt, h, v = 64, 32, 500
    g = torch.Generator(device=dev).manual_seed(0)
    S = torch.randn(bt, h, device=dev, generator=g).requires_grad_(True)
    W = (0.05 * torch.randn(v, h, device=dev, generator=g)).requires_grad_(True)
    TH = torch.randn(bt, h, device=dev, generator=g)
    Y = torch.randint(0, v, (bt,), device=dev, generator=g)
    opt = torch.optim.SGD([S, W], lr=0.5)
    opts = LossOptions(kd_weight=0.4, temperature=1.5)
    losses = []
    for _ in range(5):
        opt.zero_grad()
        loss, _ = distillation_loss_autograd(S, W, Y, Teacher.Tied(TH), opts)
        loss.backward()
        opt.step()
        losses.append(loss.item())
    assert all(b < a for a, b in zip(losses, losses[1:])), losses
