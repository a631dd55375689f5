"""torch autograd op over the fused distillation loss.

The reference's `distillation_loss` is the Rust analogue of upstream
`api.py::distillation_loss` together with the `DistillCEFunction`
forward/backward (src/api.rs:1-12). This module is that caller for torch: the
forward runs the whole fused loss on the GPU (liborda_hip.so through the C ABI,
which computes every gradient in the same call, src/api.rs:263-399) and keeps
the gradients; the backward scales them by the incoming gradient of the loss.

Gradients follow the reference (src/api.rs:244-258, 346-375): the KL term is
teacher-detached; the teacher's hidden rows (Tied, Separate) and the teacher's
weight (Separate) receive the teacher-CE gradient only when the teacher-CE
weight is positive; Precomputed teacher logits receive none. Each gradient is
returned in its input's dtype.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import Context, distillation_loss
from .types import LossOptions, Teacher, TeacherMode


class DistillCEFunction(torch.autograd.Function):
    """loss, (student_ce, teacher_ce, kl) = DistillCEFunction.apply(
    student_hidden, weight, teacher_hidden, teacher_weight, labels,
    teacher_logits, mode, opts, lib_ctx)."""

    @staticmethod
    def forward(fctx, student_hidden, weight, teacher_hidden, teacher_weight, labels, teacher_logits,
                mode, opts, lib_ctx):
        teacher = Teacher(mode, hidden=None if teacher_hidden is None else teacher_hidden.detach(),
                          weight=None if teacher_weight is None else teacher_weight.detach(),
                          logits=None if teacher_logits is None else teacher_logits.detach())
        out = distillation_loss(student_hidden.detach(), weight.detach(), labels, teacher, opts,
                                ctx=lib_ctx)
        fctx.grads = (out.grad_student_hidden, out.grad_weight, out.grad_teacher_hidden,
                      out.grad_teacher_weight)
        fctx.dtypes = tuple(None if t is None else t.dtype
                            for t in (student_hidden, weight, teacher_hidden, teacher_weight))
        fctx.chunk_plan = out.chunk_plan
        dev = student_hidden.device
        loss = torch.tensor(out.loss, dtype=torch.float32, device=dev)
        comps = torch.tensor([out.student_ce, out.teacher_ce, out.kl], dtype=torch.float32,
                             device=dev)
        fctx.mark_non_differentiable(comps)
        return loss, comps

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(fctx, g_loss, g_comps):
        res = []
        for i, (g, dt) in enumerate(zip(fctx.grads, fctx.dtypes)):
            if g is None or dt is None or not fctx.needs_input_grad[i]:
                res.append(None)
            else:
                res.append((g * g_loss.to(g.dtype)).to(dt))
        fctx.grads = None
        return (*res, None, None, None, None, None)


def distillation_loss_autograd(student_hidden: torch.Tensor, weight: torch.Tensor, labels,
                               teacher: Teacher, opts: Optional[LossOptions] = None, *,
                               ctx: Optional[Context] = None
                               ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Differentiable form of `distillation_loss` for a training step.

    Returns ``(loss, components)``: ``loss`` is a 0-dim float32 tensor whose
    backward delivers the reference's gradients (scaled by the incoming
    gradient) to ``student_hidden``, ``weight`` and, where the reference has
    them, the teacher's hidden rows and weight; ``components`` holds
    ``[student_ce, teacher_ce, kl]`` (weight-free, kl including T², as in
    the reference's output, src/api.rs:71-92) and is not differentiable.
    Inputs must be GPU tensors.
    """
    opts = opts or LossOptions()
    if not (hasattr(student_hidden, "is_cuda") and student_hidden.is_cuda):
        raise ValueError("distillation_loss_autograd needs GPU tensors")
    mode = teacher.mode()
    th = teacher.hidden if mode in (TeacherMode.Tied, TeacherMode.Separate) else None
    tw = teacher.weight if mode == TeacherMode.Separate else None
    tl = teacher.logits if mode == TeacherMode.Precomputed else None
    return DistillCEFunction.apply(student_hidden, weight, th, tw, labels, tl, mode, opts, ctx)
