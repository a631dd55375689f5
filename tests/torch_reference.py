"""Plain-torch restatement of the distillation loss, float64 autograd on the CPU.

Independent of the oracle's chunked arithmetic: the loss is written as the
textbook expression of src/api.rs:188-422 (S-rules of the reference:
label-smoothed CE per row, src/reference/cross_entropy.rs:27-73;
teacher-detached forward KL at temperature T times T², src/reference/kl.rs:83-124;
weights and deferred mean, src/api.rs:211-230, 401-405) and the gradients come
from torch autograd. Used to pin the torch autograd op: the CPU tests check it
against the oracle, the GPU tests check the op's .grad values against it.
"""
import numpy as np
import torch
import torch.nn.functional as F


def loss_f64(hs, w, labels, mode, th=None, tw=None, tl=None, *, w_s=1.0, w_t=None, kd=0.0,
             T=1.0, alpha=0.0, ignore=-100, mean=True):
    """Returns dict(loss, student_ce, teacher_ce, kl, grad_student_hidden,
    grad_weight, grad_teacher_hidden, grad_teacher_weight) as float64 numpy
    values; absent gradients are None (src/api.rs:244-258)."""
    f64 = torch.float64
    hs = torch.tensor(np.asarray(hs, np.float64), dtype=f64, requires_grad=True)
    w = torch.tensor(np.asarray(w, np.float64), dtype=f64, requires_grad=True)
    y = torch.tensor(np.asarray(labels, np.int64))
    if w_t is None:
        w_t = 1.0 if mode == "tied" else 0.0
    th_t = tw_t = None
    if mode in ("tied", "separate"):
        th_t = torch.tensor(np.asarray(th, np.float64), dtype=f64, requires_grad=True)
    if mode == "separate":
        tw_t = torch.tensor(np.asarray(tw, np.float64), dtype=f64, requires_grad=True)
    valid = y != ignore
    n = max(int(valid.sum()), 1) if mean else 1
    ls = hs @ w.T
    ce_s = F.cross_entropy(ls, y, ignore_index=ignore, reduction="none", label_smoothing=alpha)
    if mode == "tied":
        lt = th_t @ w.T
    elif mode == "separate":
        lt = th_t @ tw_t.T
    elif mode == "precomputed":
        lt = torch.tensor(np.asarray(tl, np.float64), dtype=f64)
    else:
        lt = None
    zero = torch.zeros((), dtype=f64)
    ce_t = zero
    if lt is not None and w_t > 0:
        ce_t = F.cross_entropy(lt, y, ignore_index=ignore, reduction="none",
                               label_smoothing=alpha).sum()
    kl = zero
    if lt is not None and kd > 0:
        pt = torch.softmax(lt.detach() / T, dim=-1)
        kl_rows = (pt * (torch.log_softmax(lt.detach() / T, -1) -
                         torch.log_softmax(ls / T, -1))).sum(-1) * (T * T)
        kl = torch.where(valid, kl_rows, torch.zeros_like(kl_rows)).sum()
    s_ce = ce_s.sum()
    loss = (w_s * s_ce + w_t * ce_t + kd * kl) / n
    loss.backward()

    def g(t, keep):
        return t.grad.numpy() if (keep and t is not None and t.grad is not None) else None
    has_t = mode in ("tied", "separate") and w_t > 0
    return {
        "loss": loss.item(), "student_ce": s_ce.item() / n, "teacher_ce": ce_t.item() / n,
        "kl": kl.item() / n,
        "grad_student_hidden": g(hs, True), "grad_weight": g(w, True),
        "grad_teacher_hidden": g(th_t, has_t),
        "grad_teacher_weight": g(tw_t, has_t and mode == "separate"),
    }
