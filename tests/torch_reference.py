"""Plain-torch restatement of the distillation loss, float64 autograd on the CPU.

Independent of the oracle's chunked arithmetic: the loss is written as the
textbook expression of src/api.rs:188-422 (S-rules of the reference:
label-smoothed CE per row, src/reference/cross_entropy.rs:27-73;
teacher-detached forward KL at temperature T times T², src/reference/kl.rs:83-124;
weights and deferred mean, src/api.rs:211-230, 401-405) and the gradients come
from torch autograd. Used to pin the torch autograd op: the CPU tests check it
against the oracle, the GPU tests check the op's .grad values against it.

`loss_chunked` states the same loss row-chunked with explicit gradients
(float32 GEMMs, float64 row arithmetic) for every teacher mode, on any
device: the full-size GPU tests run it on the GPU beside the library; the CPU
tests pin it to the oracle at small sizes.
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


def loss_chunked(hs, w, labels, mode, th=None, tw=None, tl=None, *, kd, T, alpha, w_s=1.0,
                 w_t=None, ignore=-100, mean=True, rows=1024):
    """Any teacher mode at any size, on the tensors' own device, `rows` rows
    at a time: logits hs·Wᵀ and the teacher's (th·Wᵀ Tied, th·twᵀ Separate,
    tl Precomputed) as float32 GEMMs; log-sum-exp, losses and dlogits in
    float64 (label-smoothed CE per row, src/reference/cross_entropy.rs:27-73;
    teacher-detached KL at T, gradient kd·T·(p_s − p_t), src/reference/
    kl.rs:83-124; KL merged into the student rows, src/api.rs:336-344;
    teacher CE and its gradient to the teacher's parameters when w_t > 0,
    src/api.rs:316-333); the deferred mean as the float32 1/max(n_valid, 1)
    applied to every gradient (src/api.rs:225-230, 381-388); backward GEMMs
    in float32 (src/api.rs:346-370). Explicit gradients, no autograd, so the
    full benchmark shapes fit. Returns the loss terms as floats and float32
    gradient tensors (None where the reference returns none,
    src/api.rs:244-258)."""
    dev = hs.device
    if w_t is None:
        w_t = 1.0 if mode == "tied" else 0.0
    wf = w.float()
    twf = tw.float() if mode == "separate" else None
    n, h = hs.shape
    V = w.shape[0]
    y = labels.to(dev)
    valid = y != ignore
    nv = int(valid.sum())
    scale = float(np.float32(1.0) / np.float32(max(nv, 1))) if mean else 1.0
    f32 = torch.float32
    t_grad = mode in ("tied", "separate") and w_t > 0
    gs = torch.empty(n, h, dtype=f32, device=dev)
    gw = torch.zeros(V, h, dtype=f32, device=dev)
    gt = torch.empty(n, th.shape[1], dtype=f32, device=dev) if t_grad else None
    gtw = torch.zeros(V, th.shape[1], dtype=f32, device=dev) if t_grad and mode == "separate" else None
    sums = {"s": 0.0, "t": 0.0, "kl": 0.0}

    def ce(x, vm, ys, idx):
        xd = x.double()
        lse = torch.logsumexp(xd, 1)
        nll = lse - xd[idx, ys]
        if alpha > 0:
            nll = lse - (1 - alpha) * xd[idx, ys] - (alpha / V) * xd.sum(1)
        g = torch.exp(xd - lse[:, None])
        if alpha > 0:
            g -= alpha / V
        g[idx, ys] -= 1 - alpha
        g[~vm] = 0
        return float(torch.where(vm, nll, torch.zeros_like(nll)).sum()), g

    for r0 in range(0, n, rows):
        r1 = min(r0 + rows, n)
        hs_c = hs[r0:r1].float()
        vm = valid[r0:r1]
        ys = torch.where(vm, y[r0:r1], torch.zeros_like(y[r0:r1]))
        idx = torch.arange(r1 - r0, device=dev)
        ls = hs_c @ wf.T
        ht_c = th[r0:r1].float() if mode in ("tied", "separate") else None
        if mode == "tied":
            lt = ht_c @ wf.T
        elif mode == "separate":
            lt = ht_c @ twf.T
        else:
            lt = tl[r0:r1].float()
        nll, ds = ce(ls, vm, ys, idx)
        sums["s"] += nll
        ds *= w_s
        if kd > 0:
            lps = torch.log_softmax(ls.double() / T, 1)
            lpt = torch.log_softmax(lt.double() / T, 1)
            pt = lpt.exp()
            kl = (pt * (lpt - lps)).sum(1) * (T * T)
            sums["kl"] += float(torch.where(vm, kl, torch.zeros_like(kl)).sum())
            gk = kd * T * (lps.exp() - pt)
            gk[~vm] = 0
            ds += gk
            del lps, lpt, pt, gk
        dsf = (ds * scale).to(f32)
        del ds
        gs[r0:r1] = dsf @ wf
        gw += dsf.T @ hs_c
        if w_t > 0:
            nll, dt = ce(lt, vm, ys, idx)
            sums["t"] += nll
            if t_grad:
                dtf = (dt * (w_t * scale)).to(f32)
                if mode == "tied":
                    gt[r0:r1] = dtf @ wf
                    gw += dtf.T @ ht_c
                else:
                    gt[r0:r1] = dtf @ twf
                    gtw += dtf.T @ ht_c
                del dtf
            del dt
    loss = (w_s * sums["s"] + w_t * sums["t"] + kd * sums["kl"]) * scale
    return {"loss": loss, "student_ce": sums["s"] * scale, "teacher_ce": sums["t"] * scale,
            "kl": sums["kl"] * scale, "grad_student_hidden": gs, "grad_weight": gw,
            "grad_teacher_hidden": gt, "grad_teacher_weight": gtw}


def loss_tied_chunked(hs, ht, w, labels, *, kd, T, alpha, w_s=1.0, w_t=1.0, ignore=-100,
                      mean=True, rows=1024):
    """loss_chunked for a Tied teacher (teacher CE weight 1 by default)."""
    return loss_chunked(hs, w, labels, "tied", th=ht, kd=kd, T=T, alpha=alpha, w_s=w_s, w_t=w_t,
                        ignore=ignore, mean=mean, rows=rows)
