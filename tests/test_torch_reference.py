"""The float64 torch-autograd restatement (tests/torch_reference.py) against
the CPU oracle, on the reference's LCG inputs (tests/end_to_end.rs:14-36):
loss, components and every gradient of all teacher modes. This pins the torch
restatement that the GPU autograd-op tests compare with.
"""
import numpy as np
import pytest

import oracle as O
from helpers import labels, mat
from orda_hip.types import LossOptions, Reduction, Teacher
from torch_reference import loss_chunked, loss_f64, loss_tied_chunked

CASES = {
    # name: (mode, bt, h, ht, v, options, ignore_every)
    "tied_tce_smooth_mean": ("tied", 9, 6, 6, 11,
                             dict(kd_weight=0.5, temperature=1.5, teacher_ce_weight=1.0,
                                  label_smoothing=0.1), 4),
    "tied_default_weight": ("tied", 7, 5, 5, 13, dict(kd_weight=0.4, temperature=2.0), None),
    "tied_pure_student": ("tied", 6, 4, 4, 9, dict(teacher_ce_weight=0.0), 3),
    "separate_tce_sum": ("separate", 8, 5, 7, 10,
                         dict(kd_weight=0.5, temperature=2.0, teacher_ce_weight=1.0,
                              reduction=Reduction.Sum), None),
    "separate_default_weight": ("separate", 6, 4, 6, 9,
                                dict(kd_weight=0.5, temperature=2.0, label_smoothing=0.1), 5),
    "precomputed": ("precomputed", 7, 5, 5, 12, dict(kd_weight=0.7, temperature=1.0), 3),
}


def run_case(name):
    mode, bt, h, ht, v, o, every = CASES[name]
    s = mat(bt, h, 1, 0.5)
    w = mat(v, h, 2, 0.4)
    y = labels(bt, v, every)
    th = tw = tl = None
    if mode == "tied":
        th = mat(bt, h, 3, 0.5)
        teacher = Teacher.Tied(th)
    elif mode == "separate":
        th = mat(bt, ht, 3, 0.5)
        tw = mat(v, ht, 4, 0.4)
        teacher = Teacher.Separate(th, tw)
    else:
        tl = mat(bt, v, 5, 2.0)
        teacher = Teacher.Precomputed(tl)
    opts = LossOptions(**o)
    ref = O.distillation_loss(s, w, y, teacher, opts)
    tr = loss_f64(s, w, y, mode, th, tw, tl, w_s=opts.student_ce_weight,
                  w_t=opts.teacher_ce_weight, kd=opts.kd_weight, T=opts.temperature,
                  alpha=opts.label_smoothing, ignore=opts.ignore_index,
                  mean=opts.reduction == Reduction.Mean)
    return ref, tr


@pytest.mark.parametrize("name", sorted(CASES))
def test_torch_reference_matches_oracle(name):
    ref, tr = run_case(name)
    for k in ("loss", "student_ce", "teacher_ce", "kl"):
        r = getattr(ref, k)
        assert abs(tr[k] - r) <= 1e-5 * max(abs(r), 1e-2), f"{k}: torch {tr[k]!r} oracle {r!r}"
    for k in ("grad_student_hidden", "grad_weight", "grad_teacher_hidden", "grad_teacher_weight"):
        r = getattr(ref, k)
        t = tr[k]
        assert (r is None) == (t is None), f"{k}: presence differs"
        if r is None:
            continue
        r = np.asarray(r, np.float64)
        err = np.linalg.norm(t - r) / max(np.linalg.norm(r), 1e-30)
        assert err <= 1e-5, f"{k}: rel fro err {err:.3e}"


@pytest.mark.parametrize("opts,rows", [
    (dict(kd_weight=0.4, temperature=1.5, label_smoothing=0.1, teacher_ce_weight=1.0), 8),
    (dict(kd_weight=0.4, temperature=1.5, label_smoothing=0.1, teacher_ce_weight=1.0), 1024),
    (dict(kd_weight=0.7, temperature=0.5, teacher_ce_weight=0.5, reduction=Reduction.Sum), 5),
    (dict(teacher_ce_weight=0.0), 16),
])
def test_chunked_tied_reference_matches_oracle(opts, rows):
    """The row-chunked float32/float64 restatement used at the full benchmark
    shape, against the oracle: loss terms to 1e-6, gradients to 1e-5
    (float32 GEMMs in a different summation order)."""
    import torch
    bt, h, v = 37, 24, 300
    s, th, w = mat(bt, h, 1, 0.5), mat(bt, h, 3, 0.5), mat(v, h, 2, 0.4)
    y = labels(bt, v, 6)
    o = LossOptions(**opts)
    ref = O.distillation_loss(s, w, y, Teacher.Tied(th), o)
    got = loss_tied_chunked(torch.from_numpy(s), torch.from_numpy(th), torch.from_numpy(w),
                            torch.from_numpy(y), kd=o.kd_weight, T=o.temperature,
                            alpha=o.label_smoothing, w_s=o.student_ce_weight,
                            w_t=o.teacher_ce_weight if o.teacher_ce_weight is not None else 1.0,
                            ignore=o.ignore_index, mean=o.reduction == Reduction.Mean, rows=rows)
    for k in ("loss", "student_ce", "teacher_ce", "kl"):
        r = getattr(ref, k)
        assert abs(got[k] - r) <= 1e-6 * max(abs(r), 1e-2), f"{k}: chunked {got[k]!r} oracle {r!r}"
    for k in ("grad_student_hidden", "grad_weight", "grad_teacher_hidden"):
        r = getattr(ref, k)
        assert (r is None) == (got[k] is None), f"{k}: presence differs"
        if r is None:
            continue
        t = got[k].numpy().astype(np.float64)
        r = np.asarray(r, np.float64)
        err = np.linalg.norm(t - r) / max(np.linalg.norm(r), 1e-30)
        assert err <= 1e-5, f"{k}: rel fro err {err:.3e}"


@pytest.mark.parametrize("name,rows", [(n, r) for n in sorted(CASES) for r in (3, 1024)])
def test_chunked_reference_matches_oracle_all_modes(name, rows):
    """loss_chunked for every teacher mode (the full-size GPU tests' reference)
    against the oracle on the CASES inputs, in chunks of 3 rows and in one
    chunk: loss terms to 1e-6, gradients to 1e-5."""
    import torch
    mode, bt, h, ht, v, o, every = CASES[name]
    s, w = mat(bt, h, 1, 0.5), mat(v, h, 2, 0.4)
    y = labels(bt, v, every)
    th = tw = tl = None
    if mode == "tied":
        th = mat(bt, h, 3, 0.5)
        teacher = Teacher.Tied(th)
    elif mode == "separate":
        th, tw = mat(bt, ht, 3, 0.5), mat(v, ht, 4, 0.4)
        teacher = Teacher.Separate(th, tw)
    else:
        tl = mat(bt, v, 5, 2.0)
        teacher = Teacher.Precomputed(tl)
    opts = LossOptions(**o)
    ref = O.distillation_loss(s, w, y, teacher, opts)
    t = lambda a: None if a is None else torch.from_numpy(a)
    got = loss_chunked(t(s), t(w), t(y), mode, t(th), t(tw), t(tl), kd=opts.kd_weight,
                       T=opts.temperature, alpha=opts.label_smoothing, w_s=opts.student_ce_weight,
                       w_t=opts.teacher_ce_weight, ignore=opts.ignore_index,
                       mean=opts.reduction == Reduction.Mean, rows=rows)
    for k in ("loss", "student_ce", "teacher_ce", "kl"):
        r = getattr(ref, k)
        assert abs(got[k] - r) <= 1e-6 * max(abs(r), 1e-2), f"{k}: chunked {got[k]!r} oracle {r!r}"
    for k in ("grad_student_hidden", "grad_weight", "grad_teacher_hidden", "grad_teacher_weight"):
        r = getattr(ref, k)
        assert (r is None) == (got[k] is None), f"{k}: presence differs"
        if r is None:
            continue
        g = got[k].numpy().astype(np.float64)
        r = np.asarray(r, np.float64)
        err = np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-30)
        assert err <= 1e-5, f"{k}: rel fro err {err:.3e}"
