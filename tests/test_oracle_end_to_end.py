"""The reference's end-to-end tests (tests/end_to_end.rs) restated against
the CPU oracle, plus an independent NumPy float64 textbook derivation of the
whole loss and every gradient (a second pin for the orchestration).

Inputs use the reference's own LCG `fill` and `labels` helpers
(tests/end_to_end.rs:14-36), so these are the same cases the Rust tests run.
"""
import numpy as np
import pytest

import oracle as O
from helpers import fill, labels, mat
from orda_hip.types import (ChunkSize, KernelConfig, LossOptions, Reduction, Teacher)


def check_grad(param, analytic, eps, atol, rtol, loss_at):
    """tests/end_to_end.rs:43-78"""
    assert param.shape == analytic.shape
    work = param.copy()
    flat = work.reshape(-1)
    ana_flat = analytic.reshape(-1)
    max_rel = 0.0
    for idx in range(flat.size):
        base = flat[idx]
        flat[idx] = np.float32(base + np.float32(eps))
        lp = loss_at(work)
        flat[idx] = np.float32(base - np.float32(eps))
        lm = loss_at(work)
        flat[idx] = base
        num = (lp - lm) / (2.0 * eps)
        ana = float(ana_flat[idx])
        assert abs(ana - num) <= atol + rtol * max(abs(ana), abs(num)), \
            f"grad mismatch at {idx}: analytic={ana:.6e} numeric={num:.6e}"
        if max(abs(ana), abs(num)) > 1e-3:
            max_rel = max(max_rel, abs(ana - num) / max(abs(ana), abs(num)))
    assert max_rel < 0.05, f"max relative grad error too high: {max_rel}"


@pytest.fixture
def dl():
    """The distillation_loss under test: the oracle here (the same tests run
    against the HIP library in tests/test_gpu_end_to_end.py)."""
    return O.distillation_loss


def base_opts(**kw):
    """tests/end_to_end.rs:80-87"""
    d = dict(student_ce_weight=1.0, kd_weight=0.5, temperature=1.5)
    d.update(kw)
    return LossOptions(**d)


def test_tied_teacher_gradients_match_finite_difference(dl):
    # tests/end_to_end.rs:89-128
    bt, h, v = 6, 5, 7
    student = mat(bt, h, 1, 0.3)
    weight = mat(v, h, 2, 0.2)
    t_hidden = mat(bt, h, 3, 0.3)
    labs = labels(bt, v, 4)
    teacher = Teacher.Tied(t_hidden)
    opts = base_opts(teacher_ce_weight=1.0, label_smoothing=0.1)
    out = dl(student, weight, labs, teacher, opts)
    kt = O.teacher_logits(teacher, weight)
    check_grad(student, out.grad_student_hidden, 1e-3, 1e-3, 1e-2,
               lambda s: O.forward_loss_f64(s, weight, labs, teacher, opts, kt))
    check_grad(weight, out.grad_weight, 1e-3, 1e-3, 1e-2,
               lambda w: O.forward_loss_f64(student, w, labs, teacher, opts, kt))
    assert out.grad_teacher_hidden is not None
    check_grad(t_hidden, out.grad_teacher_hidden, 1e-3, 1e-3, 1e-2,
               lambda th: O.forward_loss_f64(student, weight, labs, Teacher.Tied(th), opts, kt))


def test_separate_teacher_gradients_match_finite_difference(dl):
    # tests/end_to_end.rs:130-178
    bt, h, ht, v = 6, 5, 4, 7
    student = mat(bt, h, 11, 0.3)
    weight = mat(v, h, 12, 0.2)
    t_hidden = mat(bt, ht, 13, 0.3)
    t_weight = mat(v, ht, 14, 0.2)
    labs = labels(bt, v, None)
    opts = base_opts(teacher_ce_weight=0.7)
    teacher = Teacher.Separate(t_hidden, t_weight)
    out = dl(student, weight, labs, teacher, opts)
    kt = O.teacher_logits(teacher, weight)
    check_grad(student, out.grad_student_hidden, 1e-3, 1e-3, 1e-2,
               lambda s: O.forward_loss_f64(s, weight, labs, teacher, opts, kt))
    check_grad(weight, out.grad_weight, 1e-3, 1e-3, 1e-2,
               lambda w: O.forward_loss_f64(student, w, labs, teacher, opts, kt))
    check_grad(t_hidden, out.grad_teacher_hidden, 1e-3, 1e-3, 1e-2,
               lambda th: O.forward_loss_f64(student, weight, labs,
                                             Teacher.Separate(th, t_weight), opts, kt))
    check_grad(t_weight, out.grad_teacher_weight, 1e-3, 1e-3, 1e-2,
               lambda tw: O.forward_loss_f64(student, weight, labs,
                                             Teacher.Separate(t_hidden, tw), opts, kt))


def test_precomputed_teacher_gradients_match_finite_difference(dl):
    # tests/end_to_end.rs:180-204
    bt, h, v = 6, 5, 7
    student = mat(bt, h, 21, 0.3)
    weight = mat(v, h, 22, 0.2)
    t_logits = mat(bt, v, 23, 0.5)
    labs = labels(bt, v, 5)
    opts = base_opts()
    teacher = Teacher.Precomputed(t_logits)
    out = dl(student, weight, labs, teacher, opts)
    assert out.grad_teacher_hidden is None and out.grad_teacher_weight is None
    check_grad(student, out.grad_student_hidden, 1e-3, 1e-3, 1e-2,
               lambda s: O.loss_only_f64(s, weight, labs, teacher, opts))
    check_grad(weight, out.grad_weight, 1e-3, 1e-3, 1e-2,
               lambda w: O.loss_only_f64(student, w, labs, teacher, opts))


def test_pure_student_ce_no_teacher_term(dl):
    # tests/end_to_end.rs:206-228
    bt, h, v = 8, 4, 6
    student = mat(bt, h, 31, 0.3)
    weight = mat(v, h, 32, 0.2)
    labs = labels(bt, v, None)
    teacher = Teacher.Tied(np.zeros((bt, h), np.float32))
    opts = LossOptions(kd_weight=0.0, teacher_ce_weight=0.0)
    out = dl(student, weight, labs, teacher, opts)
    assert out.teacher_ce == 0.0 and out.kl == 0.0
    check_grad(student, out.grad_student_hidden, 1e-3, 1e-3, 1e-2,
               lambda s: O.loss_only_f64(s, weight, labs, teacher, opts))


def test_chunking_is_exact_invariant(dl):
    # tests/end_to_end.rs:230-278
    bt, h, v = 16, 5, 9
    student = mat(bt, h, 41, 0.3)
    weight = mat(v, h, 42, 0.2)
    teacher = Teacher.Tied(mat(bt, h, 43, 0.3))
    labs = labels(bt, v, 3)

    def mk(cs):
        return dl(student, weight, labs, teacher,
                                   base_opts(chunk_size=cs, teacher_ce_weight=1.0))
    full = mk(ChunkSize.Fixed(bt))
    for other in (mk(ChunkSize.Fixed(1)), mk(ChunkSize.Fixed(3)), mk(ChunkSize.Auto)):
        assert abs(full.loss - other.loss) < 1e-5
        assert np.max(np.abs(full.grad_weight - other.grad_weight)) < 1e-5
        assert np.max(np.abs(full.grad_student_hidden - other.grad_student_hidden)) < 1e-5


def test_loss_components_and_total_are_consistent(dl):
    # tests/end_to_end.rs:280-311
    bt, h, v = 10, 4, 8
    student = mat(bt, h, 51, 0.3)
    weight = mat(v, h, 52, 0.2)
    teacher = Teacher.Tied(mat(bt, h, 53, 0.3))
    labs = labels(bt, v, None)
    w_s, w_t, kd = 1.0, 0.8, 0.5
    opts = LossOptions(student_ce_weight=w_s, teacher_ce_weight=w_t, kd_weight=kd,
                       temperature=2.0)
    out = dl(student, weight, labs, teacher, opts)
    f32 = np.float32
    recon = f32(w_s) * f32(out.student_ce) + f32(w_t) * f32(out.teacher_ce) + \
        f32(kd) * f32(out.kl)
    assert abs(recon - out.loss) < 1e-4
    assert abs(np.float32(O.loss_only_f64(student, weight, labs, teacher, opts)) - out.loss) < 1e-3


def test_sum_reduction_is_mean_times_token_count(dl):
    # tests/end_to_end.rs:313-358
    bt, h, v = 8, 4, 6
    student = mat(bt, h, 61, 0.3)
    weight = mat(v, h, 62, 0.2)
    teacher = Teacher.Tied(mat(bt, h, 63, 0.3))
    labs = labels(bt, v, 4)
    n_valid = float(np.sum(labs != -100))
    mean = dl(student, weight, labs, teacher,
                               base_opts(reduction=Reduction.Mean, teacher_ce_weight=1.0))
    summ = dl(student, weight, labs, teacher,
                               base_opts(reduction=Reduction.Sum, teacher_ce_weight=1.0))
    assert abs(summ.loss - mean.loss * n_valid) < 1e-3
    assert np.all(np.abs(summ.grad_weight - mean.grad_weight * n_valid) < 1e-3)


def test_int8_quant_grad_w_is_close_but_lossy(dl):
    # tests/end_to_end.rs:360-417
    bt, h, v = 8, 4, 20
    student = mat(bt, h, 71, 0.3)
    weight = mat(v, h, 72, 0.2)
    teacher = Teacher.Tied(mat(bt, h, 73, 0.3))
    labs = labels(bt, v, None)
    exact = dl(student, weight, labs, teacher, base_opts(teacher_ce_weight=1.0))
    cfg = KernelConfig(quantize_grad_weight=True)
    quant = dl(student, weight, labs, teacher,
                                base_opts(config=cfg, teacher_ce_weight=1.0))
    assert abs(exact.loss - quant.loss) < 1e-6
    max_abs = float(np.max(np.abs(exact.grad_weight - quant.grad_weight)))
    assert 0.0 < max_abs < 0.05


def test_validation_messages():
    """api.rs:104-181 error strings (the reference's Err(String))."""
    s = mat(4, 3, 1, 0.3)
    w = mat(5, 3, 2, 0.2)
    t = Teacher.Tied(mat(4, 3, 3, 0.3))
    with pytest.raises(O.OracleError, match=r"label 5 out of range \[0, 5\) and != ignore_index -100"):
        O.distillation_loss(s, w, np.array([0, 1, 5, 2]), t, LossOptions())
    with pytest.raises(O.OracleError, match="labels must have length BT=4, got 3"):
        O.distillation_loss(s, w, np.array([0, 1, 2]), t, LossOptions())
    with pytest.raises(O.OracleError, match=r"label_smoothing must be in \[0,1\], got 1.5"):
        O.distillation_loss(s, w, np.array([0, 1, 2, 3]), t, LossOptions(label_smoothing=1.5))
    with pytest.raises(O.OracleError, match="temperature must be > 0, got 0"):
        O.distillation_loss(s, w, np.array([0, 1, 2, 3]), t, LossOptions(temperature=0.0))
    with pytest.raises(O.OracleError, match="kd_weight must be >= 0"):
        O.distillation_loss(s, w, np.array([0, 1, 2, 3]), t, LossOptions(kd_weight=-1.0))
    with pytest.raises(O.OracleError, match=r"Tied teacher hidden must be \(4, 3\), got \(4, 2\)"):
        O.distillation_loss(s, w, np.array([0, 1, 2, 3]), Teacher.Tied(mat(4, 2, 3, 0.3)),
                            LossOptions())
    with pytest.raises(O.OracleError, match="teacher_ce_weight must be >= 0"):
        O.distillation_loss(s, w, np.array([0, 1, 2, 3]), t, LossOptions(teacher_ce_weight=-0.5))
    with pytest.raises(O.OracleError, match="max_fused_size must be a power of two"):
        O.distillation_loss(s, w, np.array([0, 1, 2, 3]), t,
                            LossOptions(config=KernelConfig(max_fused_size=100)))


# ------------------------------------------------------------------ textbook
def textbook(student, weight, labs, mode, t_hidden=None, t_weight=None, t_logits=None, w_s=1.0,
             w_t=None, kd=0.0, T=1.0, alpha=0.0, ignore=-100, reduction="mean"):
    """Whole loss and gradients from the definitions, in float64:
    L = [Σ_r w_s·CE_α(s_r) + w_t·CE_α(t_r) + kd·T²·KL(softmax(t_r/T) || softmax(s_r/T))]/N
    with the teacher distribution detached inside KL."""
    f = np.float64
    s_h, W = student.astype(f), weight.astype(f)
    if w_t is None:
        w_t = 1.0 if mode == "tied" else 0.0
    bt, v = s_h.shape[0], W.shape[0]
    zs = s_h @ W.T
    if mode == "tied":
        zt = t_hidden.astype(f) @ W.T
    elif mode == "separate":
        zt = t_hidden.astype(f) @ t_weight.astype(f).T
    else:
        zt = t_logits.astype(f)
    valid = labs != ignore
    n = max(int(valid.sum()), 1) if reduction == "mean" else 1
    ysafe = np.where(valid, labs, 0)
    q = np.full((bt, v), alpha / v)
    q[np.arange(bt), ysafe] += 1 - alpha

    def lsm(z):
        m = z.max(1, keepdims=True)
        return z - m - np.log(np.exp(z - m).sum(1, keepdims=True))
    lps, lpt = lsm(zs), lsm(zt)
    ce_s = -(q * lps).sum(1) * valid
    ce_t = -(q * lpt).sum(1) * valid
    lpsT, lptT = lsm(zs / T), lsm(zt / T)
    ptT = np.exp(lptT)
    kl = (ptT * (lptT - lpsT)).sum(1) * valid * T * T
    loss = (w_s * ce_s.sum() + w_t * ce_t.sum() + kd * kl.sum()) / n
    dzs = (w_s * (np.exp(lps) - q) + kd * T * (np.exp(lpsT) - ptT)) * valid[:, None] / n
    dzt = w_t * (np.exp(lpt) - q) * valid[:, None] / n
    g = dict(loss=loss, student_ce=ce_s.sum() / n, teacher_ce=(ce_t.sum() / n) if w_t > 0 else 0.0,
             kl=kl.sum() / n if kd > 0 else 0.0, ghs=dzs @ W, gw=dzs.T @ s_h)
    if w_t > 0 and mode == "tied":
        g["ght"] = dzt @ W
        g["gw"] = g["gw"] + dzt.T @ t_hidden.astype(f)
    if w_t > 0 and mode == "separate":
        g["ght"] = dzt @ t_weight.astype(f)
        g["gwt"] = dzt.T @ t_hidden.astype(f)
    return g


@pytest.mark.parametrize("mode", ["tied", "separate", "precomputed"])
@pytest.mark.parametrize("alpha,kd,T,w_t,reduction", [
    (0.0, 0.4, 1.5, None, "mean"), (0.1, 0.5, 2.0, 1.0, "mean"), (0.1, 0.7, 1.0, 0.3, "sum"),
    (0.0, 0.0, 1.0, 0.0, "mean")])
def test_oracle_matches_textbook_f64(mode, alpha, kd, T, w_t, reduction):
    rng = np.random.default_rng(11)
    bt, h, ht, v = 37, 24, 16, 53
    s = rng.standard_normal((bt, h)).astype(np.float32)
    W = (rng.standard_normal((v, h)) * 0.3).astype(np.float32)
    th = rng.standard_normal((bt, ht if mode == "separate" else h)).astype(np.float32)
    tw = (rng.standard_normal((v, ht)) * 0.3).astype(np.float32)
    tl = (rng.standard_normal((bt, v)) * 2).astype(np.float32)
    labs = rng.integers(0, v, bt)
    labs[::5] = -100
    teacher = {"tied": Teacher.Tied(th), "separate": Teacher.Separate(th, tw),
               "precomputed": Teacher.Precomputed(tl)}[mode]
    opts = LossOptions(kd_weight=kd, temperature=T, label_smoothing=alpha, teacher_ce_weight=w_t,
                       reduction=Reduction.Mean if reduction == "mean" else Reduction.Sum,
                       chunk_size=ChunkSize.Fixed(10))
    out = O.distillation_loss(s, W, labs, teacher, opts)
    ref = textbook(s, W, labs, mode, th, tw, tl, w_t=w_t, kd=kd, T=T, alpha=alpha,
                   reduction=reduction)
    for k in ("loss", "student_ce", "teacher_ce", "kl"):
        assert abs(getattr(out, k) - ref[k]) <= 1e-5 * max(1.0, abs(ref[k])), k

    def close(a, b):
        err = np.abs(a - b).max()
        assert err <= 1e-5 * max(1.0, np.abs(b).max()), err
    close(out.grad_student_hidden, ref["ghs"])
    close(out.grad_weight, ref["gw"])
    if "ght" in ref:
        close(out.grad_teacher_hidden, ref["ght"])
    else:
        assert out.grad_teacher_hidden is None
    if "gwt" in ref:
        close(out.grad_teacher_weight, ref["gwt"])
    else:
        assert out.grad_teacher_weight is None
    assert (out.chunk_plan.chunk_size, out.chunk_plan.num_chunks) == (10, 4)


@pytest.mark.parametrize("mode,quant", [("tied", False), ("tied", True), ("separate", False),
                                        ("precomputed", True)])
def test_threaded_products_are_bitwise_the_same(mode, quant):
    """The all-core CPU baseline shares the products' output rows (and the
    element-wise and INT8 row loops) between threads; every output element
    keeps the reference's accumulation order, so a whole loss call must come
    out bitwise identical."""
    rng = np.random.default_rng(41)
    bt, h, ht, v = 37, 29, 23, 211
    s = rng.standard_normal((bt, h), dtype=np.float32)
    W = (rng.standard_normal((v, h), dtype=np.float32) * 0.05).astype(np.float32)
    y = rng.integers(0, v, bt)
    y[::5] = -100
    if mode == "tied":
        t = Teacher.Tied(rng.standard_normal((bt, h), dtype=np.float32))
    elif mode == "separate":
        t = Teacher.Separate(rng.standard_normal((bt, ht), dtype=np.float32),
                             (rng.standard_normal((v, ht), dtype=np.float32) * 0.05))
    else:
        t = Teacher.Precomputed(rng.standard_normal((bt, v), dtype=np.float32))
    opts = LossOptions(kd_weight=0.5, temperature=1.5, label_smoothing=0.1,
                       teacher_ce_weight=0.7 if mode != "precomputed" else None,
                       chunk_size=ChunkSize.Fixed(10),
                       config=KernelConfig(quantize_grad_weight=quant))
    one = O.distillation_loss(s, W, y, t, opts)
    try:
        O.set_threads(4)
        many = O.distillation_loss(s, W, y, t, opts)
        a, b = rng.standard_normal((53, 41), dtype=np.float32), rng.standard_normal((53, 17),
                                                                                    dtype=np.float32)
        a[3, :] = 0.0
        tn4 = O.matmul_tn(a, b)
    finally:
        O.set_threads(1)
    assert np.array_equal(O.matmul_tn(a, b), tn4)
    for k in ("loss", "student_ce", "teacher_ce", "kl"):
        assert getattr(one, k) == getattr(many, k), k
    for k in ("grad_student_hidden", "grad_weight", "grad_teacher_hidden", "grad_teacher_weight"):
        x, z = getattr(one, k), getattr(many, k)
        assert (x is None) == (z is None), k
        if x is not None:
            assert np.array_equal(x, z), k
