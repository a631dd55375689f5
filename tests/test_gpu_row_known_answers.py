"""The reference's own unit tests of its row functions run on the GPU row
kernels, through the chunk-launcher slot (orda_kl_ce_on_logits_chunk,
src/cuda/launch.rs:51-158): the cases and closed forms of
src/reference/cross_entropy.rs:92-148 (ce_fwdbwd_row) and
src/reference/kl.rs:160-223 (forward_kl_row, kl_chunk), with the expected
values formed in float64 here.

Tolerances: the reference's own where it states them for float32 results
(1e-6 on a gradient element or a loss, 1e-5 on a gradient sum); its float64
KL identities (1e-12) become exact zeros where the GPU forms the KL from
identical rows or ignores a row. A KL value against its float64 closed form
is held to 1e-5 relative: it is formed in float32 from terms of order 1
(Σ p_t^T·(t − s)/T and the two log-sum-exps) that cancel to KL values of
0.05-0.5 here, so a few roundings of 2^-24 at order 1 are up to ~2e-6 of
the result (measured: 1.5e-6 at T = 4).
"""
import numpy as np
import pytest

import orda_hip as H

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    assert H.is_available(), "liborda_hip.so does not see a gfx950 device"


def slot(student, teacher, y, T=1.0, kl_grad_scale=0.0, ws=1.0, wt=1.0, ls=0.0,
         student_only=True, compute_kl=False):
    """One student/teacher row pair through the slot (host inputs)."""
    lc = np.stack([np.asarray(student, np.float32), np.asarray(teacher, np.float32)])
    out = H.kl_ce_on_logits_chunk(lc, np.array([y], np.int32), 1, 1.0 / T, kl_grad_scale, T * T,
                                  ws, wt, ls, -100, student_only, compute_kl)
    return {k: np.asarray(v, np.float64) for k, v in out.items()}


def softmax(x, inv_t=1.0):
    z = np.asarray(x, np.float32).astype(np.float64) * inv_t
    e = np.exp(z - z.max())
    return e / e.sum()


def kl64(s, t, T):
    ps, pt = softmax(s, 1.0 / T), softmax(t, 1.0 / T)
    return float(np.sum(pt * (np.log(pt) - np.log(ps))))


# ---------------------------------------------- src/reference/cross_entropy.rs
def test_nll_equals_negative_log_softmax_of_target():
    # cross_entropy.rs:91-99
    x, y = [1.0, 2.0, 0.5, -1.0], 1
    got = slot(x, x, y)
    assert abs(got["ce_loss"][0] - (-np.log(softmax(x)[y]))) < 1e-6


def test_grad_is_softmax_minus_onehot():
    # cross_entropy.rs:101-120
    x, y = [0.3, -0.7, 1.1, 0.0], 2
    g = slot(x, x, y)["grad_ce"][0]
    expected = softmax(x)
    expected[y] -= 1.0
    assert np.max(np.abs(g - expected)) < 1e-6
    assert abs(g.sum()) < 1e-5


def test_ignored_row_is_zero():
    # cross_entropy.rs:122-128, and no KL term or KL gradient for the row
    x = [3.0, 1.0, -2.0]
    got = slot(x, [0.5, -0.5, 0.0], -100, T=1.5, kl_grad_scale=0.6, student_only=False,
               compute_kl=True)
    assert np.all(got["ce_loss"] == 0.0) and np.all(got["grad_ce"] == 0.0)
    assert got["kl_per_row"][0] == 0.0 and np.all(got["grad_kl_student"] == 0.0)


def test_scale_scales_gradient():
    # cross_entropy.rs:130-138: the row's CE weight scales its gradient
    x = [0.5, -0.5, 1.0]
    g1 = slot(x, x, 0, ws=1.0)["grad_ce"][0]
    g2 = slot(x, x, 0, ws=2.5)["grad_ce"][0]
    assert np.max(np.abs(g2 - 2.5 * g1)) < 1e-6


def test_label_smoothing_grad_sums_to_zero():
    # cross_entropy.rs:140-147
    x = [0.2, 1.3, -0.4, 0.9, 0.0]
    g = slot(x, x, 3, ls=0.1)["grad_ce"][0]
    assert abs(g.sum()) < 1e-5


# ------------------------------------------------------- src/reference/kl.rs
def test_identical_distributions_have_zero_kl():
    # kl.rs:160-165
    row = [0.3, 1.2, -0.7, 2.1, 0.0]
    got = slot(row, row, 0, T=1.5, kl_grad_scale=0.6, compute_kl=True)
    assert got["kl_per_row"][0] == 0.0
    assert np.all(got["grad_kl_student"] == 0.0)


@pytest.mark.parametrize("T", [0.5, 1.0, 1.5, 4.0])
def test_kl_is_nonnegative(T):
    # kl.rs:167-176, and the value itself against float64 (kl_per_row is KL·T²)
    s = [0.1, 0.2, 0.3, -1.0, 2.0]
    t = [1.0, -0.5, 0.0, 0.7, 0.2]
    k = slot(s, t, 0, T=T, compute_kl=True)["kl_per_row"][0]
    assert k >= 0.0
    assert abs(k - kl64(s, t, T) * T * T) <= 1e-5 * kl64(s, t, T) * T * T


def test_kl_matches_closed_form_two_class():
    # kl.rs:178-199: two logits, softmax(x/T) is a sigmoid
    T = 2.0
    s, t = [0.7, -0.4], [-0.2, 1.1]
    sig = lambda a, b: 1.0 / (1.0 + np.exp(-(a - b) / T))
    ps0, pt0 = sig(np.float32(s[0]), np.float32(s[1])), sig(np.float32(t[0]), np.float32(t[1]))
    ps1, pt1 = 1.0 - ps0, 1.0 - pt0
    expected = pt0 * (np.log(pt0) - np.log(ps0)) + pt1 * (np.log(pt1) - np.log(ps1))
    k = slot(s, t, 0, T=T, compute_kl=True)["kl_per_row"][0]
    assert abs(k - expected * T * T) <= 1e-5 * expected * T * T


def test_ignored_rows_contribute_zero():
    # kl.rs:201-209
    got = slot([1.0, 2.0, 3.0], [0.5, -0.5, 0.0], -100, T=1.5, kl_grad_scale=0.4 * 1.5,
               compute_kl=True)
    assert got["kl_per_row"][0] == 0.0
    assert np.all(got["grad_kl_student"] == 0.0)


def test_grad_matches_temperature_scaling():
    # kl.rs:211-223: grad = kl_weight·T/denom·(p_s − p_t), denom 1
    kw, T = 0.4, 1.5
    s, t = [0.2, 0.5, -0.1], [1.0, -1.0, 0.3]
    g = slot(s, t, 1, T=T, kl_grad_scale=np.float32(kw) * np.float32(T),
             compute_kl=True)["grad_kl_student"][0]
    expected = np.float32(kw * T) * (softmax(s, 1.0 / T) - softmax(t, 1.0 / T))
    assert np.max(np.abs(g - expected)) < 1e-6
