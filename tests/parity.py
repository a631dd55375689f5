"""Comparison helpers for the GPU parity tests.

Tolerances (stated once, used everywhere):
* loss, student_ce, teacher_ce, kl: |gpu - ref| <= 1e-4 * max(|ref|, 1e-2)
  (a 1e-6 absolute floor covers components that are exactly zero);
* gradients, fp32 inputs: ||gpu - ref||_F <= 1e-3 * ||ref||_F and every
  element within 1e-3 * max|ref| (+1e-7);
* gradients, bf16 inputs (the oracle runs on the same bf16-rounded values):
  ||gpu - ref||_F <= 2e-2 * ||ref||_F and every element within
  2e-2 * max|ref|;
* INT8 codes of one and the same fp32 matrix: identical; scales identical.
"""
import numpy as np

LOSS_RTOL = 1e-4
GRAD_RTOL = {"f32": 1e-3, "bf16": 2e-2}


def to_np(x):
    if x is None:
        return None
    if hasattr(x, "detach"):
        x = x.detach()
        if x.dtype.is_floating_point:
            x = x.float()
        return x.cpu().numpy()
    return np.asarray(x)


def check_scalar(name, got, ref, rtol=LOSS_RTOL):
    tol = rtol * max(abs(ref), 1e-2) + 1e-6
    assert abs(got - ref) <= tol, f"{name}: gpu {got!r} vs ref {ref!r} (tol {tol:.3g})"


def check_grad(name, got, ref, kind="f32"):
    got, ref = to_np(got), to_np(ref)
    assert got.shape == ref.shape, f"{name}: shape {got.shape} vs {ref.shape}"
    assert np.all(np.isfinite(got)), f"{name}: non-finite values"
    rtol = GRAD_RTOL[kind]
    nref = float(np.linalg.norm(ref.astype(np.float64)))
    diff = got.astype(np.float64) - ref.astype(np.float64)
    ndiff = float(np.linalg.norm(diff))
    assert ndiff <= rtol * nref + 1e-12, f"{name}: rel fro err {ndiff / max(nref, 1e-30):.3e}"
    amax = float(np.max(np.abs(ref))) if ref.size else 0.0
    emax = float(np.max(np.abs(diff))) if ref.size else 0.0
    assert emax <= rtol * amax + 1e-7, f"{name}: max elem err {emax:.3e} vs max|ref| {amax:.3e}"
    return ndiff / max(nref, 1e-30)


def check_grad_device(name, got, ref, kind="f32", block=8192):
    """check_grad's criteria evaluated with torch on the tensors' device, a
    block of rows at a time in float64, for gradients too large to copy to
    the host."""
    import torch
    assert tuple(got.shape) == tuple(ref.shape), f"{name}: shape {tuple(got.shape)} vs {tuple(ref.shape)}"
    rtol = GRAD_RTOL[kind]
    sref = sdiff = 0.0
    amax = emax = 0.0
    for r0 in range(0, got.shape[0], block):
        g = got[r0:r0 + block].double()
        r = ref[r0:r0 + block].double()
        assert bool(torch.isfinite(g).all()), f"{name}: non-finite values"
        d = g - r
        sref += float((r * r).sum())
        sdiff += float((d * d).sum())
        amax = max(amax, float(r.abs().max()))
        emax = max(emax, float(d.abs().max()))
    nref, ndiff = sref ** 0.5, sdiff ** 0.5
    assert ndiff <= rtol * nref + 1e-12, f"{name}: rel fro err {ndiff / max(nref, 1e-30):.3e}"
    assert emax <= rtol * amax + 1e-7, f"{name}: max elem err {emax:.3e} vs max|ref| {amax:.3e}"
    return ndiff / max(nref, 1e-30)


def check_quantized_grad_weight(got, ref, y, ignore=-100):
    """Dequantized grad_W of an fp32 run: target rows carry the exact
    gradient (fp32 tolerance); other rows are code*scale with codes within
    ±1 of the oracle's (grad_W itself differs in its last bits, so a code may
    flip at a rounding boundary) and scales within 1e-3 relative."""
    gw, rw = to_np(got.grad_weight), ref.grad_weight
    gq, rq = to_np(got.quant_codes).astype(np.int32), ref.quant_codes.astype(np.int32)
    gs, rs = to_np(got.quant_scales).reshape(-1), ref.quant_scales
    tgt = sorted({int(t) for t in y if t != ignore})
    assert np.all(np.abs(gq - rq) <= 1)
    assert np.mean(gq != rq) < 0.01
    np.testing.assert_allclose(gs, rs, rtol=1e-3, atol=1e-30)
    mask = np.zeros(rw.shape[0], bool)
    mask[tgt] = True
    if tgt:
        check_grad("grad_weight[target rows]", gw[mask], rw[mask])
    # non-target rows are exactly code * scale
    np.testing.assert_array_equal(gw[~mask], (gq[~mask] * gs[~mask, None]).astype(np.float32))


def check_output(got, ref, kind="f32", skip_grad_weight=False):
    for k in ("loss", "student_ce", "teacher_ce", "kl"):
        check_scalar(k, getattr(got, k), getattr(ref, k))
    check_grad("grad_student_hidden", got.grad_student_hidden, ref.grad_student_hidden, kind)
    if not skip_grad_weight:
        check_grad("grad_weight", got.grad_weight, ref.grad_weight, kind)
    for k in ("grad_teacher_hidden", "grad_teacher_weight"):
        g, r = getattr(got, k), getattr(ref, k)
        assert (g is None) == (r is None), f"{k}: presence differs"
        if r is not None:
            check_grad(k, g, r, kind)
    assert (got.chunk_plan.chunk_size, got.chunk_plan.num_chunks) == \
        (ref.chunk_plan.chunk_size, ref.chunk_plan.num_chunks), "chunk plan differs"
