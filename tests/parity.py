"""Comparison helpers for the GPU parity tests.

Tolerances (stated once, used everywhere):
* loss, student_ce, teacher_ce, kl: |gpu - ref| <= 1e-4 * |ref| + an
  absolute floor per component (SCALAR_FLOOR), the fp32 resolution of the
  terms it is formed from;
* gradients, fp32 inputs: ||gpu - ref||_F <= 1e-3 * ||ref||_F and every
  element within 1e-3 * max|ref| (+1e-7);
* gradients, bf16 inputs (the oracle runs on the same bf16-rounded values):
  ||gpu - ref||_F <= 2e-2 * ||ref||_F and every element within
  2e-2 * max|ref|;
* INT8 codes of one and the same fp32 matrix: identical; scales identical;
* INT8 codes against the oracle (fp32 runs): scales within 1e-5 relative,
  codes equal except at rounding boundaries that the two unquantized
  gradients straddle (check_quantized_grad_weight).
"""
import numpy as np

LOSS_RTOL = 1e-4
# Scaled INT8 values x/s lie in [-127, 127]; the quantizer forms them with an
# fp32 division, whose rounding (half an ulp, at most 2^-17 at 127) can put a
# value onto a rounding boundary that the exact quotient sits beside.
TIE_EPS = 2.0 ** -16
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


# Absolute floors of the scalar gate, per component:
# * the CE terms (and the loss, which sums them): each row's NLL is
#   lse - x_y with |lse| up to ~20 at these vocabularies, where fp32 values
#   are spaced 1.9e-6 apart; a mean of such rows keeps that resolution;
# * kl: the fp32 formation floor of KL·T² per row, at most 0.5·2^-24·T²
#   (tests/test_gpu_kl_precision.py measures it per path), below 1e-6 for
#   T <= 4; the small-KL regime is tested there against tighter bounds.
SCALAR_FLOOR = {"loss": 2e-6, "student_ce": 2e-6, "teacher_ce": 2e-6, "kl": 1e-6}


def check_scalar(name, got, ref, rtol=LOSS_RTOL, floor=None):
    if floor is None:
        floor = SCALAR_FLOOR.get(name, 2e-6)
    tol = rtol * abs(ref) + floor
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


def _uniforms(seed, n):
    """The reference's draw sequence (quant.rs:18-44) from the oracle's Rng."""
    import oracle as O
    rng = O.Rng(seed)
    return np.array([rng.next_f32() for _ in range(n)], np.float32)


def check_quantized_grad_weight(got, ref, y, got_plain, ref_plain, ignore=-100,
                                stochastic=False, seed=0):
    """INT8 grad_W of an fp32 run against the oracle, at the gate's terms
    (src/quant.rs:91-144, 157-202): scales within 1e-5 relative; codes equal
    except where the two unquantized fp32 gradients (got_plain, ref_plain:
    the same calls with quantization off) fall on opposite sides of a
    rounding boundary — x.5 for round-half-even, floor(x) + u for stochastic
    rounding with the reference's draw u, allowing TIE_EPS for the rounding
    of the quantizer's fp32 quotient x/s — and those two scaled values within
    127 * 1e-4 of each other; target rows exact (fp32 tolerance); other rows
    exactly code * scale."""
    gw, rw = to_np(got.grad_weight), ref.grad_weight
    gq, rq = to_np(got.quant_codes).astype(np.int32), ref.quant_codes.astype(np.int32)
    gs, rs = to_np(got.quant_scales).reshape(-1), ref.quant_scales
    np.testing.assert_allclose(gs, rs, rtol=1e-5, atol=0)
    a_g = to_np(got_plain).astype(np.float64) / gs[:, None].astype(np.float64)
    a_o = np.asarray(ref_plain, np.float64) / rs[:, None].astype(np.float64)
    assert float(np.max(np.abs(a_g - a_o))) <= 127 * 1e-4, "unquantized gradients too far apart"
    flip = gq != rq
    assert np.all(np.abs(gq - rq) <= 1)
    if np.any(flip):
        lo = np.minimum(a_g, a_o)[flip] - TIE_EPS
        hi = np.maximum(a_g, a_o)[flip] + TIE_EPS
        if stochastic:
            u = _uniforms(seed, rw.size).reshape(rw.shape)[flip].astype(np.float64)
            bound = np.floor(lo) + u
            bound = np.where(bound < lo, bound + 1.0, bound)
        else:
            bound = np.floor(lo) + 0.5
            bound = np.where(bound < lo, bound + 1.0, bound)
        assert np.all(bound <= hi), "a code differs away from a rounding boundary"
    tgt = sorted({int(t) for t in y if t != ignore and 0 <= t < rw.shape[0]})
    mask = np.zeros(rw.shape[0], bool)
    mask[tgt] = True
    if tgt:
        check_grad("grad_weight[target rows]", gw[mask], rw[mask])
    # non-target rows are exactly code * scale
    np.testing.assert_array_equal(gw[~mask], (gq[~mask] * gs[~mask, None]).astype(np.float32))
    return int(np.count_nonzero(flip))


def check_quant_of_own_gradient(got, plain_gw, y, ignore=-100, stochastic=False, seed=0,
                                quant=None):
    """The quantized call's codes, scales and returned grad_W are identical to
    quantizing the same call's fp32 grad_W (the call with quantization off):
    the step 'mean-scale, then quantize the final grad_W' of
    src/api.rs:380-399. `quant(m, y)` -> (dequantized, codes, scales) is the
    quantizer used, by default the oracle's quant_dequant_grad_w on the host."""
    if quant is None:
        import oracle as O

        def quant(m, t):
            return O.quant_dequant_grad_w(to_np(m), to_np(t), ignore, stochastic, seed)
    deq, q, s = quant(plain_gw, y)
    if hasattr(deq, "is_cuda"):
        import torch
        assert torch.equal(got.quant_codes, q), "codes differ"
        assert torch.equal(got.quant_scales.reshape(-1), s.reshape(-1)), "scales differ"
        assert torch.equal(got.grad_weight, deq), "dequantized grad_W differs"
        return
    np.testing.assert_array_equal(to_np(got.quant_codes), q)
    np.testing.assert_array_equal(to_np(got.quant_scales).reshape(-1), s.reshape(-1))
    np.testing.assert_array_equal(to_np(got.grad_weight), deq)


def check_quantized_vs_reference_device(got, got_plain_gw, ref_gw, ref_codes, ref_scales):
    """check_quantized_grad_weight's code and scale criteria (deterministic
    rounding) on the device, for shapes the oracle cannot run: the reference
    codes and scales are those of an fp32 reference grad_W quantized by a
    quantizer pinned bit-exactly to the oracle's. Returns the number of
    codes that differ."""
    import torch
    gs = got.quant_scales.reshape(-1).double()
    rs = ref_scales.reshape(-1).double()
    assert float(((gs - rs).abs() / rs.abs()).max()) <= 1e-5, "scales differ by more than 1e-5"
    flips = 0
    for r0 in range(0, ref_gw.shape[0], 8192):
        sl = slice(r0, r0 + 8192)
        a_g = got_plain_gw[sl].double() / gs[sl, None]
        a_o = ref_gw[sl].double() / rs[sl, None]
        assert float((a_g - a_o).abs().max()) <= 127 * 1e-4, "unquantized gradients too far apart"
        gq, rq = got.quant_codes[sl].int(), ref_codes[sl].int()
        d = gq != rq
        assert int((gq - rq).abs().max()) <= 1
        if bool(d.any()):
            lo = torch.minimum(a_g, a_o)[d] - TIE_EPS
            hi = torch.maximum(a_g, a_o)[d] + TIE_EPS
            bound = torch.floor(lo) + 0.5
            bound = torch.where(bound < lo, bound + 1.0, bound)
            assert bool((bound <= hi).all()), "a code differs away from a rounding boundary"
            flips += int(d.sum())
    return flips


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
