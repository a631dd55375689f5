"""GPU parity on the edges of the bf16 and staging paths, against the CPU
oracle on identical seeded inputs (bf16 runs feed the oracle the same
bf16-rounded values; tolerances as in tests/parity.py):

* Separate teacher in bf16 with a teacher width that is not a multiple of 8
  (staged into a padded copy) and Hs != Ht;
* Precomputed teacher logits next to bf16 hidden states: fp32 logits used in
  place, fp32 logits with an odd vocabulary (converted), bf16 logits
  (read in the logits GEMM's epilogue where aligned), and a strided device
  view; fp32 and bf16 logits read in the logits GEMM's epilogue (ragged
  vocabularies, their own pitch, teacher CE) or converted where they cannot
  be;
* a Separate teacher's fp32 logits read in the student logits GEMM's
  epilogue (bf16 inputs, KL, with and without teacher CE);
* hidden widths that are not a multiple of 8 (padded staging of bf16);
* strided device views of the inputs, 16-byte aligned (used in place) and
  not (staged);
* paired student/teacher rows at a row count that is not a multiple of 16;
* temperatures far from 1 and full label smoothing (alpha = 1);
* stochastic INT8 rounding of grad_W through the whole path;
* an empty hidden width (H = 0, or a Separate teacher's Ht = 0) and an
  empty vocabulary (V = 0, every label ignored), which the reference
  accepts (src/api.rs:104-181).
"""
import numpy as np
import pytest

import oracle as O
from helpers import bf16_round, normal, uniform_labels
from parity import (check_grad, check_output, check_quant_of_own_gradient,
                    check_quantized_grad_weight, to_np)

import orda_hip as H
from orda_hip import ChunkSize, KernelConfig, LossOptions, Teacher

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    assert H.is_available(), "liborda_hip.so does not see a gfx950 device"
    return torch, torch.device("cuda:0")


def dev(torch_dev, a, dtype=None):
    torch, d = torch_dev
    t = torch.from_numpy(np.ascontiguousarray(a)).to(d)
    return t.to(torch.bfloat16) if dtype == "bf16" else t


def strided(torch_dev, a, offset, pad, dtype=None):
    """Device view of `a` inside a wider buffer: columns [offset, offset+cols)
    of rows `pad` elements longer than `a`'s, so the view has a row pitch of
    cols + pad and a base `offset` elements into the allocation."""
    torch, d = torch_dev
    rows, cols = a.shape
    big = np.full((rows, cols + pad), np.nan, np.float32)
    big[:, offset:offset + cols] = a
    t = dev(torch_dev, big, dtype)
    v = t[:, offset:offset + cols]
    assert v.stride(0) == cols + pad and v.stride(1) == 1
    return v


def tied_inputs(bt, h, v, seed, wstd=0.03):
    s = bf16_round(normal((bt, h), seed))
    th = bf16_round(normal((bt, h), seed + 1))
    w = bf16_round(normal((v, h), seed + 2, wstd))
    y = uniform_labels(bt, v, seed + 3)
    return s, th, w, y


def test_separate_bf16_unaligned_teacher_width(torch_dev):
    bt, hs, ht, v = 192, 96, 100, 1500
    s, ws = bf16_round(normal((bt, hs), 81)), bf16_round(normal((v, hs), 82, 0.03))
    th, wt = bf16_round(normal((bt, ht), 83)), bf16_round(normal((v, ht), 84, 0.03))
    y = uniform_labels(bt, v, 85)
    y[::9] = -100
    opts = LossOptions(kd_weight=0.5, temperature=2.0, label_smoothing=0.1,
                       teacher_ce_weight=1.0, chunk_size=ChunkSize.Fixed(64))
    got = H.distillation_loss(dev(torch_dev, s, "bf16"), dev(torch_dev, ws, "bf16"),
                              dev(torch_dev, y),
                              Teacher.Separate(dev(torch_dev, th, "bf16"),
                                               dev(torch_dev, wt, "bf16")), opts)
    ref = O.distillation_loss(s, ws, y, Teacher.Separate(th, wt), opts)
    check_output(got, ref, kind="bf16")


@pytest.mark.parametrize("bt,hs,ht,v,chunk,w_t", [
    (192, 96, 100, 1500, 64, None),    # Ht != Hs, ragged V, two staging groups
    (257, 64, 64, 4096, None, 0.0),    # full tiles, M not a multiple of 256
    (70, 40, 24, 1003, 16, None),      # V odd: a partial last vector of 8
    (96, 64, 64, 1000, 32, 0.5),       # teacher CE: the teacher's bf16 gradient rows
    (130, 48, 72, 2050, 40, 1.0),      # teacher CE, Ht != Hs, V % 8 = 2
])
def test_separate_bf16_teacher_logits_in_the_gemm_epilogue(torch_dev, bt, hs, ht, v, chunk, w_t):
    """A Separate teacher with bf16 inputs and a KL term: the teacher's
    logits GEMM stores fp32 logits first, and the student's logits GEMM reads
    them in its epilogue (teacher statistics, label logit and KL sums) and
    stores the student logits in bf16; the row pass reads the fp32 teacher
    rows, and with teacher CE writes the teacher's gradient rows in bf16 to
    their own buffer (grad_teacher_hidden and grad_teacher_weight read them)."""
    s, ws = bf16_round(normal((bt, hs), 141)), bf16_round(normal((v, hs), 142, 0.05))
    th, wt = bf16_round(normal((bt, ht), 143)), bf16_round(normal((v, ht), 144, 0.05))
    y = uniform_labels(bt, v, 145)
    y[::7] = -100
    opts = LossOptions(kd_weight=0.6, temperature=2.5, label_smoothing=0.05, teacher_ce_weight=w_t,
                       chunk_size=ChunkSize.Auto if chunk is None else ChunkSize.Fixed(chunk))
    got = H.distillation_loss(dev(torch_dev, s, "bf16"), dev(torch_dev, ws, "bf16"),
                              dev(torch_dev, y),
                              Teacher.Separate(dev(torch_dev, th, "bf16"),
                                               dev(torch_dev, wt, "bf16")), opts, rows=True)
    ref = O.distillation_loss(s, ws, y, Teacher.Separate(th, wt), opts)
    check_output(got, ref, kind="bf16")
    keep = y != -100
    rk = got.row_kl.cpu().numpy()
    assert np.all(rk[~keep] == 0.0)
    np.testing.assert_allclose(rk[keep], ref.row_kl[keep], rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("tl_dtype,v,view", [(None, 1024, False), (None, 1001, False),
                                             ("bf16", 1024, False), (None, 1024, True)])
def test_precomputed_logits_with_bf16_hidden(torch_dev, tl_dtype, v, view):
    bt, h = 160, 64
    s, w = bf16_round(normal((bt, h), 91)), bf16_round(normal((v, h), 92, 0.03))
    y = uniform_labels(bt, v, 93)
    tl = normal((bt, v), 94, 2.0)
    tl[np.arange(bt), y] += 6.0
    if tl_dtype == "bf16":
        tl = bf16_round(tl)
    tl_dev = strided(torch_dev, tl, 8, 16, tl_dtype) if view else dev(torch_dev, tl, tl_dtype)
    opts = LossOptions(kd_weight=0.7, temperature=1.0, chunk_size=ChunkSize.Fixed(48))
    got = H.distillation_loss(dev(torch_dev, s, "bf16"), dev(torch_dev, w, "bf16"),
                              dev(torch_dev, y), Teacher.Precomputed(tl_dev), opts)
    ref = O.distillation_loss(s, w, y, Teacher.Precomputed(tl), opts)
    assert got.grad_teacher_hidden is None
    check_output(got, ref, kind="bf16")


@pytest.mark.parametrize("tl_dtype,bt,v,offset,pad,chunk,w_t", [
    (None, 160, 1004, 0, 0, 48, None),    # V % 8 = 4: a ragged last tile, a partial last vector
    (None, 300, 2052, 4, 8, 128, 0.6),    # pitch V + 8 (a multiple of 4, not 8), base 16 bytes in
    (None, 257, 4096, 8, 8, None, 0.6),   # full tiles, M not a multiple of 256
    (None, 96, 1000, 3, 5, 32, None),     # misaligned view: converted instead
    ("bf16", 160, 1000, 0, 0, 48, None),  # bf16 logits: a ragged last tile
    ("bf16", 300, 2056, 8, 8, 128, 0.6),  # bf16, pitch V + 8, base 16 bytes in
    ("bf16", 257, 4096, 0, 0, None, 0.6), # bf16, full tiles
    ("bf16", 96, 1004, 0, 0, 32, None),   # bf16 at a pitch of 4 mod 8: converted instead
])
def test_precomputed_logits_in_the_bf16_gemm_epilogue(torch_dev, tl_dtype, bt, v, offset, pad,
                                                      chunk, w_t):
    """Precomputed logits beside bf16 hidden states with a KL term, fp32 at a
    pitch of a multiple of 4 or bf16 at a multiple of 8, 16-byte aligned: the
    logits GEMM reads each tile's teacher logits in its epilogue (teacher
    statistics, label logit and KL sums there), the student logits are
    stored in bf16 and the row pass reads the teacher rows in place. Ignored
    rows, label smoothing, T != 1, the teacher CE term and views with their
    own pitch; a view that is not 16-byte aligned and bf16 logits at a pitch
    of 4 mod 8 are converted into staging instead (the oracle is fed the same
    bf16-rounded logits)."""
    h = 96
    s, w = bf16_round(normal((bt, h), 131)), bf16_round(normal((v, h), 132, 0.03))
    y = uniform_labels(bt, v, 133)
    y[::11] = -100
    tl = normal((bt, v), 134, 2.0)
    tl[np.arange(bt), np.maximum(y, 0)] += 4.0
    if tl_dtype == "bf16":
        tl = bf16_round(tl)
    tl_dev = strided(torch_dev, tl, offset, pad, tl_dtype) if pad else dev(torch_dev, tl, tl_dtype)
    opts = LossOptions(kd_weight=0.7, temperature=1.7, label_smoothing=0.1, teacher_ce_weight=w_t,
                       chunk_size=ChunkSize.Auto if chunk is None else ChunkSize.Fixed(chunk))
    got = H.distillation_loss(dev(torch_dev, s, "bf16"), dev(torch_dev, w, "bf16"),
                              dev(torch_dev, y), Teacher.Precomputed(tl_dev), opts, rows=True)
    ref = O.distillation_loss(s, w, y, Teacher.Precomputed(tl), opts)
    assert got.grad_teacher_hidden is None
    check_output(got, ref, kind="bf16")
    keep = y != -100
    rk = got.row_kl.cpu().numpy()
    assert np.all(rk[~keep] == 0.0)
    np.testing.assert_allclose(rk[keep], ref.row_kl[keep], rtol=1e-4, atol=1e-6)
    if w_t:
        rt = got.row_nll_teacher.cpu().numpy()
        np.testing.assert_allclose(rt[keep], ref.row_nll_teacher[keep], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("h", [100, 13])
def test_tied_bf16_hidden_width_not_multiple_of_8(torch_dev, h):
    bt, v = 144, 999
    s, th, w, y = tied_inputs(bt, h, v, 101)
    opts = LossOptions(kd_weight=0.4, temperature=1.5, label_smoothing=0.1,
                       teacher_ce_weight=1.0, chunk_size=ChunkSize.Fixed(64))
    got = H.distillation_loss(dev(torch_dev, s, "bf16"), dev(torch_dev, w, "bf16"),
                              dev(torch_dev, y), Teacher.Tied(dev(torch_dev, th, "bf16")), opts)
    ref = O.distillation_loss(s, w, y, Teacher.Tied(th), opts)
    check_output(got, ref, kind="bf16")


@pytest.mark.parametrize("dtype", [None, "bf16"])
@pytest.mark.parametrize("offset", [8, 3])
def test_strided_device_views(torch_dev, dtype, offset):
    """offset 8 keeps every row 16-byte aligned (inputs used in place),
    offset 3 does not (inputs staged into packed copies)."""
    bt, h, v = 128, 64, 1200
    s, th, w, y = tied_inputs(bt, h, v, 111)
    opts = LossOptions(kd_weight=0.4, temperature=1.5, teacher_ce_weight=1.0,
                       chunk_size=ChunkSize.Fixed(32))
    got = H.distillation_loss(strided(torch_dev, s, offset, 16, dtype),
                              strided(torch_dev, w, offset, 16, dtype), dev(torch_dev, y),
                              Teacher.Tied(strided(torch_dev, th, offset, 16, dtype)), opts)
    ref = O.distillation_loss(s, w, y, Teacher.Tied(th), opts)
    check_output(got, ref, kind="bf16" if dtype else "f32")


@pytest.mark.parametrize("bt,chunk", [(37, None), (203, 70)])
def test_paired_rows_not_multiple_of_16(torch_dev, bt, chunk):
    h, v = 64, 500
    s, th, w, y = tied_inputs(bt, h, v, 121)
    y[::5] = -100
    cs = ChunkSize.Fixed(chunk) if chunk else ChunkSize.Auto
    opts = LossOptions(kd_weight=0.4, temperature=1.5, label_smoothing=0.1, chunk_size=cs)
    got = H.distillation_loss(dev(torch_dev, s, "bf16"), dev(torch_dev, w, "bf16"),
                              dev(torch_dev, y), Teacher.Tied(dev(torch_dev, th, "bf16")), opts)
    ref = O.distillation_loss(s, w, y, Teacher.Tied(th), opts)
    check_output(got, ref, kind="bf16")


@pytest.mark.parametrize("dtype", [None, "bf16"])
@pytest.mark.parametrize("temperature,alpha", [(0.25, 0.1), (8.0, 0.1), (1.5, 1.0)])
def test_temperature_and_smoothing_extremes(torch_dev, dtype, temperature, alpha):
    bt, h, v = 192, 64, 2000
    s, th, w, y = tied_inputs(bt, h, v, 131, wstd=0.1)
    opts = LossOptions(kd_weight=0.6, temperature=temperature, label_smoothing=alpha,
                       teacher_ce_weight=1.0, chunk_size=ChunkSize.Fixed(64))
    got = H.distillation_loss(dev(torch_dev, s, dtype), dev(torch_dev, w, dtype),
                              dev(torch_dev, y), Teacher.Tied(dev(torch_dev, th, dtype)), opts)
    ref = O.distillation_loss(s, w, y, Teacher.Tied(th), opts)
    check_output(got, ref, kind="bf16" if dtype else "f32")


@pytest.mark.parametrize("dtype", [None, "bf16"])
def test_stochastic_int8_through_the_path(torch_dev, dtype):
    """Stochastic rounding draws one SplitMix64 number per grad_W element in
    row-major order (src/quant.rs:120-144). fp32: codes within ±1 of the
    oracle's and target rows exact; bf16: the dequantized grad_W within the
    bf16 gradient tolerance (its codes follow bf16-rounded gradients)."""
    bt, h, v = 256, 64, 1500
    s, th, w, y = tied_inputs(bt, h, v, 141)
    if dtype is None:
        s, th, w = normal((bt, h), 141), normal((bt, h), 142), normal((v, h), 143, 0.03)
    cfg = KernelConfig(quantize_grad_weight=True, stochastic_rounding=True, stochastic_seed=987)
    opts = LossOptions(kd_weight=0.4, temperature=1.5, label_smoothing=0.1, config=cfg,
                       chunk_size=ChunkSize.Fixed(64))
    args = (dev(torch_dev, s, dtype), dev(torch_dev, w, dtype), dev(torch_dev, y),
            Teacher.Tied(dev(torch_dev, th, dtype)))
    got = H.distillation_loss(*args, opts, quant_codes=True)
    plain_opts = LossOptions(kd_weight=0.4, temperature=1.5, label_smoothing=0.1,
                             chunk_size=ChunkSize.Fixed(64))
    plain = H.distillation_loss(*args, plain_opts)
    check_quant_of_own_gradient(got, plain.grad_weight, y, stochastic=True, seed=987)
    ref = O.distillation_loss(s, w, y, Teacher.Tied(th), opts)
    if dtype is None:
        ref_plain = O.distillation_loss(s, w, y, Teacher.Tied(th), plain_opts)
        check_output(got, ref, skip_grad_weight=True)
        check_quantized_grad_weight(got, ref, y, plain.grad_weight, ref_plain.grad_weight,
                                    stochastic=True, seed=987)
    else:
        check_output(got, ref, kind="bf16", skip_grad_weight=True)
        check_grad("grad_weight (dequantized)", to_np(got.grad_weight), ref.grad_weight, "bf16")


EMPTY_CASES = [
    # mode, dtype, H, Ht (Separate), V, inputs on the host, INT8 grad_W
    ("tied", None, 0, None, 9, False, False),
    ("tied", "bf16", 0, None, 9, False, True),
    ("tied", None, 6, None, 0, False, True),
    ("tied", None, 0, None, 0, True, False),
    ("tied", None, 0, None, 9, True, True),
    ("separate", None, 0, 5, 9, False, False),
    ("separate", "bf16", 6, 0, 9, False, False),
    ("separate", None, 6, 0, 9, True, False),
    ("separate", None, 6, 5, 0, False, False),
    ("precomputed", None, 0, None, 9, False, False),
    ("precomputed", "bf16", 0, None, 9, False, True),
    ("precomputed", None, 6, None, 0, False, False),
]


@pytest.mark.parametrize("mode,dtype,h,ht,v,host,quant", EMPTY_CASES,
                         ids=[f"{c[0]}-{c[1] or 'f32'}-h{c[2]}" + (f"-ht{c[3]}" if c[3] is not None else "")
                              + f"-v{c[4]}" + ("-host" if c[5] else "") + ("-int8" if c[6] else "")
                              for c in EMPTY_CASES])
def test_empty_hidden_width_or_vocabulary(torch_dev, mode, dtype, h, ht, v, host, quant):
    """H = 0 gives logits of exactly 0 (every CE term log V, the Tied KL 0)
    and gradients with no columns; V = 0 leaves only ignored rows (every
    term 0, grad_hidden 0, grad_W with no rows); with INT8, rows of no
    columns keep the scale of an all-zero row (src/quant.rs:52-57). All
    against the oracle, including the per-row losses."""
    bt = 5
    rnd = bf16_round if dtype == "bf16" else (lambda a: a)
    s = rnd(normal((bt, h), 311))
    w = rnd(normal((v, h), 312, 0.1))
    y = uniform_labels(bt, v, 313) if v > 0 else np.full(bt, -100, np.int64)
    if mode == "tied":
        t = Teacher.Tied(rnd(normal((bt, h), 314)))
    elif mode == "separate":
        t = Teacher.Separate(rnd(normal((bt, ht), 315)), rnd(normal((v, ht), 316, 0.1)))
    else:
        t = Teacher.Precomputed(normal((bt, v), 317, 2.0))
    cfg = KernelConfig(quantize_grad_weight=quant)
    opts = LossOptions(kd_weight=0.5, temperature=1.5, label_smoothing=0.1,
                       teacher_ce_weight=None if mode == "precomputed" else 0.7, config=cfg)
    print(f"case {mode} {dtype} h={h} ht={ht} v={v} host={host} quant={quant}", flush=True)
    if host:
        args = (s, w, y, t)
    else:
        if mode == "tied":
            tg = Teacher.Tied(dev(torch_dev, t.hidden, dtype))
        elif mode == "separate":
            tg = Teacher.Separate(dev(torch_dev, t.hidden, dtype), dev(torch_dev, t.weight, dtype))
        else:
            tg = Teacher.Precomputed(dev(torch_dev, t.logits))
        args = (dev(torch_dev, s, dtype), dev(torch_dev, w, dtype), dev(torch_dev, y), tg)
    got = H.distillation_loss(*args, opts, rows=True, quant_codes=quant)
    ref = O.distillation_loss(s, w, y, t, opts)
    check_output(got, ref, kind="bf16" if dtype else "f32")
    for k in ("row_nll_student", "row_nll_teacher", "row_kl"):
        np.testing.assert_allclose(to_np(getattr(got, k)).reshape(-1), getattr(ref, k),
                                   rtol=1e-4, atol=2e-6, err_msg=k)
    if h == 0 and v > 0:
        assert abs(got.student_ce - np.log(v)) <= 1e-5 * np.log(v)
    if v == 0:
        assert got.loss == 0.0 and np.all(to_np(got.grad_student_hidden) == 0.0)
    if quant:
        assert to_np(got.quant_codes).shape == (v, h)
        np.testing.assert_array_equal(to_np(got.quant_scales).reshape(-1), ref.quant_scales)
        np.testing.assert_array_equal(to_np(got.quant_codes), ref.quant_codes)
