"""GPU parity: liborda_hip.so (through the C ABI) against the CPU oracle on
identical seeded inputs. Tolerances are stated in tests/parity.py.

Cases: the reference's own end-to-end cases (tests/end_to_end.rs, tiny odd
shapes that exercise every tail and padding path), the Tied
256/512/8192 fp32 shape in full, and reduced versions of the four larger
shapes (same mode, dtype and options; sizes the oracle finishes in seconds).
"""
import dataclasses

import numpy as np
import pytest

import oracle as O
from helpers import bf16_round, labels, mat, normal, uniform_labels
from parity import (check_grad, check_output, check_quant_of_own_gradient,
                    check_quantized_grad_weight, check_scalar, to_np)

import orda_hip as H
from orda_hip import (ChunkSize, KernelConfig, LossOptions, OrdaError, Reduction, Teacher)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    assert H.is_available(), "liborda_hip.so does not see a gfx950 device"
    return torch, torch.device("cuda:0")


def gpu(torch_dev, a, dtype=None):
    torch, dev = torch_dev
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    if dtype == "bf16":
        t = t.to(torch.bfloat16)
    return t


def gpu_teacher(torch_dev, teacher, dtype=None):
    m = teacher.mode()
    if m == H.TeacherMode.Tied:
        return Teacher.Tied(gpu(torch_dev, teacher.hidden, dtype))
    if m == H.TeacherMode.Separate:
        return Teacher.Separate(gpu(torch_dev, teacher.hidden, dtype),
                                gpu(torch_dev, teacher.weight, dtype))
    return Teacher.Precomputed(gpu(torch_dev, teacher.logits))


def run_pair(torch_dev, s, w, y, teacher, opts, dtype=None):
    """(gpu output, oracle output); bf16 runs feed the oracle the rounded values."""
    if dtype == "bf16":
        s, w = bf16_round(s), bf16_round(w)
        if teacher.hidden is not None:
            teacher = Teacher(teacher.mode(), hidden=bf16_round(teacher.hidden),
                              weight=None if teacher.weight is None else bf16_round(teacher.weight),
                              logits=teacher.logits)
    got = H.distillation_loss(gpu(torch_dev, s, dtype), gpu(torch_dev, w, dtype),
                              gpu(torch_dev, y), gpu_teacher(torch_dev, teacher, dtype), opts,
                              rows=True, quant_codes=True)
    ref = O.distillation_loss(s, w, y, teacher, opts)
    return got, ref


def base_opts(**kw):
    d = dict(student_ce_weight=1.0, kd_weight=0.5, temperature=1.5)
    d.update(kw)
    return LossOptions(**d)


def quant_off(opts):
    """The same options with quantize_grad_weight off."""
    return dataclasses.replace(opts, config=dataclasses.replace(opts.config,
                                                                quantize_grad_weight=False))


def int8_runs(torch_dev, s, w, y, teacher, opts, dtype=None):
    """The quantized call and the same call with quantization off, on the GPU
    and in the oracle: (got, ref, got_plain, ref_plain)."""
    got, ref = run_pair(torch_dev, s, w, y, teacher, opts, dtype)
    got_plain, ref_plain = run_pair(torch_dev, s, w, y, teacher, quant_off(opts), dtype)
    return got, ref, got_plain, ref_plain


# ------------------------------------------------ reference end-to-end cases
def test_tied_small(torch_dev):
    bt, h, v = 6, 5, 7
    got, ref = run_pair(torch_dev, mat(bt, h, 1, 0.3), mat(v, h, 2, 0.2), labels(bt, v, 4),
                        Teacher.Tied(mat(bt, h, 3, 0.3)),
                        base_opts(teacher_ce_weight=1.0, label_smoothing=0.1))
    check_output(got, ref)


def test_separate_small(torch_dev):
    bt, h, ht, v = 6, 5, 4, 7
    got, ref = run_pair(torch_dev, mat(bt, h, 11, 0.3), mat(v, h, 12, 0.2), labels(bt, v, None),
                        Teacher.Separate(mat(bt, ht, 13, 0.3), mat(v, ht, 14, 0.2)),
                        base_opts(teacher_ce_weight=0.7))
    check_output(got, ref)


def test_precomputed_small(torch_dev):
    bt, h, v = 6, 5, 7
    got, ref = run_pair(torch_dev, mat(bt, h, 21, 0.3), mat(v, h, 22, 0.2), labels(bt, v, 5),
                        Teacher.Precomputed(mat(bt, v, 23, 0.5)), base_opts())
    assert got.grad_teacher_hidden is None and got.grad_teacher_weight is None
    check_output(got, ref)


def test_pure_student_small(torch_dev):
    bt, h, v = 8, 4, 6
    got, ref = run_pair(torch_dev, mat(bt, h, 31, 0.3), mat(v, h, 32, 0.2), labels(bt, v, None),
                        Teacher.Tied(np.zeros((bt, h), np.float32)),
                        LossOptions(kd_weight=0.0, teacher_ce_weight=0.0))
    assert got.teacher_ce == 0.0 and got.kl == 0.0
    check_output(got, ref)


@pytest.mark.parametrize("cs", [ChunkSize.Fixed(16), ChunkSize.Fixed(1), ChunkSize.Fixed(3),
                                ChunkSize.Auto])
def test_chunking_small(torch_dev, cs):
    bt, h, v = 16, 5, 9
    got, ref = run_pair(torch_dev, mat(bt, h, 41, 0.3), mat(v, h, 42, 0.2), labels(bt, v, 3),
                        Teacher.Tied(mat(bt, h, 43, 0.3)),
                        base_opts(chunk_size=cs, teacher_ce_weight=1.0))
    check_output(got, ref)


def test_sum_reduction_small(torch_dev):
    bt, h, v = 8, 4, 6
    got, ref = run_pair(torch_dev, mat(bt, h, 61, 0.3), mat(v, h, 62, 0.2), labels(bt, v, 4),
                        Teacher.Tied(mat(bt, h, 63, 0.3)),
                        base_opts(reduction=Reduction.Sum, teacher_ce_weight=1.0))
    check_output(got, ref)


def test_int8_small(torch_dev):
    bt, h, v = 8, 4, 20
    y = labels(bt, v, None)
    got, ref, plain, ref_plain = int8_runs(
        torch_dev, mat(bt, h, 71, 0.3), mat(v, h, 72, 0.2), y, Teacher.Tied(mat(bt, h, 73, 0.3)),
        base_opts(teacher_ce_weight=1.0, config=KernelConfig(quantize_grad_weight=True)))
    check_output(got, ref, skip_grad_weight=True)
    check_quantized_grad_weight(got, ref, y, plain.grad_weight, ref_plain.grad_weight)
    check_quant_of_own_gradient(got, plain.grad_weight, y)


@pytest.mark.parametrize("stochastic", [False, True])
def test_int8_fp32_gate(torch_dev, stochastic):
    """The INT8 clause of the gate end to end on an fp32 multi-chunk Tied
    run with smoothing and ignored labels: codes, scales and the returned
    grad_W are those of quantizing the call's own fp32 grad_W (the same call
    with quantization off), and against the oracle the scales agree to 1e-5
    relative and a code differs (by 1) only where the two fp32 gradients
    straddle a rounding boundary (src/api.rs:380-399, src/quant.rs:91-202)."""
    bt, h, v = 512, 128, 3000
    s, th = normal((bt, h), 201), normal((bt, h), 202)
    w = normal((v, h), 203, 0.03)
    y = uniform_labels(bt, v, 204)
    y[::7] = -100
    seed = 4242 if stochastic else 0
    cfg = KernelConfig(quantize_grad_weight=True, stochastic_rounding=stochastic,
                       stochastic_seed=seed if stochastic else None)
    opts = LossOptions(kd_weight=0.4, temperature=1.5, label_smoothing=0.1, config=cfg,
                       chunk_size=ChunkSize.Fixed(128))
    got, ref, plain, ref_plain = int8_runs(torch_dev, s, w, y, Teacher.Tied(th), opts)
    check_output(got, ref, skip_grad_weight=True)
    flips = check_quantized_grad_weight(got, ref, y, plain.grad_weight, ref_plain.grad_weight,
                                        stochastic=stochastic, seed=seed)
    check_quant_of_own_gradient(got, plain.grad_weight, y, stochastic=stochastic, seed=seed)
    print(f"codes differing from the oracle at rounding boundaries: {flips} of {v * h}")


# ------------------------------------------------ benchmark-shape cases
def test_tied_256_512_8192_fp32(torch_dev):
    """Tied 256/512/8192 fp32, kd 0.4, T 1.5, no smoothing, mean, Auto chunks."""
    bt, h, v = 256, 512, 8192
    s, th = normal((bt, h), 1), normal((bt, h), 2)
    w = normal((v, h), 3, 0.02)
    y = uniform_labels(bt, v, 5)
    got, ref = run_pair(torch_dev, s, w, y, Teacher.Tied(th),
                        LossOptions(kd_weight=0.4, temperature=1.5))
    check_output(got, ref)
    assert (got.chunk_plan.chunk_size, got.chunk_plan.num_chunks) == (256, 1)
    np.testing.assert_allclose(to_np(got.row_nll_student), ref.row_nll_student, rtol=1e-4)
    np.testing.assert_allclose(to_np(got.row_kl), ref.row_kl, rtol=1e-3, atol=1e-5)


def test_tied_reduced_fp32_multichunk(torch_dev):
    """Tied fp32 at a reduced shape with a non-power-of-two vocabulary and
    four chunks (one backward group)."""
    bt, h, v = 512, 256, 3200
    s, th = normal((bt, h), 11), normal((bt, h), 12)
    w = normal((v, h), 13, 0.02)
    y = uniform_labels(bt, v, 15)
    got, ref = run_pair(torch_dev, s, w, y, Teacher.Tied(th),
                        LossOptions(kd_weight=0.4, temperature=1.5,
                                    chunk_size=ChunkSize.Fixed(128)))
    check_output(got, ref)


def test_separate_reduced_fp32(torch_dev):
    """Separate teacher: Hs != Ht, kd 0.5, T 2, smoothing 0.1, teacher CE weight 1."""
    bt, hs, ht, v = 256, 128, 256, 3000
    s = normal((bt, hs), 21)
    ws = normal((v, hs), 22, 0.02)
    th = normal((bt, ht), 23)
    wt = normal((v, ht), 24, 0.015)
    y = uniform_labels(bt, v, 25)
    got, ref = run_pair(torch_dev, s, ws, y, Teacher.Separate(th, wt),
                        LossOptions(kd_weight=0.5, temperature=2.0, label_smoothing=0.1,
                                    teacher_ce_weight=1.0, chunk_size=ChunkSize.Fixed(64)))
    check_output(got, ref)


def test_separate_default_teacher_weight(torch_dev):
    """Separate with the default teacher-CE weight 0: no teacher gradients."""
    bt, hs, ht, v = 128, 64, 96, 1000
    got, ref = run_pair(torch_dev, normal((bt, hs), 1), normal((v, hs), 2, 0.05),
                        uniform_labels(bt, v, 3),
                        Teacher.Separate(normal((bt, ht), 4), normal((v, ht), 5, 0.05)),
                        LossOptions(kd_weight=0.5, temperature=2.0))
    assert got.grad_teacher_hidden is None and got.grad_teacher_weight is None
    check_output(got, ref)


def test_precomputed_reduced_fp32(torch_dev):
    """Precomputed peaked teacher: N(0, 2²) + 8 at the label, kd 0.7, T 1."""
    bt, h, v = 256, 256, 4096
    s = normal((bt, h), 31)
    w = normal((v, h), 32, 0.02)
    y = uniform_labels(bt, v, 35)
    tl = normal((bt, v), 36, 2.0)
    tl[np.arange(bt), y] += 8.0
    got, ref = run_pair(torch_dev, s, w, y, Teacher.Precomputed(tl),
                        LossOptions(kd_weight=0.7, temperature=1.0,
                                    chunk_size=ChunkSize.Fixed(64)))
    check_output(got, ref)


def test_tied_reduced_bf16_int8(torch_dev):
    """bf16 inputs (fp32 accumulation), kd 0.4, T 1.5, smoothing 0.1, INT8 grad_W."""
    bt, h, v = 512, 256, 4096
    s, th = normal((bt, h), 41), normal((bt, h), 42)
    w = normal((v, h), 43, 0.02)
    y = uniform_labels(bt, v, 45)
    opts = LossOptions(kd_weight=0.4, temperature=1.5, label_smoothing=0.1,
                       chunk_size=ChunkSize.Fixed(128),
                       config=KernelConfig(quantize_grad_weight=True))
    got, ref, plain, _ = int8_runs(torch_dev, s, w, y, Teacher.Tied(th), opts, dtype="bf16")
    check_output(got, ref, kind="bf16", skip_grad_weight=True)
    gw, rw = to_np(got.grad_weight), ref.grad_weight
    check_grad("grad_weight (dequantized)", gw, rw, "bf16")
    # the quant step itself is exact on the call's own fp32 grad_W
    check_quant_of_own_gradient(got, plain.grad_weight, y)


@pytest.mark.parametrize("bt,h,v,chunk", [(300, 224, 1000, 200), (96, 112, 1064, 48)])
def test_tied_bf16_k_tails(torch_dev, bt, h, v, chunk):
    """bf16 GEMMs whose K (H for the logits, V for grad_hidden, chunk rows
    for grad_W) is a whole number of 64-element stage pairs followed by an
    odd 32-element stage and a ragged rest, with teacher CE so that every
    product runs on both halves."""
    s, th = normal((bt, h), 61), normal((bt, h), 62)
    w = normal((v, h), 63, 0.03)
    y = uniform_labels(bt, v, 65)
    opts = LossOptions(kd_weight=0.4, temperature=1.5, label_smoothing=0.1,
                       teacher_ce_weight=0.5, chunk_size=ChunkSize.Fixed(chunk))
    got, ref = run_pair(torch_dev, s, w, y, Teacher.Tied(th), opts, dtype="bf16")
    check_output(got, ref, kind="bf16")


@pytest.mark.parametrize("dtype", [None, "bf16"])
def test_multi_group_split_k(torch_dev, dtype):
    """A staging budget of one chunk runs four groups, so grad_W accumulates
    across groups; with V=2000 and H=64 both backward GEMMs have fewer tiles
    than CUs and split K (grad_W over 2048 rows in 4 splits, then the
    accumulating reduction)."""
    bt, h, v = 4096, 64, 2000
    s, th = normal((bt, h), 71), normal((bt, h), 72)
    w = normal((v, h), 73, 0.05)
    y = uniform_labels(bt, v, 74)
    y[::11] = -100
    opts = LossOptions(kd_weight=0.4, temperature=1.5, label_smoothing=0.1,
                       chunk_size=ChunkSize.Fixed(1024))
    if dtype == "bf16":
        s, th, w = bf16_round(s), bf16_round(th), bf16_round(w)
    ctx = H.Context(0)
    ctx.set_staging_budget(1)   # one chunk per group
    got = H.distillation_loss(gpu(torch_dev, s, dtype), gpu(torch_dev, w, dtype),
                              gpu(torch_dev, y), Teacher.Tied(gpu(torch_dev, th, dtype)), opts,
                              ctx=ctx)
    ref = O.distillation_loss(s, w, y, Teacher.Tied(th), opts)
    check_output(got, ref, kind="bf16" if dtype else "f32")
    ctx.close()


@pytest.mark.parametrize("mode", ["separate", "precomputed"])
def test_multi_group_bf16_teacher_logits_beside_gemm(torch_dev, mode):
    """bf16 inputs with a Separate teacher (teacher CE on) or fp32
    Precomputed logits, whose fp32 logits the student's logits GEMM reads in
    its epilogue, over four staging groups of one chunk: the teacher logits
    buffer (Separate) or the caller's logits (Precomputed, at each group's
    row offset) and the teacher gradient rows are reused or offset per
    group, and grad_W and grad_teacher_weight accumulate across groups."""
    bt, h, ht, v = 1024, 64, 96, 2000
    s = bf16_round(normal((bt, h), 75))
    w = bf16_round(normal((v, h), 76, 0.05))
    y = uniform_labels(bt, v, 77)
    y[::9] = -100
    if mode == "separate":
        th, tw = bf16_round(normal((bt, ht), 78)), bf16_round(normal((v, ht), 79, 0.05))
        tg = Teacher.Separate(gpu(torch_dev, th, "bf16"), gpu(torch_dev, tw, "bf16"))
        to = Teacher.Separate(th, tw)
        w_t = 0.6
    else:
        tl = normal((bt, v), 78, 2.0)
        tg, to = Teacher.Precomputed(gpu(torch_dev, tl)), Teacher.Precomputed(tl)
        w_t = None
    opts = LossOptions(kd_weight=0.5, temperature=1.3, label_smoothing=0.1, teacher_ce_weight=w_t,
                       chunk_size=ChunkSize.Fixed(256))
    ctx = H.Context(0)
    ctx.set_staging_budget(1)   # one chunk per group
    ctx.set_timing(True)
    got = H.distillation_loss(gpu(torch_dev, s, "bf16"), gpu(torch_dev, w, "bf16"),
                              gpu(torch_dev, y), tg, opts, ctx=ctx)
    _, groups = ctx.kernel_time("row_pass")
    ref = O.distillation_loss(s, w, y, to, opts)
    check_output(got, ref, kind="bf16")
    assert groups == 4, groups
    ctx.close()


def test_ignored_labels_and_reductions(torch_dev):
    bt, h, v = 200, 64, 777
    s, th = normal((bt, h), 51), normal((bt, h), 52)
    w = normal((v, h), 53, 0.1)
    y = uniform_labels(bt, v, 54)
    y[::3] = -7
    for red in (Reduction.Mean, Reduction.Sum):
        got, ref = run_pair(torch_dev, s, w, y, Teacher.Tied(th),
                            LossOptions(kd_weight=0.3, temperature=0.7, label_smoothing=0.2,
                                        ignore_index=-7, reduction=red,
                                        chunk_size=ChunkSize.Fixed(48)))
        check_output(got, ref)
        assert np.all(to_np(got.row_nll_student)[::3] == 0.0)


def test_all_labels_ignored(torch_dev):
    bt, h, v = 32, 16, 50
    y = np.full(bt, -100)
    got, ref = run_pair(torch_dev, normal((bt, h), 1), normal((v, h), 2, 0.1), y,
                        Teacher.Tied(normal((bt, h), 3)), LossOptions(kd_weight=0.5))
    check_output(got, ref)
    assert got.loss == 0.0 and np.all(to_np(got.grad_weight) == 0.0)


def test_inputs_from_pending_default_stream_work(torch_dev):
    """Inputs whose producing kernels are still queued on torch's default
    stream (the null stream, handle NULL) when the call starts. The call runs
    on the context's own stream, which must be ordered after them: the labels
    are read back for validation and every input is read by the kernels."""
    torch, dev = torch_dev
    assert torch.cuda.current_stream(dev).cuda_stream == 0
    bt, h, v = 256, 64, 1000
    s, th = normal((bt, h), 151), normal((bt, h), 152)
    w = normal((v, h), 153, 0.05)
    y = uniform_labels(bt, v, 154)
    y[::9] = -100
    # ~60 ms of queued work ending in an exact zero that every input depends on
    a = torch.full((4096, 4096), 1e-3, device=dev)
    for _ in range(40):
        a = torch.tanh(a @ a)
    zf = a[0, 0] * 0.0
    zi = zf.to(torch.int64)
    opts = base_opts(teacher_ce_weight=1.0, label_smoothing=0.1, chunk_size=ChunkSize.Fixed(64))
    got = H.distillation_loss(gpu(torch_dev, s) + zf, gpu(torch_dev, w) + zf,
                              gpu(torch_dev, y) + zi, Teacher.Tied(gpu(torch_dev, th) + zf), opts)
    ref = O.distillation_loss(s, w, y, Teacher.Tied(th), opts)
    check_output(got, ref)


def test_concurrent_calls_from_two_threads(torch_dev):
    """Two Python threads in the library at once (ctypes releases the GIL
    for the call): each thread's default context has its own stream and
    workspace, and every result matches the oracle."""
    import threading
    torch, dev = torch_dev
    cases = []
    for k in range(2):
        bt, h, v = 192 + 64 * k, 64, 1500 + 500 * k
        cases.append((normal((bt, h), 160 + k), normal((bt, h), 170 + k),
                      normal((v, h), 180 + k, 0.05), uniform_labels(bt, v, 190 + k)))
    opts = base_opts(teacher_ce_weight=1.0, label_smoothing=0.1, chunk_size=ChunkSize.Fixed(64))
    got, errors = [None, None], []
    start = threading.Barrier(2)

    def run(k):
        try:
            s, th, w, y = cases[k]
            args = (gpu(torch_dev, s), gpu(torch_dev, w), gpu(torch_dev, y),
                    Teacher.Tied(gpu(torch_dev, th)))
            torch.cuda.synchronize()
            start.wait()
            outs = [H.distillation_loss(*args, opts) for _ in range(5)]
            got[k] = (outs, H.default_context(0))
        except BaseException as e:   # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=run, args=(k,)) for k in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    assert got[0][1] is not got[1][1] and got[0][1] is not H.default_context(0)
    for k in range(2):
        s, th, w, y = cases[k]
        ref = O.distillation_loss(s, w, y, Teacher.Tied(th), opts)
        for out in got[k][0]:
            check_output(out, ref)


# ------------------------------------------------ entry points and host logic
@pytest.mark.parametrize("stochastic", [False, True])
@pytest.mark.parametrize("cols", [257, 256, 1000, 4096, 8192])
def test_quant_entry_point_bit_exact(torch_dev, stochastic, cols):
    """orda_quant_rows_int8 on the same fp32 matrix as the oracle: codes,
    scales and the dequantized matrix are identical (quant.rs:96-202). The
    column counts cover the one-read register path (multiples of 4 up to
    8192, one to eight float4 per thread, the last partly filled) and the
    two-pass path (257)."""
    rows = 300 if cols <= 1000 else 64
    rng = np.random.default_rng(9)
    m = (rng.standard_normal((rows, cols)) * rng.uniform(0.001, 3, (rows, 1))).astype(np.float32)
    m[5] = 0.0
    m[7, :10] = [0.5, 1.5, 2.5, -0.5, -1.5, 127, -127, 63.5, -63.5, 0.0]
    targets = np.array([3, 3, 17, -100, rows - 1, 0])
    out, q, s = H.quant_rows_int8(gpu(torch_dev, m), gpu(torch_dev, targets), -100, stochastic,
                                  seed=12345)
    rout, rq, rs = O.quant_dequant_grad_w(m, targets, -100, stochastic, 12345)
    np.testing.assert_array_equal(to_np(q), rq)
    np.testing.assert_array_equal(to_np(s), rs)
    np.testing.assert_array_equal(to_np(out), rout)
    # in place: kept target rows are left as they are, the rest dequantized
    g = gpu(torch_dev, m)
    H.quant_rows_int8(g, gpu(torch_dev, targets), -100, stochastic, seed=12345, out=g)
    np.testing.assert_array_equal(to_np(g), rout)


def test_kl_ce_chunk_entry_point(torch_dev):
    """The chunk launcher slot (src/cuda/launch.rs:51-158) against kl_chunk
    and ce_fwdbwd_row."""
    n, v = 24, 1003
    rng = np.random.default_rng(4)
    lc = (rng.standard_normal((2 * n, v)) * 2).astype(np.float32)
    y = rng.integers(0, v, n).astype(np.int32)
    y[::5] = -100
    T, kd, ws_, wt_, ls = 1.5, 0.4, 1.0, 0.8, 0.1
    for student_only in (False, True):
        got = H.kl_ce_on_logits_chunk(gpu(torch_dev, lc), gpu(torch_dev, y), n, 1.0 / T,
                                      kd * T, T * T, ws_, wt_, ls, -100, student_only, True)
        kl, gkl = O.kl_chunk(lc, y.astype(np.int64), n, kd, T, -100, 1.0, True)
        check_grad("grad_kl_student", got["grad_kl_student"], gkl)
        rows = n if student_only else 2 * n
        for r in range(rows):
            scale = ws_ if r < n else wt_
            nll, g = O.ce_fwdbwd_row(lc[r], int(y[r % n]), -100, ls, scale)
            check_scalar(f"ce_loss[{r}]", float(to_np(got["ce_loss"])[r]), nll)
            check_grad(f"grad_ce[{r}]", to_np(got["grad_ce"])[r], g)
        check_scalar("sum kl_per_row", float(np.sum(to_np(got["kl_per_row"]), dtype=np.float64)), kl)


def test_validation_errors_match_reference(torch_dev):
    s = gpu(torch_dev, mat(4, 3, 1, 0.3))
    w = gpu(torch_dev, mat(5, 3, 2, 0.2))
    t = Teacher.Tied(gpu(torch_dev, mat(4, 3, 3, 0.3)))
    cases = [
        (np.array([0, 1, 5, 2]), LossOptions(), "label 5 out of range [0, 5) and != ignore_index -100"),
        (np.array([0, 1, 2]), LossOptions(), "labels must have length BT=4, got 3"),
        (np.array([0, 1, 2, 3]), LossOptions(label_smoothing=1.5), "label_smoothing must be in [0,1], got 1.5"),
        (np.array([0, 1, 2, 3]), LossOptions(temperature=0.0), "temperature must be > 0, got 0"),
        (np.array([0, 1, 2, 3]), LossOptions(kd_weight=-1.0), "kd_weight must be >= 0, got -1"),
        (np.array([0, 1, 2, 3]), LossOptions(teacher_ce_weight=-0.5), "teacher_ce_weight must be >= 0, got -0.5"),
    ]
    for y, o, msg in cases:
        with pytest.raises(OrdaError) as e:
            H.distillation_loss(s, w, y, t, o)
        assert str(e.value) == msg
        with pytest.raises(O.OracleError) as e2:
            O.distillation_loss(to_np(s), to_np(w), y, Teacher.Tied(to_np(t.hidden)), o)
        assert str(e2.value) == msg


# Device bytes one staged chunk row takes at this fp32 Tied shape with teacher
# CE: student and teacher logits rows (pitch 20032), the per-256-column tile
# statistics and label logits of both rows, and the two hidden rows that
# grad_W multiplies ([h_s; h_t]).
def _tied_f32_row_bytes(h, v):
    pitch = (v + 63) // 64 * 64
    pitch += 64 if pitch % 1024 == 0 else 0
    return 2 * pitch * 4 + 2 * ((v + 255) // 256) * 16 + 2 * 4 + 2 * ((h + 7) // 8 * 8) * 4


def _split_k_bytes(m, n, k, nprob, trans=False):
    """fp32 partial bytes of a backward GEMM that splits K (the library's
    policy: about 256 workgroups, at least 128 elements of K per split, at most
    64 splits and 256 MB; partials in C's orientation, rows padded to 4), or 0
    when it does not split."""
    cdiv = lambda a, b: -(-a // b)
    rows, cols = (n, m) if trans else (m, n)
    ldp = cdiv(cols, 4) * 4
    tiles = cdiv(m, 256) * cdiv(n, 256) * nprob
    if tiles >= 192:
        return 0
    s = min(cdiv(256, tiles), k // 128, 64, (256 << 20) // (nprob * rows * ldp * 4))
    if s <= 1:
        return 0
    length = cdiv(cdiv(k, s), 64) * 64
    s = cdiv(k, length)
    return s * nprob * rows * ldp * 4 if s > 1 else 0


def test_oom_retry_walks_the_doubling_schedule(torch_dev):
    """A memory limit that one chunk of 1024 rows exceeds and two chunks of
    512 rows fit: the retry takes the next entry of chunk_doubling_schedule
    (src/resolver.rs:103-126) after the Auto plan, and the result equals the
    oracle's at that plan (ChunkSize::Fixed(512), src/api.rs:232,264-270)."""
    bt, h, v = 1024, 64, 20000
    s, th = normal((bt, h), 61), normal((bt, h), 62)
    w = normal((v, h), 63, 0.05)
    y = uniform_labels(bt, v, 64)
    y[::9] = -100
    opts = LossOptions(kd_weight=0.4, temperature=1.5, label_smoothing=0.1)
    start = H.resolve_chunk_size(bt, ChunkSize.Auto, v, None)
    assert (start.chunk_size, start.num_chunks) == (1024, 1)
    sched = O.chunk_doubling_schedule(bt, start.num_chunks, O.default_max_chunks_limit(bt))
    nxt = next(n for n in sched if n > start.num_chunks)
    want = (O.ceil_div(bt, nxt), nxt)
    row = _tied_f32_row_bytes(h, v)
    limit = int(1.25 * want[0] * row) + (4 << 20)
    assert limit < bt * row          # the Auto plan does not fit
    ctx = H.Context(0)
    ctx.set_memory_limit(limit)
    got = H.distillation_loss(gpu(torch_dev, s), gpu(torch_dev, w), gpu(torch_dev, y),
                              Teacher.Tied(gpu(torch_dev, th)), opts, ctx=ctx)
    ctx.close()
    assert (got.chunk_plan.chunk_size, got.chunk_plan.num_chunks) == want
    ref = O.distillation_loss(s, w, y, Teacher.Tied(th),
                              dataclasses.replace(opts, chunk_size=ChunkSize.Fixed(want[0])))
    check_output(got, ref)


def test_oom_retry_halves_the_staging_group(torch_dev):
    """Eight Fixed(128) chunks staged together exceed the limit, two fit: the
    first stage of the retry halves the group (8 -> 4 -> 2 chunks) and keeps
    the plan; four groups run (four logits GEMMs). Result as the oracle's."""
    bt, h, v = 1024, 64, 20000
    s, th = normal((bt, h), 71), normal((bt, h), 72)
    w = normal((v, h), 73, 0.05)
    y = uniform_labels(bt, v, 74)
    opts = LossOptions(kd_weight=0.4, temperature=1.5, chunk_size=ChunkSize.Fixed(128))
    row = _tied_f32_row_bytes(h, v)
    # two chunks (256 rows) per group plus the split-K partials of their
    # backward GEMMs (one buffer, sized for the larger of the two)
    split = max(_split_k_bytes(256, h, v, 2), _split_k_bytes(h, v, 2 * 256, 1, trans=True))
    limit = int(1.25 * 256 * row) + (4 << 20) + split
    assert limit < 512 * row
    ctx = H.Context(0)
    ctx.set_memory_limit(limit)
    ctx.set_timing(True)
    got = H.distillation_loss(gpu(torch_dev, s), gpu(torch_dev, w), gpu(torch_dev, y),
                              Teacher.Tied(gpu(torch_dev, th)), opts, ctx=ctx)
    _, launches = ctx.kernel_time("gemm_logits")
    ctx.close()
    assert (got.chunk_plan.chunk_size, got.chunk_plan.num_chunks) == (128, 8)
    # attempts at 8 and 4 chunks per group fail before their logits GEMM; the
    # run at 2 chunks per group launches one logits GEMM per group
    assert launches == 4, launches
    ref = O.distillation_loss(s, w, y, Teacher.Tied(th), opts)
    check_output(got, ref)


def test_host_buffers_round_trip(torch_dev):
    """numpy (host) inputs and outputs go through the same device path."""
    bt, h, v = 40, 24, 130
    s, th, w = normal((bt, h), 1), normal((bt, h), 2), normal((v, h), 3, 0.1)
    y = uniform_labels(bt, v, 4)
    opts = LossOptions(kd_weight=0.2, label_smoothing=0.05)
    got = H.distillation_loss(s, w, y, Teacher.Tied(th), opts)
    ref = O.distillation_loss(s, w, y, Teacher.Tied(th), opts)
    assert isinstance(got.grad_weight, np.ndarray)
    check_output(got, ref)
