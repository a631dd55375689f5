"""GPU tests of the host paths around the kernels: labels validated on the
device (src/api.rs:104-181, read back at the call's one synchronisation),
the checks on caller tensor views, the chunk-launcher slot reading device
logits in place at any pitch, and the staging budget. All through the C
ABI; tolerances as in tests/parity.py unless stated. (KL near zero:
tests/test_gpu_kl_precision.py.)
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from helpers import bf16_round, normal, uniform_labels
from parity import check_grad, check_output, check_scalar, to_np

import orda_hip as H
from orda_hip import _lib as L
from orda_hip import ChunkSize, KernelConfig, LossOptions, OrdaError, Teacher

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
    return t.to(torch.bfloat16) if dtype == "bf16" else t


# ------------------------------------------------ labels on the device
@pytest.mark.parametrize("bad", [5, -3, 1 << 40])
def test_device_label_out_of_range_message(torch_dev, bad):
    """A bad label on the device is reported with the reference's message
    (src/api.rs:125-133) after the call has run its kernels."""
    bt, h, v = 64, 16, 5
    s, th, w = normal((bt, h), 1), normal((bt, h), 2), normal((v, h), 3, 0.1)
    y = uniform_labels(bt, v, 4)
    y[7] = -100
    y[11] = bad
    y[40] = v + 7          # a later bad label: the first one is reported
    msg = f"label {bad} out of range [0, {v}) and != ignore_index -100"
    with pytest.raises(OrdaError) as e:
        H.distillation_loss(gpu(torch_dev, s), gpu(torch_dev, w), gpu(torch_dev, y),
                            Teacher.Tied(gpu(torch_dev, th)), LossOptions(kd_weight=0.5))
    assert str(e.value) == msg
    with pytest.raises(O.OracleError) as e2:
        O.distillation_loss(s, w, y, Teacher.Tied(th), LossOptions(kd_weight=0.5))
    assert str(e2.value) == msg


def test_device_label_error_ahead_of_later_checks(torch_dev):
    """With a bad device label and a bad later argument (label smoothing,
    teacher shape) the label error is reported, as in the reference, whose
    validate() checks labels first."""
    bt, h, v = 32, 8, 10
    s, th, w = normal((bt, h), 5), normal((bt, h), 6), normal((v, h), 7, 0.1)
    y = uniform_labels(bt, v, 8)
    y[3] = 10
    msg = "label 10 out of range [0, 10) and != ignore_index -100"
    cases = [(Teacher.Tied(gpu(torch_dev, th)), LossOptions(label_smoothing=2.0)),
             (Teacher.Tied(gpu(torch_dev, th[:, :4])), LossOptions())]
    for teacher, opts in cases:
        with pytest.raises(OrdaError) as e:
            H.distillation_loss(gpu(torch_dev, s), gpu(torch_dev, w), gpu(torch_dev, y), teacher,
                                opts)
        assert str(e.value) == msg
    # and with valid labels the later check is the one reported
    y[3] = 1
    with pytest.raises(OrdaError) as e:
        H.distillation_loss(gpu(torch_dev, s), gpu(torch_dev, w), gpu(torch_dev, y),
                            Teacher.Tied(gpu(torch_dev, th)), LossOptions(label_smoothing=2.0))
    assert str(e.value) == "label_smoothing must be in [0,1], got 2"


def _guarded(torch_dev, a, dtype=None, pad=8, sentinel=-7.25):
    """A device copy of 2-D `a` (or 1-D int64 labels) placed inside a larger
    buffer filled with `sentinel`: `pad` rows above and below and, for
    matrices, `pad` columns either side (a multiple of 8 elements, so the view
    keeps a pitch the library reads in place). Returns (view, buffer)."""
    torch, dev = torch_dev
    if a.ndim == 1:
        buf = torch.full((a.shape[0] + 2 * pad,), int(sentinel), dtype=torch.int64, device=dev)
        view = buf[pad:pad + a.shape[0]]
        view.copy_(torch.from_numpy(np.ascontiguousarray(a)).to(dev))
        return view, buf
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    rows, cols = a.shape
    buf = torch.full((rows + 2 * pad, cols + 2 * pad), sentinel, dtype=tdt, device=dev)
    view = buf[pad:pad + rows, pad:pad + cols]
    view.copy_(torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(tdt))
    return view, buf


def _guard_mask(buf, pad):
    """True outside the interior view of a _guarded buffer."""
    m = buf.new_ones(buf.shape, dtype=bool)
    if buf.dim() == 1:
        m[pad:buf.shape[0] - pad] = False
    else:
        m[pad:buf.shape[0] - pad, pad:buf.shape[1] - pad] = False
    return m


@pytest.mark.parametrize("mode,dtype", [("tied", None), ("tied", "bf16"), ("separate", None),
                                        ("precomputed", "bf16")])
def test_out_of_range_device_labels_stay_in_bounds(torch_dev, mode, dtype):
    """Labels far outside [0, V) reach every kernel before the host reads the
    check's result: each kernel treats such a row as ignored, so the call
    ends with the validation error. Every caller buffer (inputs, labels,
    gradient outputs) is an interior view of a larger buffer filled with a
    sentinel: after the rejected call the inputs are unchanged and every
    guard region still holds the sentinel. The context then computes a
    valid call exactly."""
    torch, dev = torch_dev
    bt, h, v = 96, 32, 300
    s, th, w = normal((bt, h), 11), normal((bt, h), 12), normal((v, h), 13, 0.1)
    tw = normal((v, h), 14, 0.1)
    tl = normal((bt, v), 15, 2.0)
    y = uniform_labels(bt, v, 16)
    bad = y.copy()
    bad[::5] = v + 100000
    bad[1::5] = -(1 << 50)
    if dtype == "bf16":
        s, th, w, tw = bf16_round(s), bf16_round(th), bf16_round(w), bf16_round(tw)
    pad = 8
    g_s, b_s = _guarded(torch_dev, s, dtype, pad)
    g_w, b_w = _guarded(torch_dev, w, dtype, pad)
    g_bad, b_bad = _guarded(torch_dev, bad, None, pad)
    inputs = [b_s, b_w, b_bad]
    if mode == "tied":
        g_th, b_th = _guarded(torch_dev, th, dtype, pad)
        inputs.append(b_th)
        t_g, t_o = Teacher.Tied(g_th), Teacher.Tied(th)
    elif mode == "separate":
        g_th, b_th = _guarded(torch_dev, th, dtype, pad)
        g_tw, b_tw = _guarded(torch_dev, tw, dtype, pad)
        inputs += [b_th, b_tw]
        t_g, t_o = Teacher.Separate(g_th, g_tw), Teacher.Separate(th, tw)
    else:
        g_tl, b_tl = _guarded(torch_dev, tl, None, pad)
        inputs.append(b_tl)
        t_g, t_o = Teacher.Precomputed(g_tl), Teacher.Precomputed(tl)
    saved = [b.clone() for b in inputs]
    out_shapes = {"grad_student_hidden": (bt, h), "grad_weight": (v, h)}
    if mode in ("tied", "separate"):
        out_shapes["grad_teacher_hidden"] = (bt, h)
    if mode == "separate":
        out_shapes["grad_teacher_weight"] = (v, h)
    outs, out_bufs = {}, []
    for name, shape in out_shapes.items():
        view, buf = _guarded(torch_dev, np.zeros(shape, np.float32), None, pad)
        outs[name] = view
        out_bufs.append(buf)
    opts = LossOptions(kd_weight=0.4, temperature=1.5, label_smoothing=0.1, teacher_ce_weight=1.0,
                       chunk_size=ChunkSize.Fixed(32),
                       config=KernelConfig(quantize_grad_weight=True))
    ctx = H.Context(0)
    with pytest.raises(OrdaError) as e:
        H.distillation_loss(g_s, g_w, g_bad, t_g, opts, ctx=ctx, outputs=outs)
    assert str(e.value) == f"label {v + 100000} out of range [0, {v}) and != ignore_index -100"
    torch.cuda.synchronize()
    for b, c in zip(inputs, saved):
        assert torch.equal(b, c), "an input buffer changed"
    for buf in out_bufs:
        guard = buf[_guard_mask(buf, pad)]
        assert bool((guard == -7.25).all()), "a write landed outside an output view"
    g_y, _ = _guarded(torch_dev, y, None, pad)
    got = H.distillation_loss(g_s, g_w, g_y, t_g, opts, ctx=ctx, outputs=outs)
    ctx.close()
    for buf in out_bufs:
        assert bool((buf[_guard_mask(buf, pad)] == -7.25).all())
    ref = O.distillation_loss(s, w, y, t_o, opts)
    check_output(got, ref, kind="bf16" if dtype else "f32", skip_grad_weight=True)
    # dequantized: a code one step off at a rounding boundary moves an element
    # by amax/127 of its row, inside the 2e-2 tolerance (the exact INT8
    # criteria are tested in test_gpu_parity.py)
    check_grad("grad_weight (dequantized)", got.grad_weight, ref.grad_weight, "bf16")


def test_quant_entry_point_device_targets_out_of_range(torch_dev):
    """orda_quant_rows_int8 with device targets, some out of range or
    ignored: they mark no row (src/quant.rs:147-155 keeps in-range targets
    only) and the result equals the oracle's."""
    rows, cols = 200, 512
    m = normal((rows, cols), 21)
    t = np.array([5, 5, 199, -100, 200, 1 << 40, -7, 0])
    out, q, s = H.quant_rows_int8(gpu(torch_dev, m), gpu(torch_dev, t), -100, False, 0)
    rout, rq, rs = O.quant_dequant_grad_w(m, t, -100, False, 0)
    np.testing.assert_array_equal(to_np(q), rq)
    np.testing.assert_array_equal(to_np(s), rs)
    np.testing.assert_array_equal(to_np(out), rout)


# ------------------------------------------------ caller tensor views
def _tensor(t, rows=None, cols=None, ld=None, data=None):
    d = L.Tensor()
    d.data = t.data_ptr() if data is None else data
    d.rows = t.shape[0] if rows is None else rows
    d.cols = t.shape[1] if cols is None else cols
    d.ld = t.stride(0) if ld is None else ld
    d.dtype = L.F32
    d.location = L.DEVICE
    return d


def _call(ctx, s, w, y, teacher_c, out_c, opts):
    lib = L.load()
    oc = H._options_c(opts)
    err = C.create_string_buffer(512)
    rc = lib.orda_distillation_loss(ctx.handle, C.byref(s), C.byref(w), C.c_void_p(y.data_ptr()),
                                    y.numel(), L.DEVICE, C.byref(teacher_c), C.byref(oc),
                                    C.byref(out_c), err, 512)
    return rc, err.value.decode()


def test_device_teacher_logits_and_outputs_views_checked(torch_dev):
    """Device Precomputed teacher logits and device outputs get the same
    checks as every staged input: a null pointer or ld < cols is rejected
    with ORDA_ERR_INVALID before any kernel runs."""
    torch, dev = torch_dev
    bt, h, v = 16, 8, 40
    s = torch.randn(bt, h, device=dev)
    w = torch.randn(v, h, device=dev) * 0.1
    tl = torch.randn(bt, v, device=dev)
    y = torch.randint(0, v, (bt,), device=dev)
    gh = torch.empty(bt, h, device=dev)
    gw = torch.empty(v, h, device=dev)
    opts = LossOptions(kd_weight=0.5)
    ctx = H.Context(0)
    ctx.bind_stream()

    def run(tl_desc, gw_desc):
        t = L.TeacherC()
        t.mode = int(H.TeacherMode.Precomputed)
        t.logits = tl_desc
        o = L.LossOutputC()
        o.grad_student_hidden = _tensor(gh)
        o.grad_weight = gw_desc
        return _call(ctx, _tensor(s), _tensor(w), y, t, o, opts)

    assert run(_tensor(tl), _tensor(gw))[0] == L.ORDA_OK
    rc, msg = run(_tensor(tl, data=0), _tensor(gw))
    assert rc == L.ORDA_ERR_INVALID and msg == "teacher logits has a null data pointer"
    rc, msg = run(_tensor(tl, ld=v - 1), _tensor(gw))
    assert rc == L.ORDA_ERR_INVALID and msg == "teacher logits has ld < cols"
    rc, msg = run(_tensor(tl), _tensor(gw, ld=h - 1))
    assert rc == L.ORDA_ERR_INVALID and msg == "grad_weight has ld < cols"
    rc, msg = run(_tensor(tl), _tensor(gw, data=0))
    assert rc == L.ORDA_ERR_INVALID and msg == "grad_weight has a null data pointer"
    ctx.close()


# ------------------------------------------------ the chunk-launcher slot
@pytest.mark.parametrize("pitch_pad,offset", [(0, 0), (3, 0), (5, 1)])
def test_slot_reads_device_logits_in_place(torch_dev, pitch_pad, offset):
    """kl_ce_on_logits_chunk on a device logits_chunk viewed with a padded
    pitch and a base that is not 16-byte aligned (offset in elements):
    read in place, results as the oracle's kl_chunk / ce_fwdbwd_row. The
    padding holds NaN, so a read past a row's V columns fails the test."""
    torch, dev = torch_dev
    n, v = 20, 777
    rng = np.random.default_rng(31)
    lc = (rng.standard_normal((2 * n, v)) * 2).astype(np.float32)
    y = rng.integers(0, v, n).astype(np.int32)
    y[::4] = -100
    big = torch.full((2 * n * (v + pitch_pad) + offset + 8,), float("nan"), device=dev)
    view = big[offset:offset + 2 * n * (v + pitch_pad)].view(2 * n, v + pitch_pad)[:, :v]
    view.copy_(torch.from_numpy(lc).to(dev))
    T, kd = 2.0, 0.7
    for targets in (gpu(torch_dev, y), y):
        got = H.kl_ce_on_logits_chunk(view, targets, n, 1.0 / T, kd * T, T * T, 1.0, 0.5, 0.05,
                                      -100, False, True)
        kl, gkl = O.kl_chunk(lc, y.astype(np.int64), n, kd, T, -100, 1.0, True)
        check_grad("grad_kl_student", got["grad_kl_student"], gkl)
        check_scalar("sum kl_per_row", float(np.sum(to_np(got["kl_per_row"]), dtype=np.float64)),
                     kl)
        gce = to_np(got["grad_ce"])
        cel = to_np(got["ce_loss"])
        for r in range(2 * n):
            nll, g = O.ce_fwdbwd_row(lc[r], int(y[r % n]), -100, 0.05, 1.0 if r < n else 0.5)
            check_scalar(f"ce_loss[{r}]", float(cel[r]), nll)
            check_grad(f"grad_ce[{r}]", gce[r], g)


# ------------------------------------------------ the staging budget
def test_staging_budget_bounds_the_group(torch_dev):
    """The group of chunks staged together is sized so that its device
    buffers fit the context's staging budget, counting every per-row buffer:
    bf16 logits of both rows, tile statistics, label logits, the two KL
    partials per tile and the row constants, the half-tile maxima of both
    rows, and the [h_s; h_t] rows grad_W multiplies. Bytes per row at
    H=4096, V=8192 (pitch 8256): 2*8256*2 + 2*32*16 + 2*4 + 32*8 + 16 +
    2*64*4 + 2*4096*2 = 51224. With a budget of 2.5 chunks of 1024 rows,
    two chunks are staged at a time (two logits GEMMs; the groups are large
    enough that no backward GEMM splits K) and the workspace stays within
    the budget (plus the per-call row losses)."""
    torch, dev = torch_dev
    bt, h, v, cs = 4096, 4096, 8192, 1024
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    hs = torch.randn(bt, h, generator=g, device=dev).to(torch.bfloat16)
    ht = torch.randn(bt, h, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(v, h, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    y = torch.randint(0, v, (bt,), generator=g, device=dev)
    row = 2 * 8256 * 2 + 2 * 32 * 16 + 2 * 4 + 32 * 8 + 16 + 2 * 64 * 4 + 2 * 4096 * 2
    budget = int(2.5 * cs * row)
    ctx = H.Context(0)
    ctx.set_staging_budget(budget)
    ctx.set_timing(True)
    opts = LossOptions(kd_weight=0.4, temperature=1.5, chunk_size=ChunkSize.Fixed(cs))
    out = H.distillation_loss(hs, w, y, Teacher.Tied(ht), opts, ctx=ctx)
    _, groups = ctx.kernel_time("gemm_logits")
    held = ctx.workspace_bytes()
    ctx.close()
    assert (out.chunk_plan.chunk_size, out.chunk_plan.num_chunks) == (cs, 4)
    assert groups == 2, groups
    assert held <= budget + 3 * bt * 4 + 4096, (held, budget)
