"""orda_hip — MI355X (gfx950) backend of the chunked fused cross-entropy +
forward-KL distillation loss of malcolmgreaves/orda-cutile-rs.

The public surface mirrors the reference crate (src/lib.rs:57-64):
``distillation_loss``, ``LossOptions``, ``DistillationLossOutput``,
``KernelConfig``, ``Profile``, ``Reduction``, ``Backend``, ``ChunkSize``,
``ChunkPlan``, ``Teacher``, ``TeacherMode``, ``is_available`` and the
resolver functions. Compute runs in liborda_hip.so through the C ABI of
include/orda/orda.h; torch tensors (or numpy arrays) carry the memory.
"""
from __future__ import annotations

import ctypes as C
import threading
from typing import Any, Optional

import numpy as np

from . import _lib as L
from .types import (Backend, ChunkPlan, ChunkSize, DistillationLossOutput, KernelConfig,
                    LossOptions, OrdaError, Profile, Reduction, Teacher, TeacherMode,
                    DEFAULT_MAX_FUSED_SIZE, is_power_of_two)

__all__ = [
    "Backend", "ChunkPlan", "ChunkSize", "Context", "DistillationLossOutput", "KernelConfig",
    "LossOptions", "OrdaError", "Profile", "Reduction", "Teacher", "TeacherMode",
    "DEFAULT_MAX_FUSED_SIZE", "chunk_doubling_schedule", "chunks_from_raw",
    "default_max_chunks_limit", "distillation_loss", "is_available", "is_power_of_two",
    "kl_ce_on_logits_chunk", "quant_rows_int8", "resolve_chunk_size", "lib_path",
]

lib_path = L.LIB_PATH


def _torch():
    import torch
    return torch


# ------------------------------------------------------------------ resolver
def resolve_chunk_size(bt: int, chunk_size: ChunkSize, v: Optional[int],
                       max_chunks: Optional[int]) -> ChunkPlan:
    """src/resolver.rs:53-99"""
    if bt <= 0:
        raise ValueError("BT (batch * sequence length) must be > 0")
    cs, nc = C.c_int64(), C.c_int64()
    fixed = chunk_size.fixed
    rc = L.load().orda_resolve_chunk_size(bt, int(fixed is not None), int(fixed or 0),
                                          int(v is not None), int(v or 0),
                                          int(max_chunks is not None), int(max_chunks or 0),
                                          C.byref(cs), C.byref(nc))
    if rc != L.ORDA_OK:
        raise OrdaError("resolve_chunk_size failed", rc)
    return ChunkPlan(cs.value, nc.value)


def chunks_from_raw(raw: float) -> int:
    """src/resolver.rs:27-36"""
    return L.load().orda_chunks_from_raw(raw)


def default_max_chunks_limit(bt: int) -> int:
    """src/resolver.rs:103-105"""
    return L.load().orda_default_max_chunks_limit(bt)


def chunk_doubling_schedule(bt: int, start: int, limit: int) -> list:
    """src/resolver.rs:114-126"""
    buf = (C.c_int64 * 128)()
    n = L.load().orda_chunk_doubling_schedule(bt, start, limit, buf, 128)
    return [buf[i] for i in range(min(n, 128))]


def is_available() -> bool:
    """src/lib.rs:70-79: a gfx950 device is visible to the HIP library."""
    try:
        return bool(L.load().orda_is_available())
    except (OSError, RuntimeError):
        return False


# ------------------------------------------------------------------ tensors
class _Keep:
    """Holds Python objects alive for the duration of a call."""

    def __init__(self):
        self.items = []

    def __call__(self, x):
        self.items.append(x)
        return x


def _desc(x, keep: _Keep, what: str) -> L.Tensor:
    """orda_tensor for a 2-D torch tensor / numpy array (or 1-D as [n,1])."""
    t = L.Tensor()
    if x is None:
        return t
    if isinstance(x, np.ndarray):
        a = x
        if a.ndim == 1:
            a = a.reshape(-1, 1)
        if a.ndim != 2:
            raise OrdaError(f"{what} must be 2-D")
        if a.dtype not in (np.float32, np.int8) or a.strides[1] != a.itemsize:
            a = keep(np.ascontiguousarray(a, dtype=np.float32 if a.dtype != np.int8 else np.int8))
        t.data = a.ctypes.data
        t.rows, t.cols = a.shape
        t.ld = a.strides[0] // a.itemsize
        t.dtype = L.I8 if a.dtype == np.int8 else L.F32
        t.location = L.HOST
        return t
    torch = _torch()
    a = x
    if a.dim() == 1:
        a = a.view(-1, 1)
    if a.dim() != 2:
        raise OrdaError(f"{what} must be 2-D")
    if a.stride(1) != 1 or (a.size(0) > 1 and a.stride(0) < a.size(1)):
        a = keep(a.contiguous())
    if a.dtype == torch.float32:
        dt = L.F32
    elif a.dtype == torch.bfloat16:
        dt = L.BF16
    elif a.dtype == torch.int8:
        dt = L.I8
    else:
        raise OrdaError(f"{what} must be float32 or bfloat16, got {a.dtype}")
    t.data = a.data_ptr()
    t.rows, t.cols = a.shape
    t.ld = a.stride(0) if a.size(0) > 1 else a.size(1)
    t.dtype = dt
    t.location = L.DEVICE if a.is_cuda else L.HOST
    return t


def _labels_ptr(labels, keep: _Keep):
    """(pointer, n, location) of int64 labels."""
    if isinstance(labels, np.ndarray) or isinstance(labels, (list, tuple)):
        a = keep(np.ascontiguousarray(labels, dtype=np.int64))
        return a.ctypes.data, a.size, L.HOST
    torch = _torch()
    a = labels
    if a.dtype != torch.int64 or not a.is_contiguous():
        a = keep(a.to(torch.int64).contiguous())
    return a.data_ptr(), a.numel(), (L.DEVICE if a.is_cuda else L.HOST)


def _is_device(x) -> bool:
    return hasattr(x, "is_cuda") and x.is_cuda


def _alloc(like, rows, cols, dtype="f32"):
    if _is_device(like):
        torch = _torch()
        dt = {"f32": torch.float32, "i8": torch.int8}[dtype]
        return torch.empty((rows, cols), dtype=dt, device=like.device)
    return np.empty((rows, cols), dtype={"f32": np.float32, "i8": np.int8}[dtype])


# ------------------------------------------------------------------ context
class Context:
    """orda_ctx: a HIP stream, a cached device workspace and kernel timers.
    With ``use_torch_stream`` every call runs on torch's current stream."""

    def __init__(self, device: int = 0, use_torch_stream: bool = True):
        self._lib = L.load()
        self.device = device
        self.use_torch_stream = use_torch_stream
        h = C.c_void_p()
        err = C.create_string_buffer(512)
        rc = self._lib.orda_ctx_create(device, C.byref(h), err, 512)
        if rc != L.ORDA_OK:
            raise OrdaError(err.value.decode(), rc)
        self.handle = h

    def close(self):
        if getattr(self, "handle", None):
            self._lib.orda_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def bind_stream(self):
        if self.use_torch_stream:
            torch = _torch()
            s = torch.cuda.current_stream(self.device).cuda_stream
            self._lib.orda_ctx_set_stream(self.handle, C.c_void_p(s))

    def set_memory_limit(self, nbytes: int):
        self._lib.orda_ctx_set_memory_limit(self.handle, int(nbytes))

    def set_staging_budget(self, nbytes: int):
        """Bytes of logits staging per group of chunks (default 16 GiB)."""
        if self._lib.orda_ctx_set_staging_budget(self.handle, int(nbytes)) != L.ORDA_OK:
            raise OrdaError("staging budget must be positive")

    def trim(self):
        self._lib.orda_ctx_trim(self.handle)

    def workspace_bytes(self) -> int:
        """Device bytes the context's workspace holds."""
        n = C.c_int64()
        self._lib.orda_ctx_workspace_bytes(self.handle, C.byref(n))
        return n.value

    def set_timing(self, on: bool):
        self._lib.orda_ctx_set_timing(self.handle, int(on))

    def reset_timing(self):
        self._lib.orda_ctx_reset_kernel_time(self.handle)

    def kernel_time(self, kind: str):
        """(total milliseconds, launches) recorded with HIP events."""
        ms, n = C.c_double(), C.c_int64()
        self._lib.orda_ctx_get_kernel_time(self.handle, L.KERNEL_KINDS[kind], C.byref(ms),
                                           C.byref(n))
        return ms.value, n.value


_default_ctx = threading.local()


def default_context(device: int = 0) -> Context:
    """The calling thread's context for `device`. A context's workspace
    and stream serve one call at a time, and ctypes releases the GIL during
    the call, so every thread gets its own (the C ABI's one context per
    caller thread)."""
    per_thread = getattr(_default_ctx, "by_device", None)
    if per_thread is None:
        per_thread = _default_ctx.by_device = {}
    if device not in per_thread:
        per_thread[device] = Context(device)
    return per_thread[device]


def _options_c(o: LossOptions) -> LossOptionsC:
    c = L.LossOptionsC()
    L.load().orda_loss_options_default(C.byref(c))
    c.student_ce_weight = o.student_ce_weight
    c.has_teacher_ce_weight = int(o.teacher_ce_weight is not None)
    c.teacher_ce_weight = o.teacher_ce_weight or 0.0
    c.kd_weight = o.kd_weight
    c.temperature = o.temperature
    c.ignore_index = o.ignore_index
    c.label_smoothing = o.label_smoothing
    c.reduction = int(o.reduction)
    c.chunk_fixed = int(o.chunk_size.fixed is not None)
    c.chunk_rows = int(o.chunk_size.fixed or 0)
    k = o.config
    c.config.online_softmax = int(k.online_softmax)
    c.config.fast_math = int(k.fast_math)
    c.config.quantize_grad_weight = int(k.quantize_grad_weight)
    c.config.stochastic_rounding = int(k.stochastic_rounding)
    c.config.fp32_grad_weight_accumulation = int(k.fp32_grad_weight_accumulation)
    c.config.has_max_chunks = int(k.max_chunks is not None)
    c.config.max_chunks = int(k.max_chunks or 0)
    c.config.max_fused_size = int(k.max_fused_size)
    c.config.has_stochastic_seed = int(k.stochastic_seed is not None)
    c.config.stochastic_seed = int(k.stochastic_seed or 0)
    c.config.profile = int(k.profile)
    c.backend = int(o.backend)
    return c


LossOptionsC = L.LossOptionsC


def distillation_loss(student_hidden: Any, weight: Any, labels: Any, teacher: Teacher,
                      opts: Optional[LossOptions] = None, *, ctx: Optional[Context] = None,
                      outputs: Optional[dict] = None, rows: bool = False,
                      quant_codes: bool = False) -> DistillationLossOutput:
    """src/api.rs:188-422 on the GPU.

    Inputs are torch tensors (on the GPU, or on the CPU) or numpy arrays,
    float32 or bfloat16; gradients come back as float32 on the inputs'
    device. ``outputs`` may pass preallocated gradient buffers
    (keys grad_student_hidden, grad_weight, grad_teacher_hidden,
    grad_teacher_weight). ``rows`` also returns per-row losses and
    ``quant_codes`` the INT8 codes/scales of grad_weight.
    Raises OrdaError with the reference's message on invalid input.
    """
    opts = opts or LossOptions()
    keep = _Keep()
    lib = L.load()
    dev = _is_device(student_hidden)
    if ctx is None:
        ctx = default_context((student_hidden.device.index or 0) if dev else 0)
    if dev:
        ctx.bind_stream()
    else:
        lib.orda_ctx_set_stream(ctx.handle, None)

    s_t = _desc(student_hidden, keep, "student_hidden")
    w_t = _desc(weight, keep, "weight")
    lp, nl, lloc = _labels_ptr(labels, keep)
    tc = L.TeacherC()
    mode = teacher.mode()
    tc.mode = int(mode)
    if teacher.hidden is not None:
        tc.hidden = _desc(teacher.hidden, keep, "teacher hidden")
    if teacher.weight is not None:
        tc.weight = _desc(teacher.weight, keep, "teacher weight")
    if teacher.logits is not None:
        tc.logits = _desc(teacher.logits, keep, "teacher logits")

    bt, h = s_t.rows, s_t.cols
    v = w_t.rows
    w_tv = opts.teacher_ce_weight if opts.teacher_ce_weight is not None \
        else teacher.default_teacher_ce_weight()
    ht = tc.hidden.cols if mode == TeacherMode.Separate else h
    has_ght = w_tv > 0 and mode in (TeacherMode.Tied, TeacherMode.Separate)
    has_gwt = w_tv > 0 and mode == TeacherMode.Separate
    outputs = dict(outputs or {})
    like = student_hidden
    gh = outputs.get("grad_student_hidden")
    gw = outputs.get("grad_weight")
    ght = outputs.get("grad_teacher_hidden")
    gwt = outputs.get("grad_teacher_weight")
    if gh is None:
        gh = _alloc(like, max(bt, 0), max(h, 0))
    if gw is None:
        gw = _alloc(like, max(v, 0), max(h, 0))
    if has_ght and ght is None:
        ght = _alloc(like, bt, ht)
    if has_gwt and gwt is None:
        gwt = _alloc(like, v, ht)
    out = L.LossOutputC()
    out.grad_student_hidden = _desc(gh, keep, "grad_student_hidden")
    out.grad_weight = _desc(gw, keep, "grad_weight")
    if has_ght:
        out.grad_teacher_hidden = _desc(ght, keep, "grad_teacher_hidden")
    if has_gwt:
        out.grad_teacher_weight = _desc(gwt, keep, "grad_teacher_weight")
    row_bufs = None
    if rows:
        row_bufs = [_alloc(like, bt, 1) for _ in range(3)]
        out.row_nll_student = _desc(row_bufs[0], keep, "row_nll_student")
        out.row_nll_teacher = _desc(row_bufs[1], keep, "row_nll_teacher")
        out.row_kl = _desc(row_bufs[2], keep, "row_kl")
    codes = scales = None
    if quant_codes and opts.config.quantize_grad_weight:
        codes = _alloc(like, v, h, "i8")
        scales = _alloc(like, v, 1)
        out.quant_codes = _desc(codes, keep, "quant_codes")
        out.quant_scales = _desc(scales, keep, "quant_scales")
    oc = _options_c(opts)
    err = C.create_string_buffer(1024)
    rc = lib.orda_distillation_loss(ctx.handle, C.byref(s_t), C.byref(w_t), C.c_void_p(lp), nl,
                                    lloc, C.byref(tc), C.byref(oc), C.byref(out), err, 1024)
    if rc != L.ORDA_OK:
        raise OrdaError(err.value.decode(), rc)

    def flat(x):
        return None if x is None else x.reshape(-1)
    return DistillationLossOutput(
        loss=out.loss, student_ce=out.student_ce, teacher_ce=out.teacher_ce, kl=out.kl,
        grad_student_hidden=gh, grad_weight=gw,
        grad_teacher_hidden=ght if out.has_grad_teacher_hidden else None,
        grad_teacher_weight=gwt if out.has_grad_teacher_weight else None,
        chunk_plan=ChunkPlan(out.chunk_size, out.num_chunks),
        row_nll_student=flat(row_bufs[0]) if rows else None,
        row_nll_teacher=flat(row_bufs[1]) if rows else None,
        row_kl=flat(row_bufs[2]) if rows else None,
        quant_codes=codes, quant_scales=flat(scales))


def kl_ce_on_logits_chunk(logits_chunk, targets, n_rows: int, inv_t: float, kl_grad_scale: float,
                          t_sq: float, student_ce_weight: float, teacher_ce_weight: float,
                          label_smoothing: float, ignore_index: int, student_only: bool,
                          compute_kl: bool, *, ctx: Optional[Context] = None):
    """src/cuda/launch.rs:51-158 (KlCeChunkOutput fields as a dict)."""
    keep = _Keep()
    lib = L.load()
    dev = _is_device(logits_chunk)
    ctx = ctx or default_context((logits_chunk.device.index or 0) if dev else 0)
    if dev:
        ctx.bind_stream()
    else:
        lib.orda_ctx_set_stream(ctx.handle, None)
    lc = _desc(logits_chunk, keep, "logits_chunk")
    v = lc.cols
    if isinstance(targets, (np.ndarray, list, tuple)):
        ta = keep(np.ascontiguousarray(targets, dtype=np.int32))
        tp, tloc = ta.ctypes.data, L.HOST
    else:
        torch = _torch()
        ta = keep(targets.to(torch.int32).contiguous())
        tp, tloc = ta.data_ptr(), (L.DEVICE if ta.is_cuda else L.HOST)
    grid = n_rows if student_only else 2 * n_rows
    gkl = _alloc(logits_chunk, n_rows, v)
    klr = _alloc(logits_chunk, n_rows, 1)
    gce = _alloc(logits_chunk, grid, v)
    cel = _alloc(logits_chunk, grid, 1)
    d = [_desc(x, keep, nm) for x, nm in ((gkl, "grad_kl_student"), (klr, "kl_per_row"),
                                          (gce, "grad_ce"), (cel, "ce_loss"))]
    err = C.create_string_buffer(1024)
    rc = lib.orda_kl_ce_on_logits_chunk(ctx.handle, C.byref(lc), C.c_void_p(tp), tloc, n_rows,
                                        inv_t, kl_grad_scale, t_sq, student_ce_weight,
                                        teacher_ce_weight, label_smoothing, ignore_index,
                                        int(student_only), int(compute_kl), C.byref(d[0]),
                                        C.byref(d[1]), C.byref(d[2]), C.byref(d[3]), err, 1024)
    if rc != L.ORDA_OK:
        raise OrdaError(err.value.decode(), rc)
    return dict(grad_kl_student=gkl, kl_per_row=klr.reshape(-1), grad_ce=gce,
                ce_loss=cel.reshape(-1))


def quant_rows_int8(m, targets, ignore_index: int = -100, stochastic: bool = False,
                    seed: int = 0, grad_output: float = 1.0, *, out=None,
                    ctx: Optional[Context] = None):
    """quantize_grad_w + dequantize_grad_w (src/quant.rs:157-202).
    Returns (dequantized, codes, scales)."""
    keep = _Keep()
    lib = L.load()
    dev = _is_device(m)
    ctx = ctx or default_context((m.device.index or 0) if dev else 0)
    if dev:
        ctx.bind_stream()
    else:
        lib.orda_ctx_set_stream(ctx.handle, None)
    md = _desc(m, keep, "m")
    rows, cols = md.rows, md.cols
    if out is None:
        out = _alloc(m, rows, cols)
    codes = _alloc(m, rows, cols, "i8")
    scales = _alloc(m, rows, 1)
    od, cd, sd = _desc(out, keep, "out"), _desc(codes, keep, "codes"), _desc(scales, keep, "scales")
    lp, nl, lloc = _labels_ptr(targets, keep)
    err = C.create_string_buffer(1024)
    rc = lib.orda_quant_rows_int8(ctx.handle, C.byref(md), C.c_void_p(lp), nl, lloc, ignore_index,
                                  int(stochastic), seed, grad_output, C.byref(od), C.byref(cd),
                                  C.byref(sd), err, 1024)
    if rc != L.ORDA_OK:
        raise OrdaError(err.value.decode(), rc)
    return out, codes, scales.reshape(-1)
