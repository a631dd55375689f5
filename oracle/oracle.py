"""ctypes/numpy front end of the CPU oracle (liborda_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of bench.py, always as the reference side of a
comparison or as the timed CPU baseline. The product never imports it.

The functions mirror the reference crate's Rust API (file:line cited on each
C entry point in orda_oracle.c). Teacher/option objects are duck-typed: any
object with the attributes of ``orda_hip.types.Teacher`` / ``LossOptions``
works, so tests build one set of arguments and hand it to both sides.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from types import SimpleNamespace

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# ORDA_ORACLE_LIB selects another build of the same source (the Makefile's
# `asan` target builds one with AddressSanitizer).
_LIB_PATH = os.environ.get("ORDA_ORACLE_LIB", os.path.join(_HERE, "liborda_oracle.so"))

_f32p = C.POINTER(C.c_float)
_f64p = C.POINTER(C.c_double)
_i64p = C.POINTER(C.c_int64)
_i8p = C.POINTER(C.c_int8)
_szp = C.POINTER(C.c_size_t)
_u64p = C.POINTER(C.c_uint64)


class _Options(C.Structure):
    _fields_ = [
        ("student_ce_weight", C.c_float),
        ("has_teacher_ce_weight", C.c_int),
        ("teacher_ce_weight", C.c_float),
        ("kd_weight", C.c_float),
        ("temperature", C.c_float),
        ("ignore_index", C.c_int64),
        ("label_smoothing", C.c_float),
        ("reduction", C.c_int),
        ("chunk_fixed", C.c_int),
        ("chunk_rows", C.c_size_t),
        ("backend", C.c_int),
        ("online_softmax", C.c_int),
        ("fast_math", C.c_int),
        ("quantize_grad_weight", C.c_int),
        ("stochastic_rounding", C.c_int),
        ("fp32_grad_weight_accumulation", C.c_int),
        ("has_max_chunks", C.c_int),
        ("max_chunks", C.c_size_t),
        ("max_fused_size", C.c_size_t),
        ("has_stochastic_seed", C.c_int),
        ("stochastic_seed", C.c_uint64),
    ]


class _Teacher(C.Structure):
    _fields_ = [
        ("mode", C.c_int),
        ("hidden", _f32p), ("hidden_rows", C.c_size_t), ("hidden_cols", C.c_size_t),
        ("weight", _f32p), ("weight_rows", C.c_size_t), ("weight_cols", C.c_size_t),
        ("logits", _f32p), ("logits_rows", C.c_size_t), ("logits_cols", C.c_size_t),
    ]


class _Output(C.Structure):
    _fields_ = [
        ("loss", C.c_float), ("student_ce", C.c_float), ("teacher_ce", C.c_float),
        ("kl", C.c_float),
        ("grad_student_hidden", _f32p),
        ("grad_weight", _f32p),
        ("grad_teacher_hidden", _f32p), ("has_grad_teacher_hidden", C.c_int),
        ("grad_teacher_weight", _f32p), ("has_grad_teacher_weight", C.c_int),
        ("chunk_size", C.c_size_t), ("num_chunks", C.c_size_t),
        ("row_nll_s", _f32p), ("row_nll_t", _f32p), ("row_kl", _f32p),
        ("q_codes", _i8p), ("q_scales", _f32p),
    ]


def build() -> None:
    """Compile liborda_oracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is not built; run `make -C oracle`")
        L = C.CDLL(_LIB_PATH)
        L.ora_ceil_div.restype = C.c_size_t
        L.ora_ceil_div.argtypes = [C.c_size_t, C.c_size_t]
        L.ora_chunks_from_raw.restype = C.c_size_t
        L.ora_chunks_from_raw.argtypes = [C.c_double]
        L.ora_resolve_chunk_size.restype = None
        L.ora_resolve_chunk_size.argtypes = [C.c_size_t, C.c_int, C.c_size_t, C.c_int,
                                             C.c_size_t, C.c_int, C.c_size_t, _szp, _szp]
        L.ora_default_max_chunks_limit.restype = C.c_size_t
        L.ora_default_max_chunks_limit.argtypes = [C.c_size_t]
        L.ora_chunk_doubling_schedule.restype = C.c_size_t
        L.ora_chunk_doubling_schedule.argtypes = [C.c_size_t, C.c_size_t, C.c_size_t,
                                                  _szp, C.c_size_t]
        L.ora_is_power_of_two.restype = C.c_int
        L.ora_is_power_of_two.argtypes = [C.c_size_t]
        L.ora_set_threads.restype = None
        L.ora_set_threads.argtypes = [C.c_int]
        for nm in ("ora_matmul_nt", "ora_matmul_nn", "ora_matmul_tn"):
            f = getattr(L, nm)
            f.restype = None
            f.argtypes = [_f32p, _f32p, _f32p, C.c_size_t, C.c_size_t, C.c_size_t]
        L.ora_ce_fwdbwd_row.restype = C.c_float
        L.ora_ce_fwdbwd_row.argtypes = [_f32p, C.c_size_t, C.c_int64, C.c_int64, C.c_float,
                                        C.c_float, _f32p]
        L.ora_softmax_logsoftmax.restype = None
        L.ora_softmax_logsoftmax.argtypes = [_f32p, C.c_size_t, C.c_double, _f64p, _f64p]
        L.ora_forward_kl_row.restype = C.c_double
        L.ora_forward_kl_row.argtypes = [_f32p, _f32p, C.c_size_t, C.c_double]
        L.ora_kl_chunk.restype = C.c_float
        L.ora_kl_chunk.argtypes = [_f32p, _i64p, C.c_size_t, C.c_size_t, C.c_float, C.c_float,
                                   C.c_int64, C.c_float, _f32p]
        L.ora_rng_new.restype = C.c_uint64
        L.ora_rng_new.argtypes = [C.c_uint64]
        L.ora_rng_next_u64.restype = C.c_uint64
        L.ora_rng_next_u64.argtypes = [_u64p]
        L.ora_rng_next_f32.restype = C.c_float
        L.ora_rng_next_f32.argtypes = [_u64p]
        L.ora_round_half_even.restype = C.c_float
        L.ora_round_half_even.argtypes = [C.c_float]
        L.ora_row_scale.restype = C.c_float
        L.ora_row_scale.argtypes = [_f32p, C.c_size_t]
        L.ora_quantize_rowwise_int8.restype = None
        L.ora_quantize_rowwise_int8.argtypes = [_f32p, C.c_size_t, C.c_size_t, _i8p, _f32p]
        L.ora_quantize_rowwise_int8_stochastic.restype = None
        L.ora_quantize_rowwise_int8_stochastic.argtypes = [_f32p, C.c_size_t, C.c_size_t,
                                                           _u64p, _i8p, _f32p]
        L.ora_unique_targets.restype = C.c_size_t
        L.ora_unique_targets.argtypes = [_i64p, C.c_size_t, C.c_int64, C.c_size_t, _szp]
        L.ora_quant_dequant_grad_w.restype = None
        L.ora_quant_dequant_grad_w.argtypes = [_f32p, C.c_size_t, C.c_size_t, _i64p,
                                               C.c_size_t, C.c_int64, C.c_int, C.c_uint64,
                                               C.c_float, _f32p, _i8p, _f32p]
        L.ora_options_default.restype = None
        L.ora_options_default.argtypes = [C.POINTER(_Options)]
        L.ora_distillation_loss.restype = C.c_int
        L.ora_distillation_loss.argtypes = [_f32p, C.c_size_t, C.c_size_t, _f32p, C.c_size_t,
                                            C.c_size_t, _i64p, C.c_size_t,
                                            C.POINTER(_Teacher), C.POINTER(_Options),
                                            C.POINTER(_Output), C.c_char_p, C.c_size_t]
        L.ora_forward_loss_f64.restype = C.c_int
        L.ora_forward_loss_f64.argtypes = [_f32p, C.c_size_t, C.c_size_t, _f32p, C.c_size_t,
                                           C.c_size_t, _i64p, C.c_size_t,
                                           C.POINTER(_Teacher), C.POINTER(_Options), _f32p,
                                           _f64p, C.c_char_p, C.c_size_t]
        _lib = L
    return _lib


# ---------------------------------------------------------------- helpers
def _f32(a) -> np.ndarray:
    a = _to_numpy(a)
    return np.ascontiguousarray(a, dtype=np.float32)


def _to_numpy(a):
    if a is None:
        return None
    if hasattr(a, "detach"):  # torch tensor
        t = a.detach()
        if t.dtype.is_floating_point and t.dtype != __import__("torch").float32:
            t = t.float()
        return t.cpu().numpy()
    return np.asarray(a)


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t) if a is not None else C.cast(None, t)


def _shape2(a: np.ndarray):
    if a.ndim != 2:
        raise ValueError("matrices are 2-D")
    return a.shape


class OracleError(RuntimeError):
    pass


# ---------------------------------------------------------------- resolver
def ceil_div(a: int, b: int) -> int:
    return lib().ora_ceil_div(a, b)


def chunks_from_raw(raw: float) -> int:
    return lib().ora_chunks_from_raw(raw)


def resolve_chunk_size(bt: int, chunk_size, v, max_chunks):
    """chunk_size: an object with ``.fixed`` (None = Auto) or an int row count."""
    fixed = getattr(chunk_size, "fixed", chunk_size)
    cs, nc = C.c_size_t(), C.c_size_t()
    lib().ora_resolve_chunk_size(bt, int(fixed is not None), int(fixed or 0),
                                 int(v is not None), int(v or 0),
                                 int(max_chunks is not None), int(max_chunks or 0),
                                 C.byref(cs), C.byref(nc))
    return SimpleNamespace(chunk_size=cs.value, num_chunks=nc.value)


def default_max_chunks_limit(bt: int) -> int:
    return lib().ora_default_max_chunks_limit(bt)


def chunk_doubling_schedule(bt: int, start: int, limit: int):
    buf = (C.c_size_t * 128)()
    n = lib().ora_chunk_doubling_schedule(bt, start, limit, buf, 128)
    return [buf[i] for i in range(min(n, 128))]


def is_power_of_two(v: int) -> bool:
    return bool(lib().ora_is_power_of_two(v))


# ---------------------------------------------------------------- mat
def set_threads(n: int) -> None:
    """Threads for the three products (1, the default, is the reference's
    single thread). Results are bitwise the same for any count: each output
    element still accumulates its terms in the reference's order."""
    lib().ora_set_threads(int(n))


def matmul_nt(a, b):
    a, b = _f32(a), _f32(b)
    m, k = _shape2(a)
    n, k2 = _shape2(b)
    assert k == k2
    out = np.empty((m, n), np.float32)
    lib().ora_matmul_nt(_p(a, _f32p), _p(b, _f32p), _p(out, _f32p), m, k, n)
    return out


def matmul_nn(a, b):
    a, b = _f32(a), _f32(b)
    m, k = _shape2(a)
    k2, n = _shape2(b)
    assert k == k2
    out = np.empty((m, n), np.float32)
    lib().ora_matmul_nn(_p(a, _f32p), _p(b, _f32p), _p(out, _f32p), m, k, n)
    return out


def matmul_tn(a, b):
    a, b = _f32(a), _f32(b)
    k, m = _shape2(a)
    k2, n = _shape2(b)
    assert k == k2
    out = np.empty((m, n), np.float32)
    lib().ora_matmul_tn(_p(a, _f32p), _p(b, _f32p), _p(out, _f32p), k, m, n)
    return out


# ---------------------------------------------------------------- rows
def ce_fwdbwd_row(x, y: int, ignore_index: int, label_smoothing: float, scale: float):
    x = _f32(x).ravel()
    g = np.empty_like(x)
    nll = lib().ora_ce_fwdbwd_row(_p(x, _f32p), x.size, y, ignore_index, label_smoothing,
                                  scale, _p(g, _f32p))
    return float(np.float32(nll)), g


def ce_loss_row(x, y: int, ignore_index: int, label_smoothing: float) -> float:
    return ce_fwdbwd_row(x, y, ignore_index, label_smoothing, 1.0)[0]


def softmax_logsoftmax(x, inv_t: float):
    x = _f32(x).ravel()
    p = np.empty(x.size, np.float64)
    lp = np.empty(x.size, np.float64)
    lib().ora_softmax_logsoftmax(_p(x, _f32p), x.size, inv_t, _p(p, _f64p), _p(lp, _f64p))
    return p, lp


def forward_kl_row(s, t, temperature: float) -> float:
    s, t = _f32(s).ravel(), _f32(t).ravel()
    assert s.size == t.size
    return lib().ora_forward_kl_row(_p(s, _f32p), _p(t, _f32p), s.size, temperature)


def kl_chunk(logits_chunk, targets, n_rows: int, kl_weight: float, temperature: float,
             ignore_index: int, grad_denom: float, compute_grad: bool):
    lc = _f32(logits_chunk)
    assert lc.shape[0] == 2 * n_rows, "logits_chunk must have 2*n_rows rows"
    tg = np.ascontiguousarray(targets, dtype=np.int64)
    assert tg.size == n_rows
    v = lc.shape[1]
    g = np.empty((n_rows, v), np.float32) if compute_grad else None
    kl = lib().ora_kl_chunk(_p(lc, _f32p), _p(tg, _i64p), n_rows, v, kl_weight, temperature,
                            ignore_index, grad_denom, _p(g, _f32p))
    return float(np.float32(kl)), g


def kl_reference_chunk(logits_chunk, targets, n_rows, kl_weight, temperature, n_non_ignore,
                       ignore_index, compute_grad):
    """kl.rs:132-153: the mean is baked into the gradient."""
    denom = float(np.float32(max(n_non_ignore, 1)))
    return kl_chunk(logits_chunk, targets, n_rows, kl_weight, temperature, ignore_index,
                    denom, compute_grad)


# ---------------------------------------------------------------- quant
class Rng:
    """quant.rs:18-44 (SplitMix64)."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(lib().ora_rng_new(seed))

    def next_u64(self) -> int:
        return lib().ora_rng_next_u64(C.byref(self.state))

    def next_f32(self) -> float:
        return lib().ora_rng_next_f32(C.byref(self.state))


def round_half_even(x: float) -> float:
    return lib().ora_round_half_even(x)


def quantize_rowwise_int8(m):
    m = _f32(m)
    r, c = _shape2(m)
    q = np.empty((r, c), np.int8)
    s = np.empty(r, np.float32)
    lib().ora_quantize_rowwise_int8(_p(m, _f32p), r, c, _p(q, _i8p), _p(s, _f32p))
    return q, s


def quantize_rowwise_int8_stochastic(m, rng: Rng):
    m = _f32(m)
    r, c = _shape2(m)
    q = np.empty((r, c), np.int8)
    s = np.empty(r, np.float32)
    lib().ora_quantize_rowwise_int8_stochastic(_p(m, _f32p), r, c, C.byref(rng.state),
                                               _p(q, _i8p), _p(s, _f32p))
    return q, s


def dequantize(q, s):
    """QuantRows::dequantize (quant.rs:77-87)."""
    return (q.astype(np.float32) * s[:, None].astype(np.float32)).astype(np.float32)


def unique_targets(target, ignore_index: int, rows: int):
    tg = np.ascontiguousarray(target, dtype=np.int64)
    out = (C.c_size_t * max(tg.size, 1))()
    n = lib().ora_unique_targets(_p(tg, _i64p), tg.size, ignore_index, rows, out)
    return [out[i] for i in range(n)]


def quant_dequant_grad_w(grad_w, target, ignore_index: int, stochastic: bool = False,
                         seed: int = 0, grad_output: float = 1.0):
    """quantize_grad_w → dequantize_grad_w (quant.rs:157-202).
    Returns (dequantized, codes, scales)."""
    g = _f32(grad_w)
    r, c = _shape2(g)
    tg = np.ascontiguousarray(target, dtype=np.int64)
    out = np.empty_like(g)
    q = np.empty((r, c), np.int8)
    s = np.empty(r, np.float32)
    lib().ora_quant_dequant_grad_w(_p(g, _f32p), r, c, _p(tg, _i64p), tg.size, ignore_index,
                                   int(stochastic), seed, grad_output, _p(out, _f32p),
                                   _p(q, _i8p), _p(s, _f32p))
    return out, q, s


# ---------------------------------------------------------------- api
def _options(opts) -> _Options:
    o = _Options()
    lib().ora_options_default(C.byref(o))
    o.student_ce_weight = opts.student_ce_weight
    o.has_teacher_ce_weight = int(opts.teacher_ce_weight is not None)
    o.teacher_ce_weight = opts.teacher_ce_weight or 0.0
    o.kd_weight = opts.kd_weight
    o.temperature = opts.temperature
    o.ignore_index = opts.ignore_index
    o.label_smoothing = opts.label_smoothing
    o.reduction = int(opts.reduction)
    fixed = getattr(opts.chunk_size, "fixed", None)
    o.chunk_fixed = int(fixed is not None)
    o.chunk_rows = int(fixed or 0)
    o.backend = int(opts.backend)
    cfg = opts.config
    o.online_softmax = int(cfg.online_softmax)
    o.fast_math = int(cfg.fast_math)
    o.quantize_grad_weight = int(cfg.quantize_grad_weight)
    o.stochastic_rounding = int(cfg.stochastic_rounding)
    o.fp32_grad_weight_accumulation = int(cfg.fp32_grad_weight_accumulation)
    o.has_max_chunks = int(cfg.max_chunks is not None)
    o.max_chunks = int(cfg.max_chunks or 0)
    o.max_fused_size = int(cfg.max_fused_size)
    o.has_stochastic_seed = int(cfg.stochastic_seed is not None)
    o.stochastic_seed = int(cfg.stochastic_seed or 0)
    return o


def _teacher(teacher, keep: list) -> _Teacher:
    t = _Teacher()
    mode = int(teacher.mode())
    t.mode = mode
    if teacher.hidden is not None:
        h = _f32(teacher.hidden)
        keep.append(h)
        t.hidden = _p(h, _f32p)
        t.hidden_rows, t.hidden_cols = _shape2(h)
    if teacher.weight is not None:
        w = _f32(teacher.weight)
        keep.append(w)
        t.weight = _p(w, _f32p)
        t.weight_rows, t.weight_cols = _shape2(w)
    if teacher.logits is not None:
        lg = _f32(teacher.logits)
        keep.append(lg)
        t.logits = _p(lg, _f32p)
        t.logits_rows, t.logits_cols = _shape2(lg)
    return t


def distillation_loss(student_hidden, weight, labels, teacher, opts):
    """api.rs:188-422 on the CPU. Returns a namespace with the
    DistillationLossOutput fields plus per-row diagnostics and INT8 codes."""
    keep: list = []
    s = _f32(student_hidden)
    w = _f32(weight)
    lb = np.ascontiguousarray(_to_numpy(labels), dtype=np.int64)
    bt, h = _shape2(s) if s.ndim == 2 else (0, 0)
    v, wh = _shape2(w)
    t = _teacher(teacher, keep)
    o = _options(opts)
    mode = int(teacher.mode())
    ht = t.hidden_cols if mode == 1 else h
    gh = np.empty((bt, h), np.float32)
    gw = np.empty((v, wh), np.float32)
    ght = np.empty((bt, ht), np.float32)
    gwt = np.empty((v, ht), np.float32)
    rows = [np.zeros(bt, np.float32) for _ in range(3)]
    q = np.empty((v, wh), np.int8)
    qs = np.empty(v, np.float32)
    out = _Output()
    out.grad_student_hidden = _p(gh, _f32p)
    out.grad_weight = _p(gw, _f32p)
    out.grad_teacher_hidden = _p(ght, _f32p)
    out.grad_teacher_weight = _p(gwt, _f32p)
    out.row_nll_s, out.row_nll_t, out.row_kl = (_p(r, _f32p) for r in rows)
    out.q_codes = _p(q, _i8p)
    out.q_scales = _p(qs, _f32p)
    err = C.create_string_buffer(512)
    rc = lib().ora_distillation_loss(_p(s, _f32p), bt, h, _p(w, _f32p), v, wh,
                                     _p(lb, _i64p), lb.size, C.byref(t), C.byref(o),
                                     C.byref(out), err, 512)
    if rc != 0:
        raise OracleError(err.value.decode())
    quant = bool(opts.config.quantize_grad_weight)
    return SimpleNamespace(
        loss=out.loss, student_ce=out.student_ce, teacher_ce=out.teacher_ce, kl=out.kl,
        grad_student_hidden=gh, grad_weight=gw,
        grad_teacher_hidden=ght if out.has_grad_teacher_hidden else None,
        grad_teacher_weight=gwt if out.has_grad_teacher_weight else None,
        chunk_plan=SimpleNamespace(chunk_size=out.chunk_size, num_chunks=out.num_chunks),
        row_nll_student=rows[0], row_nll_teacher=rows[1], row_kl=rows[2],
        quant_codes=q if quant else None, quant_scales=qs if quant else None)


def forward_loss_f64(student_hidden, weight, labels, teacher, opts, kl_teacher_logits=None):
    """api.rs:511-572"""
    keep: list = []
    s = _f32(student_hidden)
    w = _f32(weight)
    lb = np.ascontiguousarray(_to_numpy(labels), dtype=np.int64)
    bt, h = _shape2(s)
    v, wh = _shape2(w)
    t = _teacher(teacher, keep)
    o = _options(opts)
    kt = _f32(kl_teacher_logits) if kl_teacher_logits is not None else None
    res = C.c_double()
    err = C.create_string_buffer(512)
    rc = lib().ora_forward_loss_f64(_p(s, _f32p), bt, h, _p(w, _f32p), v, wh, _p(lb, _i64p),
                                    lb.size, C.byref(t), C.byref(o), _p(kt, _f32p),
                                    C.byref(res), err, 512)
    if rc != 0:
        raise OracleError(err.value.decode())
    return res.value


def loss_only_f64(student_hidden, weight, labels, teacher, opts):
    """api.rs:576-584"""
    return forward_loss_f64(student_hidden, weight, labels, teacher, opts, None)


def teacher_logits(teacher, weight):
    """api.rs:490-496"""
    mode = int(teacher.mode())
    if mode == 0:
        return matmul_nt(teacher.hidden, weight)
    if mode == 1:
        return matmul_nt(teacher.hidden, teacher.weight)
    return _f32(teacher.logits).copy()
