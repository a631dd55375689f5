"""ctypes declarations of include/orda/orda.h and the loader of liborda_hip.so.

The library is built in place by ``__graft_entry__.build()`` (or
``make -C orda-cutile-rs_amd``). Loading fails loudly when it is missing:
there is no CPU fallback. ``ORDA_HIP_LIB`` names another build of the same
library to load instead (the sanitizer build of the host code).
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("ORDA_HIP_LIB") or os.path.join(_HERE, "liborda_hip.so")

ORDA_OK = 0
ORDA_ERR_INVALID = 1
ORDA_ERR_OOM = 2
ORDA_ERR_HIP = 3
ORDA_ERR_UNAVAILABLE = 4
ORDA_ERR_INTERNAL = 5

F32, BF16, I8 = 0, 1, 2
HOST, DEVICE = 0, 1

KERNEL_KINDS = {
    "gemm_logits": 0,
    "row_pass": 1,
    "gemm_grad_hidden": 2,
    "gemm_grad_weight": 3,
    "quant": 4,
    "other": 5,
}


class Tensor(C.Structure):
    _fields_ = [("data", C.c_void_p), ("rows", C.c_int64), ("cols", C.c_int64),
                ("ld", C.c_int64), ("dtype", C.c_int32), ("location", C.c_int32)]


class TeacherC(C.Structure):
    _fields_ = [("mode", C.c_int32), ("hidden", Tensor), ("weight", Tensor), ("logits", Tensor)]


class KernelConfigC(C.Structure):
    _fields_ = [("online_softmax", C.c_int32), ("fast_math", C.c_int32),
                ("quantize_grad_weight", C.c_int32), ("stochastic_rounding", C.c_int32),
                ("fp32_grad_weight_accumulation", C.c_int32), ("has_max_chunks", C.c_int32),
                ("max_chunks", C.c_int64), ("max_fused_size", C.c_int64),
                ("has_stochastic_seed", C.c_int32), ("stochastic_seed", C.c_uint64),
                ("profile", C.c_int32)]


class LossOptionsC(C.Structure):
    _fields_ = [("student_ce_weight", C.c_float), ("has_teacher_ce_weight", C.c_int32),
                ("teacher_ce_weight", C.c_float), ("kd_weight", C.c_float),
                ("temperature", C.c_float), ("ignore_index", C.c_int64),
                ("label_smoothing", C.c_float), ("reduction", C.c_int32),
                ("chunk_fixed", C.c_int32), ("chunk_rows", C.c_int64),
                ("config", KernelConfigC), ("backend", C.c_int32)]


class LossOutputC(C.Structure):
    _fields_ = [("loss", C.c_float), ("student_ce", C.c_float), ("teacher_ce", C.c_float),
                ("kl", C.c_float),
                ("grad_student_hidden", Tensor), ("grad_weight", Tensor),
                ("grad_teacher_hidden", Tensor), ("grad_teacher_weight", Tensor),
                ("has_grad_teacher_hidden", C.c_int32), ("has_grad_teacher_weight", C.c_int32),
                ("chunk_size", C.c_int64), ("num_chunks", C.c_int64),
                ("row_nll_student", Tensor), ("row_nll_teacher", Tensor), ("row_kl", Tensor),
                ("quant_codes", Tensor), ("quant_scales", Tensor)]


# (name, restype, argtypes) for every entry point of include/orda/orda.h.
SIGNATURES = [
    ("orda_abi_version", C.c_int32, []),
    ("orda_is_available", C.c_int32, []),
    ("orda_loss_options_default", None, [C.POINTER(LossOptionsC)]),
    ("orda_kernel_config_from_profile", None, [C.c_int32, C.POINTER(KernelConfigC)]),
    ("orda_kernel_config_validate", C.c_int32,
     [C.POINTER(KernelConfigC), C.c_char_p, C.c_size_t]),
    ("orda_resolve_chunk_size", C.c_int32,
     [C.c_int64, C.c_int32, C.c_int64, C.c_int32, C.c_int64, C.c_int32, C.c_int64,
      C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
    ("orda_chunks_from_raw", C.c_int64, [C.c_double]),
    ("orda_default_max_chunks_limit", C.c_int64, [C.c_int64]),
    ("orda_chunk_doubling_schedule", C.c_int64,
     [C.c_int64, C.c_int64, C.c_int64, C.POINTER(C.c_int64), C.c_int64]),
    ("orda_ctx_create", C.c_int32, [C.c_int32, C.POINTER(C.c_void_p), C.c_char_p, C.c_size_t]),
    ("orda_ctx_destroy", None, [C.c_void_p]),
    ("orda_ctx_set_stream", C.c_int32, [C.c_void_p, C.c_void_p]),
    ("orda_ctx_set_memory_limit", C.c_int32, [C.c_void_p, C.c_int64]),
    ("orda_ctx_set_staging_budget", C.c_int32, [C.c_void_p, C.c_int64]),
    ("orda_ctx_trim", C.c_int32, [C.c_void_p]),
    ("orda_ctx_workspace_bytes", C.c_int32, [C.c_void_p, C.POINTER(C.c_int64)]),
    ("orda_ctx_set_timing", C.c_int32, [C.c_void_p, C.c_int32]),
    ("orda_ctx_get_kernel_time", C.c_int32,
     [C.c_void_p, C.c_int32, C.POINTER(C.c_double), C.POINTER(C.c_int64)]),
    ("orda_ctx_reset_kernel_time", C.c_int32, [C.c_void_p]),
    ("orda_distillation_loss", C.c_int32,
     [C.c_void_p, C.POINTER(Tensor), C.POINTER(Tensor), C.c_void_p, C.c_int64, C.c_int32,
      C.POINTER(TeacherC), C.POINTER(LossOptionsC), C.POINTER(LossOutputC), C.c_char_p,
      C.c_size_t]),
    ("orda_kl_ce_on_logits_chunk", C.c_int32,
     [C.c_void_p, C.POINTER(Tensor), C.c_void_p, C.c_int32, C.c_int64, C.c_float, C.c_float,
      C.c_float, C.c_float, C.c_float, C.c_float, C.c_int32, C.c_int32, C.c_int32,
      C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor), C.c_char_p,
      C.c_size_t]),
    ("orda_kl_ce_on_logits_chunk_noalloc", C.c_int32,
     [C.c_void_p, C.POINTER(Tensor), C.c_void_p, C.c_int32, C.c_int64, C.c_float, C.c_float,
      C.c_float, C.c_float, C.c_float, C.c_float, C.c_int32, C.c_int32, C.c_int32,
      C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor), C.c_char_p,
      C.c_size_t]),
    ("orda_quant_rows_int8", C.c_int32,
     [C.c_void_p, C.POINTER(Tensor), C.c_void_p, C.c_int64, C.c_int32, C.c_int64, C.c_int32,
      C.c_uint64, C.c_float, C.POINTER(Tensor), C.POINTER(Tensor), C.POINTER(Tensor),
      C.c_char_p, C.c_size_t]),
]

_lib = None


def load():
    """Load liborda_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with __graft_entry__.build() or "
                "`make -C orda-cutile-rs_amd`; there is no CPU fallback")
        lib = C.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            f = getattr(lib, name)
            f.restype = res
            f.argtypes = args
        _lib = lib
    return _lib
