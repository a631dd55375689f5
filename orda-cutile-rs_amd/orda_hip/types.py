"""Python mirror of the reference crate's public types.

Names, fields, defaults and error behaviour follow the Rust crate so that a
caller (or a test) written against ``orda_cutile_rs`` reads the same here:

* ``Reduction``, ``Backend``, ``Profile``, ``KernelConfig``  — src/config.rs:10-125
* ``ChunkSize``, ``ChunkPlan``                               — src/resolver.rs:9-47
* ``Teacher``, ``TeacherMode``                               — src/teacher.rs:11-60
* ``LossOptions``                                            — src/api.rs:22-64
* ``DistillationLossOutput``                                 — src/api.rs:66-92

``Backend.Hip`` replaces the reference's ``Backend::Cuda`` slot
(src/config.rs:28-30): it selects the HIP library. ``Backend.Cpu`` is the
reference crate's own CPU path and is not served by this library.
"""
from __future__ import annotations

import enum
from dataclasses import dataclass, field
from typing import Any, Optional


class OrdaError(RuntimeError):
    """The reference's ``Err(String)``: a validation or runtime failure."""

    def __init__(self, message: str, code: int = 1):
        super().__init__(message)
        self.code = code


class Reduction(enum.IntEnum):
    """src/config.rs:10-17"""
    Mean = 0
    Sum = 1


class Backend(enum.IntEnum):
    """src/config.rs:19-31 (``Cuda`` slot is ``Hip`` here)."""
    Auto = 0
    Cpu = 1
    Hip = 2


class Profile(enum.IntEnum):
    """src/config.rs:33-42"""
    Balanced = 0
    Fast = 1
    Debug = 2


DEFAULT_MAX_FUSED_SIZE = 65536 // 2  # src/config.rs:66


def is_power_of_two(value: int) -> bool:
    """src/config.rs:123-125"""
    return value > 0 and (value & (value - 1)) == 0


@dataclass
class KernelConfig:
    """src/config.rs:45-120. On the GPU path (the reference's CPU path
    ignores the tuning fields):

    * ``fast_math`` (``Profile.Fast``): the row pass's per-row logs and
      divisions use the hardware approximations (src/config.rs:37-40,
      93-103); inputs keep their dtype, so fp32 inputs stay on the fp32
      GEMMs and match the reference to the fp32 tolerance;
    * ``profile == Profile.Debug`` (the precise preset): bf16 inputs run the
      fp32 pipeline; ``profile`` is set by ``from_profile`` (the reference
      keeps only the fields a preset sets, so this field is added);
    * ``online_softmax``: row statistics of Precomputed teacher logits that
      the logits GEMM does not read in its epilogue (fp32 inputs, or logits
      that are unaligned or at a pitch that is not a multiple of 4 (fp32) or
      8 (bf16)) by the online-softmax merge of per-thread partial
      statistics instead of a segment-wide maximum first (the
      chunk-launcher slot takes no config and always takes the maximum
      first);
    * ``fp32_grad_weight_accumulation``, ``max_fused_size``: accepted and
      validated; grad_W always accumulates in fp32.
    """
    online_softmax: bool = False
    fast_math: bool = False
    quantize_grad_weight: bool = False
    stochastic_rounding: bool = False
    fp32_grad_weight_accumulation: bool = False
    max_chunks: Optional[int] = None
    max_fused_size: int = DEFAULT_MAX_FUSED_SIZE
    stochastic_seed: Optional[int] = None
    profile: Profile = Profile.Balanced

    @staticmethod
    def from_profile(profile: Profile) -> "KernelConfig":
        return KernelConfig(fast_math=(profile == Profile.Fast), profile=Profile(profile))

    def fast_math_exp(self) -> bool:
        return self.fast_math

    def fast_math_log(self) -> bool:
        return self.fast_math

    def fast_math_mul(self) -> bool:
        return self.fast_math

    def validate(self) -> None:
        """src/config.rs:106-119 — raises OrdaError like the Rust Err."""
        if self.max_fused_size < 1 or not is_power_of_two(self.max_fused_size):
            raise OrdaError(
                f"max_fused_size must be a power of two >= 1, got {self.max_fused_size}")
        if self.max_chunks is not None and self.max_chunks < 1:
            raise OrdaError(f"max_chunks must be >= 1, got {self.max_chunks}")


class ChunkSize:
    """src/resolver.rs:9-16: ``ChunkSize.Auto`` or ``ChunkSize.Fixed(rows)``."""
    Auto: "ChunkSize"

    def __init__(self, fixed: Optional[int]):
        self.fixed = fixed

    @staticmethod
    def Fixed(rows: int) -> "ChunkSize":
        if rows < 0:
            raise ValueError("ChunkSize.Fixed takes a row count >= 0")
        return ChunkSize(int(rows))

    @property
    def is_auto(self) -> bool:
        return self.fixed is None

    def __eq__(self, other: object) -> bool:
        return isinstance(other, ChunkSize) and other.fixed == self.fixed

    def __hash__(self) -> int:
        return hash(("ChunkSize", self.fixed))

    def __repr__(self) -> str:
        return "ChunkSize.Auto" if self.fixed is None else f"ChunkSize.Fixed({self.fixed})"


ChunkSize.Auto = ChunkSize(None)


@dataclass(frozen=True)
class ChunkPlan:
    """src/resolver.rs:39-46"""
    chunk_size: int
    num_chunks: int


class TeacherMode(enum.IntEnum):
    """src/teacher.rs:34-40"""
    Tied = 0
    Separate = 1
    Precomputed = 2


class Teacher:
    """src/teacher.rs:11-32. Build with ``Teacher.Tied(hidden)``,
    ``Teacher.Separate(hidden, weight)`` or ``Teacher.Precomputed(logits)``.
    The matrices are torch tensors or numpy arrays, row-major."""

    def __init__(self, mode: TeacherMode, hidden: Any = None, weight: Any = None,
                 logits: Any = None):
        self._mode = TeacherMode(mode)
        self.hidden = hidden
        self.weight = weight
        self.logits = logits

    @staticmethod
    def Tied(hidden: Any) -> "Teacher":
        return Teacher(TeacherMode.Tied, hidden=hidden)

    @staticmethod
    def Separate(hidden: Any, weight: Any) -> "Teacher":
        return Teacher(TeacherMode.Separate, hidden=hidden, weight=weight)

    @staticmethod
    def Precomputed(logits: Any) -> "Teacher":
        return Teacher(TeacherMode.Precomputed, logits=logits)

    def mode(self) -> TeacherMode:
        return self._mode

    def default_teacher_ce_weight(self) -> float:
        """src/teacher.rs:54-59"""
        return 1.0 if self._mode == TeacherMode.Tied else 0.0


@dataclass
class LossOptions:
    """src/api.rs:25-64 (defaults at :49-64)."""
    student_ce_weight: float = 1.0
    teacher_ce_weight: Optional[float] = None
    kd_weight: float = 0.0
    temperature: float = 1.0
    ignore_index: int = -100
    label_smoothing: float = 0.0
    reduction: Reduction = Reduction.Mean
    chunk_size: ChunkSize = field(default_factory=lambda: ChunkSize.Auto)
    config: KernelConfig = field(default_factory=KernelConfig)
    backend: Backend = Backend.Auto


@dataclass
class DistillationLossOutput:
    """src/api.rs:71-92, plus optional diagnostics that the reference keeps
    internal: per-row losses and the INT8 codes/scales of ``grad_weight``
    (``QuantRows``, src/quant.rs:66-73)."""
    loss: float
    student_ce: float
    teacher_ce: float
    kl: float
    grad_student_hidden: Any
    grad_weight: Any
    grad_teacher_hidden: Any
    grad_teacher_weight: Any
    chunk_plan: ChunkPlan
    row_nll_student: Any = None
    row_nll_teacher: Any = None
    row_kl: Any = None
    quant_codes: Any = None
    quant_scales: Any = None
