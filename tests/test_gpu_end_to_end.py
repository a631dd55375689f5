"""The reference's own end-to-end tests (tests/end_to_end.rs) run against the
HIP library, as the crate's tests would run with the library behind its
`distillation_loss`: host inputs (the crate's f32 `Mat`), the library's
gradients checked against central finite differences of the oracle's float64
forward loss (tests/end_to_end.rs:43-78, tolerances as written there), chunk
invariance, component identity, sum = mean·n and the INT8 bounds.

The test bodies are those of tests/test_oracle_end_to_end.py; only the
implementation under test (the `dl` fixture) differs.
"""
import pytest

import orda_hip as H
from test_oracle_end_to_end import (  # noqa: F401  (collected here with the GPU `dl`)
    test_chunking_is_exact_invariant, test_int8_quant_grad_w_is_close_but_lossy,
    test_loss_components_and_total_are_consistent,
    test_precomputed_teacher_gradients_match_finite_difference,
    test_pure_student_ce_no_teacher_term, test_separate_teacher_gradients_match_finite_difference,
    test_sum_reduction_is_mean_times_token_count, test_tied_teacher_gradients_match_finite_difference)

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dl():
    """distillation_loss on the GPU through the C ABI, host (numpy) inputs and
    outputs."""
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    assert H.is_available(), "liborda_hip.so does not see a gfx950 device"

    def run(student, weight, labels, teacher, opts):
        return H.distillation_loss(student, weight, labels, teacher, opts)
    return run
