"""The C++ mirror of the crate's API (include/orda/orda.hpp) on the GPU: the
prebuilt tests/cpp/_build/api_test (built by __graft_entry__.build(), linked
against the in-tree liborda_hip.so) runs the reference's end-to-end scenarios
(tests/end_to_end.rs) through orda::distillation_loss on host Mats.

* The assertions tests/end_to_end.rs makes without an f64 forward, in C++ at
  the reference's own tolerances: chunk invariance (1e-5), total = w_s·CE_s +
  w_t·CE_t + kd·KL (1e-4), sum = mean·n (1e-3), INT8 grad_W close but lossy
  and equal to orda::quant_dequant_grad_w of the unquantized gradient, no
  teacher term when kd = w_t = 0.
* The gradient scenarios' outputs (Tied, Separate, Precomputed as in
  tests/end_to_end.rs:89-204, and a Tied 300x70x1000 shape spanning several
  GEMM tiles) against the oracle on the same inputs (tests/helpers.py
  restates the reference's fill/labels generators bit for bit) at the fp32
  gate of tests/parity.py; the INT8 codes and scales bit-exact against the
  oracle's quantizer; the chunk-launcher slot against the same call through
  the Python binding.
"""
import json
import os
import subprocess

import numpy as np
import pytest

import oracle as O
from helpers import labels, mat
from parity import check_output

import orda_hip as H
from orda_hip import ChunkSize, LossOptions, Teacher

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "_build", "api_test")


@pytest.fixture(scope="module")
def run(tmp_path_factory):
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    assert os.path.exists(EXE), "tests/cpp/_build/api_test is not built (run __graft_entry__.build())"
    d = tmp_path_factory.mktemp("cpp_gpu")
    print("running the C++ API program", flush=True)
    r = subprocess.run([EXE, "gpu", str(d)], capture_output=True, text=True, timeout=300)
    assert r.stdout.strip(), r.stderr
    return r.returncode, json.loads(r.stdout), d


def base_opts(**kw):
    return LossOptions(student_ce_weight=1.0, kd_weight=0.5, temperature=1.5, **kw)


def scenarios():
    """The inputs api_test.cpp builds, regenerated here."""
    return {
        "tied": (mat(6, 5, 1, 0.3), mat(7, 5, 2, 0.2), labels(6, 7, 4),
                 Teacher.Tied(mat(6, 5, 3, 0.3)), base_opts(teacher_ce_weight=1.0, label_smoothing=0.1)),
        "separate": (mat(6, 5, 11, 0.3), mat(7, 5, 12, 0.2), labels(6, 7),
                     Teacher.Separate(mat(6, 4, 13, 0.3), mat(7, 4, 14, 0.2)),
                     base_opts(teacher_ce_weight=0.7)),
        "precomputed": (mat(6, 5, 21, 0.3), mat(7, 5, 22, 0.2), labels(6, 7, 5),
                        Teacher.Precomputed(mat(6, 7, 23, 0.5)), base_opts()),
        "tied_300x70x1000": (mat(300, 70, 81, 1.0), mat(1000, 70, 82, 0.1), labels(300, 1000, 9),
                             Teacher.Tied(mat(300, 70, 83, 1.0)),
                             base_opts(teacher_ce_weight=1.0, label_smoothing=0.1,
                                       chunk_size=ChunkSize.Fixed(100))),
    }


class _Out:
    pass


def load(d, rec):
    o = _Out()
    for k in ("loss", "student_ce", "teacher_ce", "kl"):
        setattr(o, k, rec[k])
    for k in ("grad_student_hidden", "grad_weight", "grad_teacher_hidden", "grad_teacher_weight"):
        if k in rec:
            f, r, c = rec[k]
            setattr(o, k, np.fromfile(os.path.join(d, f), np.float32).reshape(r, c))
        else:
            setattr(o, k, None)
    o.chunk_plan = type("P", (), {"chunk_size": rec["chunk_plan"][0],
                                  "num_chunks": rec["chunk_plan"][1]})()
    return o


def test_cpp_reference_assertions_pass(run):
    rc, out, _ = run
    assert out["failures"] == [] and rc == 0


@pytest.mark.parametrize("name", ["tied", "separate", "precomputed", "tied_300x70x1000"])
def test_cpp_scenarios_match_the_oracle(run, name):
    _, out, d = run
    s, w, y, t, opts = scenarios()[name]
    ref = O.distillation_loss(s, w, y, t, opts)
    check_output(load(d, out["scenarios"][name]), ref, kind="f32")


def test_cpp_components_match_the_oracle(run):
    _, out, _ = run
    opts = LossOptions(student_ce_weight=1.0, teacher_ce_weight=0.8, kd_weight=0.5, temperature=2.0)
    ref = O.distillation_loss(mat(10, 4, 51, 0.3), mat(8, 4, 52, 0.2), labels(10, 8),
                              Teacher.Tied(mat(10, 4, 53, 0.3)), opts)
    assert abs(out["components"]["loss"] - ref.loss) <= 1e-4 * abs(ref.loss) + 2e-6


def test_cpp_quantizer_matches_the_oracle(run):
    _, _, d = run
    gw = np.fromfile(os.path.join(d, "quant.grad_w.f32"), np.float32).reshape(20, 4)
    deq, q, s = O.quant_dequant_grad_w(gw, labels(8, 20), -100)
    np.testing.assert_array_equal(np.fromfile(os.path.join(d, "quant.codes.i8"), np.int8).reshape(20, 4), q)
    np.testing.assert_array_equal(np.fromfile(os.path.join(d, "quant.scales.f32"), np.float32),
                                  np.asarray(s, np.float32).reshape(-1))
    np.testing.assert_array_equal(np.fromfile(os.path.join(d, "quant.deq.f32"), np.float32).reshape(20, 4), deq)


def test_cpp_slot_matches_the_python_binding(run):
    _, out, _ = run
    lc = np.array([[0.1, 0.2, 0.3, -1.0, 2.0], [1.0, -0.5, 0.0, 0.7, 0.2]], np.float32)
    ref = H.kl_ce_on_logits_chunk(lc, np.array([4], np.int32), 1, np.float32(1.0 / 1.5), 0.6, 2.25,
                                  1.0, 1.0, 0.1, -100, False, True)
    got = out["slot"]
    assert np.float32(got["kl_per_row"]) == np.float32(ref["kl_per_row"][0])
    np.testing.assert_array_equal(np.float32(got["ce_loss"]), np.asarray(ref["ce_loss"], np.float32))
    np.testing.assert_array_equal(np.float32(got["grad_kl_student"]),
                                  np.asarray(ref["grad_kl_student"], np.float32).reshape(-1))
    np.testing.assert_array_equal(np.float32(got["grad_ce"]),
                                  np.asarray(ref["grad_ce"], np.float32).reshape(-1))
