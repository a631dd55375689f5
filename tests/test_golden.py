"""Frozen fixtures of tests/golden/ (written by tests/golden/make_golden.py).

* CPU: the oracle reproduces every stored output bit-for-bit from the stored
  inputs, so a change to the oracle cannot go unnoticed.
* GPU: liborda_hip.so, through the C ABI, matches the stored outputs within
  the parity tolerances of tests/parity.py (bf16 tolerances for the case whose
  inputs are bf16-rounded).
"""
import os
import sys

import numpy as np
import pytest

import oracle as O
from parity import check_grad, check_scalar, to_np

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)
import make_golden as G  # noqa: E402

CASES = sorted(G.CASES)


def load(name):
    with np.load(os.path.join(HERE, f"{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def teacher(name, d, conv=lambda a: a):
    mode = G.CASES[name][0]
    get = lambda k: conv(d[k]) if k in d else None  # noqa: E731
    return G.teacher_of(mode, get("teacher_hidden"), get("teacher_weight"), get("teacher_logits"))


@pytest.mark.parametrize("name", CASES)
def test_oracle_reproduces_fixture(name):
    d = load(name)
    out = O.distillation_loss(d["student_hidden"], d["weight"], d["labels"], teacher(name, d),
                              G.options_of(name))
    got = np.array([out.loss, out.student_ce, out.teacher_ce, out.kl], np.float32)
    assert np.array_equal(got, d["scalars"])
    assert [out.chunk_plan.chunk_size, out.chunk_plan.num_chunks] == list(d["plan"])
    for k in ("grad_student_hidden", "grad_weight", "grad_teacher_hidden", "grad_teacher_weight"):
        g = getattr(out, k)
        assert (g is None) == (k not in d), k
        if g is not None:
            assert np.array_equal(np.asarray(g), d[k]), k


def test_fixture_inputs_match_generator():
    """The stored inputs are the generator's (LCG of tests/end_to_end.rs:14-36)."""
    for name in CASES:
        d = load(name)
        s, w, y, th, tw, tl = G.inputs(name)
        assert np.array_equal(s, d["student_hidden"]) and np.array_equal(w, d["weight"])
        assert np.array_equal(y, d["labels"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_hip_matches_fixture(name):
    import torch
    import orda_hip as H
    assert torch.cuda.is_available() and H.is_available()
    d = load(name)
    bf = G.CASES[name][7]
    dev = torch.device("cuda:0")

    def conv(a):
        # bf16 cases are Tied: every float matrix is a bf16 input
        t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        return t.to(torch.bfloat16) if bf and t.is_floating_point() else t

    out = H.distillation_loss(conv(d["student_hidden"]), conv(d["weight"]),
                              torch.from_numpy(d["labels"]).to(dev), teacher(name, d, conv),
                              G.options_of(name))
    for i, k in enumerate(("loss", "student_ce", "teacher_ce", "kl")):
        check_scalar(k, getattr(out, k), float(d["scalars"][i]))
    assert [out.chunk_plan.chunk_size, out.chunk_plan.num_chunks] == list(d["plan"])
    kind = "bf16" if bf else "f32"
    quant = G.options_of(name).config.quantize_grad_weight
    for k in ("grad_student_hidden", "grad_weight", "grad_teacher_hidden", "grad_teacher_weight"):
        g = getattr(out, k)
        assert (g is None) == (k not in d), k
        if g is not None:
            # A dequantized grad_W may differ by one code step (1/127 of a row's
            # absmax) where the GPU's and the oracle's fp32 grad_W fall on
            # opposite sides of a rounding boundary: compared at 2e-2.
            check_grad(k, to_np(g), d[k], "bf16" if (quant and k == "grad_weight") else kind)
