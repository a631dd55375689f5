#!/usr/bin/env python3
"""Writes the frozen fixtures of tests/golden/: small inputs (the reference
tests' LCG, tests/end_to_end.rs:14-36) and the oracle's outputs for every
teacher mode, both reductions, label smoothing, ignored rows, bf16-rounded
inputs and both INT8 modes.

The reference crate ships no golden files, so these come from this
repository's oracle. They freeze its outputs: test_golden.py checks that the
oracle still reproduces them bit-for-bit and that the HIP path matches them
within the parity tolerances.

Run from the repository root after `make -C oracle`:
    python3 tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "tests"), os.path.join(ROOT, "oracle"),
                os.path.join(ROOT, "orda-cutile-rs_amd")]

import oracle as O                                        # noqa: E402
from helpers import bf16_round, labels, mat              # noqa: E402
from orda_hip.types import (ChunkSize, KernelConfig, LossOptions, Reduction,  # noqa: E402
                            Teacher)

# name: (mode, bt, h, ht, v, ignore_every, options, bf16)
CASES = {
    "tied_kd_mean": ("tied", 24, 40, 40, 136, 5,
                     dict(kd_weight=0.4, temperature=1.5, chunk_size=ChunkSize.Fixed(8)), False),
    "tied_smooth_sum": ("tied", 20, 32, 32, 200, None,
                        dict(kd_weight=0.7, temperature=2.0, label_smoothing=0.1,
                             reduction=Reduction.Sum), False),
    "separate_tce": ("separate", 17, 24, 48, 120, 4,
                     dict(kd_weight=0.5, temperature=2.0, label_smoothing=0.1,
                          teacher_ce_weight=1.0, chunk_size=ChunkSize.Fixed(6)), False),
    "precomputed": ("precomputed", 19, 32, 32, 160, 6,
                    dict(kd_weight=0.7, temperature=1.0), False),
    "tied_bf16_int8": ("tied", 32, 48, 48, 256, 7,
                       dict(kd_weight=0.4, temperature=1.5, label_smoothing=0.1,
                            config=KernelConfig(quantize_grad_weight=True)), True),
    "tied_int8_stochastic": ("tied", 16, 32, 32, 96, None,
                             dict(kd_weight=0.3, temperature=1.2,
                                  config=KernelConfig(quantize_grad_weight=True,
                                                      stochastic_rounding=True,
                                                      stochastic_seed=12345)), False),
}


def inputs(name):
    mode, bt, h, ht, v, ign, _, bf = CASES[name]
    s = mat(bt, h, 11, 1.0)
    w = mat(v, h, 12, 0.2)
    y = labels(bt, v, ign)
    th = tw = tl = None
    if mode == "tied":
        th = mat(bt, h, 13, 1.0)
    elif mode == "separate":
        th = mat(bt, ht, 13, 1.0)
        tw = mat(v, ht, 14, 0.15)
    else:
        tl = mat(bt, v, 15, 2.0)
        for i in range(bt):
            if y[i] >= 0:
                tl[i, y[i]] += np.float32(4.0)
    if bf:
        s, w = bf16_round(s), bf16_round(w)
        th = None if th is None else bf16_round(th)
        tw = None if tw is None else bf16_round(tw)
    return s, w, y, th, tw, tl


def teacher_of(mode, th, tw, tl):
    if mode == "tied":
        return Teacher.Tied(th)
    if mode == "separate":
        return Teacher.Separate(th, tw)
    return Teacher.Precomputed(tl)


def options_of(name):
    return LossOptions(**CASES[name][6])


def main():
    for name, (mode, *_rest) in CASES.items():
        s, w, y, th, tw, tl = inputs(name)
        out = O.distillation_loss(s, w, y, teacher_of(mode, th, tw, tl), options_of(name))
        arrays = {"student_hidden": s, "weight": w, "labels": y,
                  "scalars": np.array([out.loss, out.student_ce, out.teacher_ce, out.kl],
                                      np.float32),
                  "plan": np.array([out.chunk_plan.chunk_size, out.chunk_plan.num_chunks],
                                   np.int64),
                  "grad_student_hidden": out.grad_student_hidden,
                  "grad_weight": out.grad_weight}
        for k, a in (("teacher_hidden", th), ("teacher_weight", tw), ("teacher_logits", tl),
                     ("grad_teacher_hidden", out.grad_teacher_hidden),
                     ("grad_teacher_weight", out.grad_teacher_weight)):
            if a is not None:
                arrays[k] = np.asarray(a)
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **arrays)
        print(f"{name}: loss {out.loss:.6f} plan {out.chunk_plan}")


if __name__ == "__main__":
    main()
