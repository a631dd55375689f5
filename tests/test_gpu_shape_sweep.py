"""GPU parity over a seeded sweep of shapes and options, against the oracle.

Each case draws (from a fixed seed) a teacher mode, an input dtype, BT, H
(and the Separate teacher's width), V, a chunk plan, the loss weights, the
temperature, label smoothing, the reduction and a share of ignored labels.
Small cases (BT <= 96, H <= 160, V < 2600) finish in the oracle in
milliseconds; medium ones (BT up to 320, H up to 520, V up to 4200) span
several 256-wide GEMM tiles in every dimension and take about a second. The
point is the combinations: ragged K, M and N tails of every GEMM
(grad_W computed transposed over the hidden rows included), chunk plans
whose last chunk is short, staging groups of one chunk or many, odd hidden
widths that are staged with padding, the paired and unpaired row passes,
and Precomputed logits in fp32 or (every other bf16 case) bf16, read in the
logits GEMM's epilogue or converted. Tolerances as in tests/parity.py: loss
terms 1e-4 relative, gradients 1e-3 (fp32) or 2e-2 (bf16, the oracle fed
the same bf16-rounded values), chunk plans bit-exact.
"""
import os

import numpy as np
import pytest

import oracle as O
from helpers import bf16_round, normal, uniform_labels
from parity import check_output

import orda_hip as H
from orda_hip import ChunkSize, LossOptions, Reduction, Teacher

pytestmark = pytest.mark.gpu

# ORDA_SWEEP_SMALL / ORDA_SWEEP_MEDIUM draw more cases from the same generator.
N_SMALL = int(os.environ.get("ORDA_SWEEP_SMALL", 128))
N_MEDIUM = int(os.environ.get("ORDA_SWEEP_MEDIUM", 48))


def draw_case(k, medium=False):
    r = np.random.RandomState(20261202 + k + (1000 if medium else 0))
    mode = ("tied", "separate", "precomputed")[r.randint(3)]
    dtype = ("f32", "bf16")[r.randint(2)]
    if medium:
        bt = int(r.randint(97, 321))
        h = int(r.randint(161, 521))
        ht = int(r.randint(161, 521))
        v = int(r.randint(2600, 4201))
    else:
        bt = int(r.randint(1, 97))
        h = int(r.choice([int(r.randint(1, 41)), int(r.randint(41, 161))]))
        ht = int(r.randint(1, 161))
        v = int(r.choice([int(r.randint(2, 300)), int(r.randint(300, 2600))]))
    chunk = None if r.rand() < 0.3 else int(r.randint(1, bt + 1))
    w_t = None if mode == "precomputed" or r.rand() < 0.3 else float(r.choice([0.0, 0.7]))
    opts = dict(student_ce_weight=float(r.choice([1.0, 0.6])),
                teacher_ce_weight=w_t,
                kd_weight=float(r.choice([0.0, 0.5, 1.0])),
                temperature=float(r.choice([0.5, 1.0, 1.5, 3.0])),
                label_smoothing=float(r.choice([0.0, 0.1])),
                reduction=(Reduction.Mean, Reduction.Sum)[r.randint(2)],
                chunk_size=ChunkSize.Auto if chunk is None else ChunkSize.Fixed(chunk))
    ignore_every = int(r.choice([0, 3, 7]))
    return mode, dtype, bt, h, ht, v, opts, ignore_every


CASES = [draw_case(k) for k in range(N_SMALL)] + [draw_case(k, True) for k in range(N_MEDIUM)]


def case_id(c):
    mode, dtype, bt, h, ht, v, opts, ign = c
    ch = opts["chunk_size"]
    return (f"{mode}-{dtype}-bt{bt}-h{h}" + (f"-ht{ht}" if mode == "separate" else "") +
            f"-v{v}-{'auto' if ch.is_auto else 'c' + str(ch.fixed)}")


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    assert H.is_available(), "liborda_hip.so does not see a gfx950 device"
    return torch, torch.device("cuda:0")


@pytest.mark.parametrize("case", CASES, ids=[case_id(c) for c in CASES])
def test_shape_sweep(torch_dev, case):
    torch, dev = torch_dev
    mode, dtype, bt, h, ht, v, kw, ignore_every = case
    seed = bt * 7919 + h * 131 + v
    s = normal((bt, h), seed)
    w = normal((v, h), seed + 1, 0.05)
    y = uniform_labels(bt, v, seed + 2)
    if ignore_every:
        y[::ignore_every] = -100
    rnd = (lambda a: bf16_round(a)) if dtype == "bf16" else (lambda a: a)
    s, w = rnd(s), rnd(w)
    if mode == "tied":
        t = Teacher.Tied(rnd(normal((bt, h), seed + 3)))
    elif mode == "separate":
        t = Teacher.Separate(rnd(normal((bt, ht), seed + 3)), rnd(normal((v, ht), seed + 4, 0.04)))
    else:
        tl = normal((bt, v), seed + 3, 2.0)
        tl[np.arange(bt), np.maximum(y, 0)] += 4.0
        # every other case with bf16 inputs passes bf16 teacher logits (the
        # oracle gets them rounded the same way)
        tl16 = dtype == "bf16" and seed % 2 == 1
        if tl16:
            tl = bf16_round(tl)
        t = Teacher.Precomputed(tl)
    opts = LossOptions(**kw)

    def dev_t(a):
        x = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        return x.to(torch.bfloat16) if dtype == "bf16" else x

    if mode == "tied":
        tg = Teacher.Tied(dev_t(t.hidden))
    elif mode == "separate":
        tg = Teacher.Separate(dev_t(t.hidden), dev_t(t.weight))
    else:
        tl_dev = torch.from_numpy(np.ascontiguousarray(t.logits)).to(dev)
        tg = Teacher.Precomputed(tl_dev.to(torch.bfloat16) if tl16 else tl_dev)
    print(f"case {case_id(case)}", flush=True)
    got = H.distillation_loss(dev_t(s), dev_t(w), torch.from_numpy(y).to(dev), tg, opts)
    ref = O.distillation_loss(s, w, y, t, opts)
    check_output(got, ref, kind=dtype)
