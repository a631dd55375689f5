"""GPU parity over a seeded sweep of the kernel configuration and of the ways
inputs and outputs reach the library, against the oracle.

Each case draws (from a fixed seed) a teacher mode, an input dtype and a
small or medium shape (the ranges of tests/test_gpu_shape_sweep.py), the loss
options, and then:
* the profile switches of KernelConfig (src/config.rs:45-103): Balanced,
  fast_math, online_softmax, both, and for bf16 inputs Profile.Debug (the
  fp32 pipeline on the widened inputs, held to the fp32 gate);
* INT8 grad_W quantization (src/quant.rs:147-202), round-half-even or
  stochastic with a drawn seed: the quantized call's codes, scales and
  grad_W must be those of the oracle's quantizer applied to the same call's
  grad_W with quantization off (the step "mean-scale, then quantize the
  final grad_W" of src/api.rs:380-399), and that fp32 gradient is held to
  the oracle;
* where the inputs live: contiguous device tensors, device views into wider
  tensors (a row pitch above the width and an offset base), or host tensors;
* where the gradients go: fresh buffers, or device views into wider buffers
  filled with a sentinel that must be unchanged outside the views after the
  call (no write leaves an output's rows);
* labels on the device or on the host.

Tolerances as in tests/parity.py: loss terms 1e-4 relative, gradients 1e-3
(fp32 and Debug) or 2e-2 (bf16, the oracle fed the same bf16-rounded
values), chunk plans bit-exact, INT8 codes and scales exact.
"""
import os
from dataclasses import replace

import numpy as np
import pytest

import oracle as O
from helpers import bf16_round, normal, uniform_labels
from parity import check_output, check_quant_of_own_gradient, to_np

import orda_hip as H
from orda_hip import ChunkSize, KernelConfig, LossOptions, Profile, Reduction, Teacher

pytestmark = pytest.mark.gpu

# ORDA_OPTION_SWEEP draws more cases from the same generator.
N_CASES = int(os.environ.get("ORDA_OPTION_SWEEP", 128))
SENTINEL = 12345.0


def draw_case(k):
    r = np.random.RandomState(777001 + k)
    mode = ("tied", "separate", "precomputed")[r.randint(3)]
    dtype = ("f32", "bf16")[r.randint(2)]
    if r.rand() < 0.3:
        bt, h, ht, v = (int(r.randint(97, 321)), int(r.randint(161, 521)),
                        int(r.randint(161, 521)), int(r.randint(2600, 4201)))
    else:
        bt, h, ht = int(r.randint(1, 97)), int(r.randint(1, 161)), int(r.randint(1, 161))
        v = int(r.choice([int(r.randint(2, 300)), int(r.randint(300, 2600))]))
    chunk = None if r.rand() < 0.4 else int(r.randint(1, bt + 1))
    w_t = None if mode == "precomputed" or r.rand() < 0.3 else float(r.choice([0.0, 0.7]))
    profile = ("balanced", "fast", "online", "fast+online", "debug")[r.randint(4 + (dtype == "bf16"))]
    quant = ("none", "rne", "stochastic")[r.randint(3)]
    case = dict(mode=mode, dtype=dtype, bt=bt, h=h, ht=ht, v=v, chunk=chunk,
                w_s=float(r.choice([1.0, 0.6])), w_t=w_t, kd=float(r.choice([0.0, 0.5, 1.0])),
                T=float(r.choice([0.5, 1.0, 1.5, 3.0])), ls=float(r.choice([0.0, 0.1])),
                sum=bool(r.randint(2)), ignore_every=int(r.choice([0, 3, 7])),
                profile=profile, quant=quant, qseed=int(r.randint(1, 1 << 30)),
                inputs=("device", "view", "host")[r.randint(3)],
                outputs=("fresh", "view")[r.randint(2)],
                labels=("device", "host")[r.randint(2)],
                pad=int(r.choice([1, 3, 8, 64])), seed=int(r.randint(1 << 20)))
    if case["inputs"] == "host":
        case["outputs"] = "fresh"     # host inputs take host outputs
    return case


CASES = [draw_case(k) for k in range(N_CASES)]


def case_id(c):
    return (f"{c['mode']}-{c['dtype']}-bt{c['bt']}-h{c['h']}" +
            (f"-ht{c['ht']}" if c["mode"] == "separate" else "") +
            f"-v{c['v']}-{c['profile']}-q{c['quant']}-{c['inputs']}-{c['outputs']}-"
            f"lab{c['labels']}")


def config_of(c):
    if c["profile"] == "debug":
        cfg = KernelConfig.from_profile(Profile.Debug)
    else:
        cfg = KernelConfig(fast_math="fast" in c["profile"],
                           online_softmax="online" in c["profile"])
    cfg.quantize_grad_weight = c["quant"] != "none"
    cfg.stochastic_rounding = c["quant"] == "stochastic"
    cfg.stochastic_seed = c["qseed"] if c["quant"] == "stochastic" else None
    return cfg


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    assert H.is_available(), "liborda_hip.so does not see a gfx950 device"
    return torch, torch.device("cuda:0")


@pytest.mark.parametrize("case", CASES, ids=[case_id(c) for c in CASES])
def test_option_sweep(torch_dev, case):
    torch, dev = torch_dev
    c = case
    mode, dtype, bt, h, ht, v, seed = c["mode"], c["dtype"], c["bt"], c["h"], c["ht"], c["v"], c["seed"]
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float32
    rnd = bf16_round if dtype == "bf16" else (lambda a: a)
    s = rnd(normal((bt, h), seed))
    w = rnd(normal((v, h), seed + 1, 0.05))
    y = uniform_labels(bt, v, seed + 2)
    if c["ignore_every"]:
        y[::c["ignore_every"]] = -100
    if mode == "tied":
        t = Teacher.Tied(rnd(normal((bt, h), seed + 3)))
    elif mode == "separate":
        t = Teacher.Separate(rnd(normal((bt, ht), seed + 3)), rnd(normal((v, ht), seed + 4, 0.04)))
    else:
        tl = normal((bt, v), seed + 3, 2.0)
        tl[np.arange(bt), np.maximum(y, 0)] += 4.0
        t = Teacher.Precomputed(tl)
    opts = LossOptions(student_ce_weight=c["w_s"], teacher_ce_weight=c["w_t"], kd_weight=c["kd"],
                       temperature=c["T"], label_smoothing=c["ls"],
                       reduction=Reduction.Sum if c["sum"] else Reduction.Mean,
                       chunk_size=ChunkSize.Auto if c["chunk"] is None else ChunkSize.Fixed(c["chunk"]),
                       config=config_of(c))

    def put(a, dt=tdt):
        """The library's view of a host matrix, as the case places it."""
        x = torch.from_numpy(np.ascontiguousarray(a))
        if c["inputs"] == "host":
            return x.to(dt)
        x = x.to(dev).to(dt)
        if c["inputs"] == "device":
            return x
        big = torch.full((x.shape[0] + 2, x.shape[1] + c["pad"]), float("nan"), device=dev, dtype=dt)
        view = big[1:1 + x.shape[0], c["pad"]:c["pad"] + x.shape[1]]
        view.copy_(x)
        return view

    if mode == "tied":
        tg = Teacher.Tied(put(t.hidden))
    elif mode == "separate":
        tg = Teacher.Separate(put(t.hidden), put(t.weight))
    else:
        tg = Teacher.Precomputed(put(t.logits, torch.float32))
    yl = y if c["labels"] == "host" else torch.from_numpy(y).to(dev)
    if c["inputs"] == "host" and c["labels"] == "device":
        yl = y     # host inputs with host labels

    bufs = {}

    def outputs():
        """Gradient buffers: none (the library's wrapper allocates), or views
        into sentinel-filled wider buffers."""
        if c["outputs"] == "fresh":
            return None
        shapes = {"grad_student_hidden": (bt, h), "grad_weight": (v, h)}
        if c["w_t"] != 0.0 and mode != "precomputed" and (c["w_t"] is not None or mode == "tied"):
            shapes["grad_teacher_hidden"] = (bt, ht if mode == "separate" else h)
            if mode == "separate":
                shapes["grad_teacher_weight"] = (v, ht)
        out = {}
        for k, (r_, c_) in shapes.items():
            big = torch.full((r_ + 2, c_ + c["pad"]), SENTINEL, device=dev, dtype=torch.float32)
            bufs[k] = big
            out[k] = big[1:1 + r_, c["pad"]:c["pad"] + c_]
        return out

    def guards_intact():
        for k, big in bufs.items():
            mask = torch.ones_like(big, dtype=torch.bool)
            r_, c_ = big.shape[0] - 2, big.shape[1] - c["pad"]
            mask[1:1 + r_, c["pad"]:c["pad"] + c_] = False
            assert bool((big[mask] == SENTINEL).all()), f"{k}: a write left the output's view"

    print(f"case {case_id(c)}", flush=True)
    quant = c["quant"] != "none"
    ref_opts = opts
    if quant:
        # the fp32 gradient of the same call, held to the oracle
        plain = replace(opts, config=replace(opts.config, quantize_grad_weight=False,
                                             stochastic_rounding=False, stochastic_seed=None))
        got_plain = H.distillation_loss(put(s), put(w), yl, tg, plain, outputs=outputs())
        guards_intact()
        plain_gw = to_np(got_plain.grad_weight).copy()
        ref_opts = plain
        bufs.clear()
        got = H.distillation_loss(put(s), put(w), yl, tg, opts, outputs=outputs(), quant_codes=True)
        guards_intact()
        check_quant_of_own_gradient(got, plain_gw, y, stochastic=c["quant"] == "stochastic",
                                    seed=c["qseed"])
        got = got_plain
    else:
        got = H.distillation_loss(put(s), put(w), yl, tg, opts, outputs=outputs())
        guards_intact()
    ref = O.distillation_loss(s, w, y, t, ref_opts)
    kind = "f32" if dtype == "f32" or c["profile"] == "debug" else "bf16"
    check_output(got, ref, kind=kind)
