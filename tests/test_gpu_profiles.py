"""GPU parity of the KernelConfig / Profile switches (src/config.rs:45-103),
each against the oracle with its tolerance stated here:

* Profile.Fast (fast_math) on fp32 inputs: only the row pass's per-row
  logs and divisions change (hardware approximations, src/config.rs:37-40);
  the inputs stay fp32 and run the fp32 pipeline. It must match the oracle
  run on the caller's own fp32 inputs at the fp32 gate: loss terms 1e-4
  relative, gradients 1e-3.
* fast_math on bf16 inputs: the same change; the bf16 gate holds.
* Profile.Debug on bf16 inputs: the inputs are widened and the fp32
  pipeline runs; it must match the oracle on the same bf16 values at the
  fp32 gate: loss terms 1e-4, gradients 1e-3.
* online_softmax on and off for Precomputed teacher logits (whose row
  statistics are not formed by the GEMM): fp32 gate either way.
"""
import dataclasses

import numpy as np
import pytest

import oracle as O
from helpers import bf16_round, normal, uniform_labels
from parity import check_output

import orda_hip as H
from orda_hip import ChunkSize, KernelConfig, LossOptions, Profile, Teacher

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    assert H.is_available(), "liborda_hip.so does not see a gfx950 device"
    return torch, torch.device("cuda:0")


def gpu(torch_dev, a, dtype=None):
    torch, dev = torch_dev
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t.to(torch.bfloat16) if dtype == "bf16" else t


def inputs(mode, bt=384, h=96, ht=80, v=3001, seed=300):
    s = normal((bt, h), seed)
    w = normal((v, h), seed + 1, 0.04)
    y = uniform_labels(bt, v, seed + 2)
    y[::11] = -100
    if mode == "tied":
        t = Teacher.Tied(normal((bt, h), seed + 3))
    elif mode == "separate":
        t = Teacher.Separate(normal((bt, ht), seed + 3), normal((v, ht), seed + 4, 0.03))
    else:
        tl = normal((bt, v), seed + 3, 2.0)
        tl[np.arange(bt), np.maximum(y, 0)] += 8.0
        t = Teacher.Precomputed(tl)
    return s, w, y, t


def rounded(teacher):
    return Teacher(teacher.mode(), hidden=None if teacher.hidden is None else bf16_round(teacher.hidden),
                   weight=None if teacher.weight is None else bf16_round(teacher.weight),
                   logits=teacher.logits)


def on_gpu(torch_dev, teacher, dtype=None):
    m = teacher.mode()
    if m == H.TeacherMode.Tied:
        return Teacher.Tied(gpu(torch_dev, teacher.hidden, dtype))
    if m == H.TeacherMode.Separate:
        return Teacher.Separate(gpu(torch_dev, teacher.hidden, dtype),
                                gpu(torch_dev, teacher.weight, dtype))
    return Teacher.Precomputed(gpu(torch_dev, teacher.logits))


def opts_for(mode, config):
    return LossOptions(kd_weight=0.5, temperature=1.7, label_smoothing=0.1,
                       teacher_ce_weight=0.8 if mode != "precomputed" else None,
                       chunk_size=ChunkSize.Fixed(128), config=config)


@pytest.mark.parametrize("mode", ["tied", "separate", "precomputed"])
def test_fast_profile_fp32_inputs_match_the_oracle_on_the_callers_inputs(torch_dev, mode):
    s, w, y, t = inputs(mode)
    opts = opts_for(mode, KernelConfig.from_profile(Profile.Fast))
    assert opts.config.fast_math and opts.config.profile == Profile.Fast
    got = H.distillation_loss(gpu(torch_dev, s), gpu(torch_dev, w), gpu(torch_dev, y),
                              on_gpu(torch_dev, t), opts)
    ref = O.distillation_loss(s, w, y, t, opts)   # the caller's own fp32 inputs
    check_output(got, ref, kind="f32")
    balanced = H.distillation_loss(gpu(torch_dev, s), gpu(torch_dev, w), gpu(torch_dev, y),
                                   on_gpu(torch_dev, t), opts_for(mode, KernelConfig()))
    print(f"{mode}: loss Fast {got.loss:.8f}, Balanced {balanced.loss:.8f}, "
          f"oracle {ref.loss:.8f} (Fast rel {abs(got.loss - ref.loss) / ref.loss:.2e})")


def test_fast_math_bf16_inputs(torch_dev):
    s, w, y, t = inputs("tied", seed=310)
    s, w, t = bf16_round(s), bf16_round(w), rounded(t)
    opts = opts_for("tied", KernelConfig(fast_math=True))
    got = H.distillation_loss(gpu(torch_dev, s, "bf16"), gpu(torch_dev, w, "bf16"),
                              gpu(torch_dev, y), on_gpu(torch_dev, t, "bf16"), opts)
    ref = O.distillation_loss(s, w, y, t, opts)
    check_output(got, ref, kind="bf16")


@pytest.mark.parametrize("mode", ["tied", "separate", "precomputed"])
def test_debug_profile_bf16_inputs_run_the_fp32_pipeline(torch_dev, mode):
    s, w, y, t = inputs(mode, seed=320)
    s, w, t = bf16_round(s), bf16_round(w), rounded(t)
    opts = opts_for(mode, KernelConfig.from_profile(Profile.Debug))
    assert not opts.config.fast_math and opts.config.profile == Profile.Debug
    got = H.distillation_loss(gpu(torch_dev, s, "bf16"), gpu(torch_dev, w, "bf16"),
                              gpu(torch_dev, y), on_gpu(torch_dev, t, "bf16"), opts)
    ref = O.distillation_loss(s, w, y, t, opts)
    check_output(got, ref, kind="f32")


@pytest.mark.parametrize("online", [False, True])
@pytest.mark.parametrize("dtype", [None, "bf16"])
def test_online_softmax_switch_precomputed(torch_dev, online, dtype):
    s, w, y, t = inputs("precomputed", seed=330)
    if dtype == "bf16":
        s, w = bf16_round(s), bf16_round(w)
    opts = opts_for("precomputed", KernelConfig(online_softmax=online))
    got = H.distillation_loss(gpu(torch_dev, s, dtype), gpu(torch_dev, w, dtype),
                              gpu(torch_dev, y), on_gpu(torch_dev, t), opts)
    ref = O.distillation_loss(s, w, y, t, opts)
    check_output(got, ref, kind="bf16" if dtype else "f32")


def test_profile_switches_keep_int8_exact(torch_dev):
    """Under Fast and Debug the INT8 step still quantizes the call's own
    final fp32 grad_W exactly (codes, scales, dequantized rows)."""
    from parity import check_quant_of_own_gradient
    s, w, y, t = inputs("tied", seed=340)
    for prof, dtype in ((Profile.Fast, None), (Profile.Debug, "bf16")):
        cfg = KernelConfig.from_profile(prof)
        opts = opts_for("tied", dataclasses.replace(cfg, quantize_grad_weight=True))
        args = (gpu(torch_dev, s, dtype), gpu(torch_dev, w, dtype), gpu(torch_dev, y),
                on_gpu(torch_dev, t, dtype))
        got = H.distillation_loss(*args, opts, quant_codes=True)
        plain = H.distillation_loss(*args, opts_for("tied", cfg))
        check_quant_of_own_gradient(got, plain.grad_weight, y)
