"""CPU-side checks of the C ABI library (no GPU needed): it loads, exports
every entry point include/orda/orda.h declares, and its host logic (chunk
resolver, doubling schedule, option defaults, config validation) agrees with
the oracle and the reference's known answers."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import oracle as O
import orda_hip as H
from orda_hip import _lib as L
from orda_hip.types import ChunkSize

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "orda", "orda.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(orda_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = L.load()
    names = declared_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), f"{n} declared in orda.h but not exported"
    # and the ctypes signature table covers the same set
    assert sorted(n for n, _, _ in L.SIGNATURES) == names


def test_abi_version_and_availability_without_gpu():
    lib = L.load()
    assert lib.orda_abi_version() == 2
    avail = H.is_available()
    assert avail in (True, False)


def test_struct_layouts_match_header_sizes():
    # orda_tensor: ptr + 3*i64 + 2*i32 = 40 bytes
    assert C.sizeof(L.Tensor) == 40
    assert C.sizeof(L.TeacherC) == 8 + 3 * 40


@pytest.mark.parametrize("bt", [1, 2, 7, 100, 511, 512, 513, 1000, 2048, 4096, 8192, 10000])
@pytest.mark.parametrize("v", [None, 1, 7, 8192, 32000, 65536, 131072, 262144])
@pytest.mark.parametrize("mc", [None, 1, 3, 16])
def test_resolver_matches_oracle(bt, v, mc):
    for cs in (ChunkSize.Auto, ChunkSize.Fixed(1), ChunkSize.Fixed(256), ChunkSize.Fixed(bt + 5)):
        a = H.resolve_chunk_size(bt, cs, v, mc)
        b = O.resolve_chunk_size(bt, cs, v, mc)
        assert (a.chunk_size, a.num_chunks) == (b.chunk_size, b.num_chunks)


def test_resolver_known_answers_via_abi():
    assert H.resolve_chunk_size(8192, ChunkSize.Auto, 131072, None) == H.ChunkPlan(512, 16)
    assert H.resolve_chunk_size(1000, ChunkSize.Fixed(256), None, None) == H.ChunkPlan(256, 4)
    assert H.resolve_chunk_size(100, ChunkSize.Fixed(4096), None, None) == H.ChunkPlan(100, 1)
    assert H.resolve_chunk_size(8192, ChunkSize.Auto, None, None) == H.ChunkPlan(8192, 1)
    for raw, n in [(0.0, 1), (1.49, 1), (1.5, 2), (3.0, 4), (6.0, 8), (1e300, 1 << 60)]:
        assert H.chunks_from_raw(raw) == n == O.chunks_from_raw(raw)
    assert H.chunk_doubling_schedule(10_000, 4, 32) == [4, 8, 16, 32]
    assert H.chunk_doubling_schedule(20, 4, 1000) == [4, 8, 16, 20]
    for bt, st, lim in [(1, 1, 1), (9, 0, 3), (100, 7, 0), (4096, 3, 4096), (37, 40, 64)]:
        assert H.chunk_doubling_schedule(bt, st, lim) == O.chunk_doubling_schedule(bt, st, lim)
        assert H.default_max_chunks_limit(bt) == O.default_max_chunks_limit(bt)


def test_option_defaults_match_reference():
    """LossOptions::default (api.rs:49-64) and KernelConfig (config.rs:68-90)."""
    c = L.LossOptionsC()
    L.load().orda_loss_options_default(C.byref(c))
    assert c.student_ce_weight == 1.0 and c.has_teacher_ce_weight == 0
    assert c.kd_weight == 0.0 and c.temperature == 1.0 and c.ignore_index == -100
    assert c.label_smoothing == 0.0 and c.reduction == 0 and c.chunk_fixed == 0
    assert c.backend == 0 and c.config.max_fused_size == 32768
    assert not c.config.fast_math and not c.config.quantize_grad_weight
    assert c.config.profile == 0
    k = L.KernelConfigC()
    L.load().orda_kernel_config_from_profile(1, C.byref(k))
    assert k.fast_math == 1 and k.profile == 1
    L.load().orda_kernel_config_from_profile(2, C.byref(k))
    assert k.fast_math == 0 and k.profile == 2
    # the Python mirror records the preset the same way
    assert H.KernelConfig.from_profile(H.Profile.Debug).profile == H.Profile.Debug
    assert H.KernelConfig().profile == H.Profile.Balanced
    assert L.load().orda_abi_version() == 2


def test_config_validate_messages():
    k = L.KernelConfigC()
    L.load().orda_kernel_config_from_profile(0, C.byref(k))
    err = C.create_string_buffer(256)
    assert L.load().orda_kernel_config_validate(C.byref(k), err, 256) == 0
    k.max_fused_size = 100
    assert L.load().orda_kernel_config_validate(C.byref(k), err, 256) == 1
    assert err.value.decode() == "max_fused_size must be a power of two >= 1, got 100"
    k.max_fused_size = 1024
    k.has_max_chunks, k.max_chunks = 1, 0
    assert L.load().orda_kernel_config_validate(C.byref(k), err, 256) == 1
    assert err.value.decode() == "max_chunks must be >= 1, got 0"
    k.has_max_chunks, k.profile = 0, 7
    assert L.load().orda_kernel_config_validate(C.byref(k), err, 256) == 1
    assert err.value.decode() == "unknown profile 7"


def test_no_gpu_fails_loudly_not_silently():
    """Without a device the loss must raise, never fall back to a CPU path."""
    if H.is_available():
        pytest.skip("a GPU is visible")
    s = np.zeros((4, 8), np.float32)
    w = np.zeros((16, 8), np.float32)
    with pytest.raises(H.OrdaError):
        H.distillation_loss(s, w, np.zeros(4, np.int64), H.Teacher.Tied(s), H.LossOptions())


STRUCTS = {
    "orda_tensor": L.Tensor,
    "orda_teacher": L.TeacherC,
    "orda_kernel_config": L.KernelConfigC,
    "orda_loss_options": L.LossOptionsC,
    "orda_loss_output": L.LossOutputC,
}


def test_header_is_c_and_matches_the_python_layouts(tmp_path):
    """include/orda/orda.h compiles as strict C11, a C caller links against
    liborda_hip.so and gets the reference's defaults and chunk plan
    (src/api.rs:49-64, src/resolver.rs:173-181), and every struct's size
    and field offsets, as the C compiler lays them out, are those of the
    ctypes mirror the Python binding passes."""
    import shutil
    import subprocess
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    if os.environ.get("ORDA_HIP_LIB"):
        pytest.skip("another build of the library (the sanitizer build links its runtimes)")
    lines = []
    for name, py in STRUCTS.items():
        lines.append(f'  printf("{name} size %zu\\n", sizeof({name}));')
        for field, _ in py._fields_:
            lines.append(f'  printf("{name} {field} %zu\\n", offsetof({name}, {field}));')
    src = "\n".join([
        "#include <stddef.h>",
        "#include <stdio.h>",
        '#include "orda/orda.h"',
        "int main(void) {",
        *lines,
        "  orda_loss_options o;",
        "  orda_loss_options_default(&o);",
        '  printf("defaults %g %g %g %lld %d %lld\\n", (double)o.student_ce_weight,',
        "         (double)o.kd_weight, (double)o.temperature, (long long)o.ignore_index,",
        "         o.reduction, (long long)o.config.max_fused_size);",
        "  int64_t cs = 0, nc = 0;",
        "  int32_t rc = orda_resolve_chunk_size(8192, 0, 0, 1, 131072, 0, 0, &cs, &nc);",
        '  printf("plan %d %lld %lld\\n", rc, (long long)cs, (long long)nc);',
        '  printf("abi %d\\n", orda_abi_version());',
        "  return 0;",
        "}",
    ])
    prog = tmp_path / "abi.c"
    prog.write_text(src + "\n")
    exe = tmp_path / "abi"
    libdir = os.path.dirname(L.LIB_PATH)
    subprocess.run([cc, "-std=c11", "-Wall", "-Wextra", "-Werror", "-pedantic",
                    "-I", os.path.join(ROOT, "include"), str(prog), "-o", str(exe),
                    "-L", libdir, "-l:" + os.path.basename(L.LIB_PATH),
                    "-Wl,-rpath," + libdir], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    got = {}
    for line in out.splitlines():
        parts = line.split()
        got[tuple(parts[:-1])] = parts[-1]
    for name, py in STRUCTS.items():
        assert int(got[(name, "size")]) == C.sizeof(py), name
        for field, _ in py._fields_:
            assert int(got[(name, field)]) == getattr(py, field).offset, f"{name}.{field}"
    d = next(l.split()[1:] for l in out.splitlines() if l.startswith("defaults"))
    ref = H.LossOptions()
    assert (float(d[0]), float(d[1]), float(d[2]), int(d[3])) == \
        (ref.student_ce_weight, ref.kd_weight, ref.temperature, ref.ignore_index)
    assert d[4] == "0"   # ORDA_REDUCTION_MEAN
    assert int(d[5]) == 65536 // 2
    assert got[("plan", "0", "512")] == "16"
    assert got[("abi",)] == str(L.load().orda_abi_version())
