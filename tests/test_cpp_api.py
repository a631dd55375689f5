"""The C++ mirror of the crate's API (include/orda/orda.hpp) without a GPU: the
header compiles warning-free (-Wall -Wextra -Werror -pedantic) into
tests/cpp/api_test.cpp, linked against the in-tree liborda_hip.so, and the
program's CPU checks pass: LossOptions and KernelConfig defaults and presets
(src/api.rs:49-64, src/config.rs:78-90), KernelConfig::validate's messages
(src/config.rs:106-119), the resolver over a grid of plans (bit-exact against
the oracle's restatement of src/resolver.rs), Mat and Teacher, and that a loss
call without a device fails as unavailable instead of running on the host."""
import json
import os
import shutil
import subprocess

import pytest

import oracle as O
from orda_hip.types import ChunkSize, KernelConfig, OrdaError

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBDIR = os.path.join(ROOT, "orda-cutile-rs_amd", "orda_hip")


@pytest.fixture(scope="module")
def cpu_run(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("no g++")
    if os.environ.get("ORDA_HIP_LIB"):
        pytest.skip("the program links the in-tree library, not ORDA_HIP_LIB")
    exe = tmp_path_factory.mktemp("cpp") / "api_test"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", "-Werror", "-pedantic",
                    "-ffp-contract=off", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "cpp", "api_test.cpp"), "-o", str(exe),
                    "-L", LIBDIR, "-l:liborda_hip.so", f"-Wl,-rpath,{LIBDIR}"],
                   check=True, capture_output=True, text=True)
    r = subprocess.run([str(exe), "cpu"], capture_output=True, text=True, timeout=120)
    out = json.loads(r.stdout)
    return r.returncode, out


def test_cpp_cpu_checks_pass(cpu_run):
    rc, out = cpu_run
    assert out["failures"] == [] and rc == 0


def test_cpp_validate_messages_match_the_reference(cpu_run):
    _, out = cpu_run
    for field, cfg in (("validate_max_fused_size", KernelConfig(max_fused_size=3)),
                       ("validate_max_chunks", KernelConfig(max_fused_size=1024, max_chunks=0))):
        with pytest.raises(OrdaError) as e:
            cfg.validate()
        assert out[field] == str(e.value)
    assert out["resolve_bt0"] == "BT (batch * sequence length) must be > 0"


def test_cpp_resolver_matches_the_oracle(cpu_run):
    _, out = cpu_run
    assert len(out["plans"]) == 56
    for bt, fixed, has_v, has_mc, cs, nc in out["plans"]:
        ref = O.resolve_chunk_size(bt, ChunkSize.Fixed(bt // 3 + 1) if fixed else ChunkSize.Auto,
                                   131072 if has_v else None, 8 if has_mc else None)
        assert (cs, nc) == (ref.chunk_size, ref.num_chunks), (bt, fixed, has_v, has_mc)
    assert out["schedule_8192"] == O.chunk_doubling_schedule(8192, 16, O.default_max_chunks_limit(8192))
    assert out["schedule_1000_3"] == O.chunk_doubling_schedule(1000, 3, 1000)
    assert out["default_max_chunks_limit"] == [O.default_max_chunks_limit(b) for b in (1, 8192, 100000)]
    assert out["chunks_from_raw"] == [O.chunks_from_raw(x) for x in (0.5, 1.5, 3.0, 100.0)]
    assert out["ceil_div"] == [O.ceil_div(10, 3), O.ceil_div(9, 3)]
    # resolver.rs known answer: the c5 plan
    assert [8192, 0, 1, 0, 512, 16] in out["plans"]
