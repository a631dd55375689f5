"""AddressSanitizer and UndefinedBehaviorSanitizer runs on the CPU (no GPU
needed), each in a child process with the sanitizer runtime preloaded:

* the host side of liborda_hip.so (C ABI, orchestration, chunk resolver),
  built by `make -C orda-cutile-rs_amd asan` with clang's ASan + UBSan (host
  code only; the kernel objects are the normal build's), under the CPU ABI
  tests: exports, struct layouts, the resolver and doubling schedule against
  the oracle and the reference's known answers, option defaults, config
  validation messages, and the loud failure without a GPU;
* the oracle, built by `make -C oracle asan` with gcc's ASan, under its own
  known-answer, end-to-end and golden-vector tests.

A report from either sanitizer fails the test (UBSan halts on its first
error). The sanitizer builds come from __graft_entry__.build(); the test
skips when they or the runtimes are absent.
"""
import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "orda-cutile-rs_amd")
HOST_LIB = os.path.join(PKG, "_build", "asan", "liborda_hip.so")
ORACLE_LIB = os.path.join(ROOT, "oracle", "_asan", "liborda_oracle.so")


def _child(env_extra, args):
    env = dict(os.environ)
    env.update(env_extra)
    env["ASAN_OPTIONS"] = "detect_leaks=0"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    r = subprocess.run([sys.executable, *args], cwd=ROOT, env=env, capture_output=True,
                       text=True, timeout=900)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    assert "AddressSanitizer" not in out and "runtime error" not in out, out[-4000:]
    return out


def test_host_library_under_asan_and_ubsan():
    rt = sorted(glob.glob("/opt/rocm/lib/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not rt or not os.path.exists(HOST_LIB):
        pytest.skip("host sanitizer build or clang's ASan runtime absent")
    env = {"ORDA_HIP_LIB": HOST_LIB, "LD_PRELOAD": rt[-1]}
    # the sanitized build is the one that loads
    out = _child(env, ["-c", "import sys; sys.path.insert(0, 'orda-cutile-rs_amd'); "
                             "import orda_hip._lib as L; L.load(); print(L.LIB_PATH)"])
    assert out.strip().splitlines()[-1] == HOST_LIB, out
    out = _child(env, ["-m", "pytest", "tests/test_abi_cpu.py", "-q", "-m", "not gpu",
                       "-p", "no:cacheprovider"])
    assert " passed" in out, out[-2000:]


def test_oracle_under_asan():
    rt = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True,
                        text=True).stdout.strip()
    if not os.path.isabs(rt) or not os.path.exists(ORACLE_LIB):
        pytest.skip("oracle sanitizer build or gcc's ASan runtime absent")
    out = _child({"ORDA_ORACLE_LIB": ORACLE_LIB, "LD_PRELOAD": rt},
                 ["-m", "pytest", "tests/test_oracle_known_answers.py",
                  "tests/test_oracle_end_to_end.py", "tests/test_golden.py", "-q",
                  "-m", "not gpu", "-p", "no:cacheprovider"])
    assert " passed" in out, out[-2000:]
