"""The tick planner (csrc/plan.cpp, host C++) built with AddressSanitizer and
UndefinedBehaviorSanitizer by g++ and driven by tests/asan/plan_fuzz.cpp:
random decode / prefill / mixed ticks over GQA groups 1-16, page sizes
32-256, CU counts 0-304 and fixed decode split lengths, each planned with
roomy buffers, with buffers of exactly the reported counts (guard words
after each must stay untouched) and one record short of each (HY_ENOSPACE),
and every plan checked for coverage. Any out-of-bounds access, overflow or
undefined shift aborts the run with the sanitizer's report."""

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "hayate-exp_amd", "csrc")


@pytest.fixture(scope="module")
def fuzz_binary(tmp_path_factory):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ is not available")
    out = str(tmp_path_factory.mktemp("asan") / "plan_fuzz")
    cmd = [cxx, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           os.path.join(ROOT, "tests", "asan", "plan_fuzz.cpp"), os.path.join(CSRC, "plan.cpp"),
           "-o", out]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return out


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_planner_under_address_and_ub_sanitizers(fuzz_binary, seed):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    r = subprocess.run([fuzz_binary, str(seed), "150"], capture_output=True, text=True,
                       env=env, timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    assert r.stdout.strip() == "ok 150"
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr
