"""The C ABI as a C compiler sees it: tests/c_abi/abi_check.c is compiled by
gcc (C99, all warnings as errors) against include/frx_ternary.h, linked with
libfrx_ternary.so and run. It pins the declared signatures against the
library and exercises the host-side packers and error statuses (no GPU)."""
import os
import shutil
import subprocess

import pytest

import ferrisres_amd as frx

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_header_compiles_and_host_entry_points_behave(tmp_path):
    exe = tmp_path / "abi_check"
    libdir = os.path.dirname(frx.LIB_PATH)
    cmd = ["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic",
           "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "c_abi", "abi_check.c"),
           "-L", libdir, "-lfrx_ternary", f"-Wl,-rpath,{libdir}", "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "abi_check ok" in r.stdout


ASAN_BIN = os.path.join(ROOT, "tests", "c_abi", "_asan", "asan_check")


def _asan_binary():
    """Builds tests/c_abi/_asan/asan_check (make, against the built
    libfrx_ternary.so) and returns its path."""
    r = subprocess.run(["make", "-C", os.path.join(ROOT, "tests", "c_abi"), "-s"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    return ASAN_BIN


ASAN_ENV = {"ASAN_OPTIONS": "detect_leaks=0:abort_on_error=0:halt_on_error=1",
            "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1"}


@pytest.mark.skipif(not os.path.exists("/opt/rocm/llvm/bin/clang"), reason="needs the ROCm clang")
def test_host_code_under_address_sanitizer():
    """frx_pack.cpp, frx_api.cpp and the oracle built with ASan + UBSan: the
    host packers against the oracle with exact-size buffers, every host
    argument check and every null-context entry point (no GPU needed)."""
    r = subprocess.run([_asan_binary()], capture_output=True, text=True, timeout=300,
                       env={**os.environ, **ASAN_ENV})
    assert r.returncode == 0, r.stdout + r.stderr
    assert "asan_check ok" in r.stdout


@pytest.mark.gpu
def test_api_validation_under_address_sanitizer_on_device():
    """The same instrumented build (made by __graft_entry__.build()) on a
    real context: the argument checks of every compute entry point and
    frx_force_status, all rejected before any kernel launch."""
    assert os.path.exists(ASAN_BIN), "build tests/c_abi/_asan/asan_check first (__graft_entry__.build())"
    r = subprocess.run([ASAN_BIN, "--device"], capture_output=True, text=True, timeout=120,
                       env={**os.environ, **ASAN_ENV})
    assert r.returncode == 0, r.stdout + r.stderr
    assert "asan_check ok (device validation)" in r.stdout


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_workspace_growth_policy(tmp_path):
    """The context workspaces grow by at least 1.5x (frx_policy.hpp): rising
    sizes (prefill M = 17..2048 at I = 11008 among them) make O(log)
    allocations and retire less than twice the final size."""
    exe = tmp_path / "policy_check"
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", "-Werror", "-I",
           os.path.join(ROOT, "ferrisres_amd", "csrc"), os.path.join(ROOT, "tests", "c_abi", "policy_check.cpp"),
           "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "policy_check ok" in r.stdout
