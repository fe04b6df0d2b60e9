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
