"""Build recipe for libfrx_ternary.so (gfx950) — used by __graft_entry__.build().

Compiles every HIP/C++ source under ferrisres_amd/csrc with hipcc into one
shared library next to this file. No torch types cross the ABI; the library
depends only on the HIP runtime. csrc/bench/ holds bench.py's measurement
helpers (a plain streaming read), linked separately into libfrx_bench.so.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libfrx_ternary.so")
BUILD = os.path.join(HERE, "_build")

SOURCES = ["frx_api.cpp", "frx_pack.cpp", "frx_gemv.hip", "frx_gemv_sk.hip", "frx_gemm.hip", "frx_moe.hip", "frx_ffn.hip", "frx_ingest.hip", "frx_variants.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
    # packed FP32 VALU forms (v_pk_{add,mul,fma}_f32) are disabled: some of their
    # forms have given wrong results on this hardware without any error
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, src + ".o")
    cmd = [HIPCC, *COMMON, "-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")
    return obj


BENCH_OUT = os.path.join(HERE, "libfrx_bench.so")
BENCH_SOURCES = ["bench/frx_bench_read.hip"]


def build(verbose: bool = False) -> str:
    os.makedirs(os.path.join(BUILD, "bench"), exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES) + len(BENCH_SOURCES), 6)) as ex:
        objs_all = list(ex.map(_compile, SOURCES + BENCH_SOURCES))
    objs, bench_objs = objs_all[:len(SOURCES)], objs_all[len(SOURCES):]
    # measurement helpers for bench.py (not part of the ternary path)
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", BENCH_OUT, *bench_objs],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"bench helper link failed:\n{r.stderr[-6000:]}")
    tmp = OUT + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}", file=sys.stderr)
    return OUT


if __name__ == "__main__":
    build(verbose=True)
