"""Build the gfx950 kernel library and the C++17 host library in-tree.

  levo2.cpp_amd/liblevo_hip.so       C ABI (include/levo_hip.h) + HIP kernels
  levo2.cpp_amd/liblevo_hip_host.so  C++17 drop-in wrappers (levo2.cpp_amd/host/)
  levo2.cpp_amd/liblevo_bench_stream.so  plain streaming kernels bench.py compares the ops with
  levo2.cpp_amd/bench/host_dropins       bench.py's timing of the host-vector C++ drop-ins

Kernels are compiled with hipcc for gfx950 only; the host wrappers contain no
device code and are plain C++17 (g++) against the HIP runtime API. Every source is recompiled on
each call (the build is the "does it compile" check); objects are built in
parallel into levo2.cpp_amd/_build/.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
INCLUDE = os.path.join(ROOT, "include")
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(PKG, "host")
BUILD = os.path.join(PKG, "_build")
KERNEL_LIB = os.path.join(PKG, "liblevo_hip.so")
HOST_LIB = os.path.join(PKG, "liblevo_hip_host.so")
BENCH_LIB = os.path.join(PKG, "liblevo_bench_stream.so")  # measurement kernels of bench.py, not the C ABI
BENCH_HOST = os.path.join(PKG, "bench", "host_dropins")    # bench.py's host drop-in timings

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

# -ffp-contract=off: a*b+c rounds twice, as in the reference's ISO C++17 x86-64
# build; FMAs are written explicitly where the algorithm wants one.
# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 generation.
# -fma-mix-insts: no v_fma_mix{lo,hi}_f16, which would fold f16(a*b) into one
# mixed-precision FMA whose F16-subnormal results differ from the
# round-to-F32-then-F16 chain the reference computes.
COMMON = [
    "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Wall", "-Wextra", "-Wno-unused-parameter",
    "-I", INCLUDE, "-I", CSRC,
]
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-Xclang", "-target-feature", "-Xclang", "-fma-mix-insts"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        line for line in (r.stdout + r.stderr).splitlines()
        if "unknown target feature" not in line and "packed-fp32-ops" not in line
        and "fma-mix-insts" not in line
        and "argument unused during compilation: '--hip-link'" not in line
    )
    if r.returncode != 0:
        sys.stderr.write(out + "\n")
        raise RuntimeError("command failed: " + " ".join(cmd))
    if out.strip():
        sys.stderr.write(out + "\n")


def _compile(src: str, extra: list[str]) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    _run([HIPCC, *COMMON, *DEVICE, *extra, "-x", "hip", "-c", src, "-o", obj])
    return obj


HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__",
              "-I", os.path.join(ROCM, "include"), "-I", INCLUDE, "-I", HOST]


def _compile_host(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    _run([CXX, *HOST_FLAGS, "-c", src, "-o", obj])
    return obj


def build(verbose: bool = False) -> None:
    os.makedirs(BUILD, exist_ok=True)
    kernel_srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    host_srcs = sorted(glob.glob(os.path.join(HOST, "*.cpp")))
    bench_srcs = sorted(glob.glob(os.path.join(PKG, "bench", "*.hip")))
    jobs = min(8, os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(jobs) as ex:
        bobjs_f = [ex.submit(_compile, s, []) for s in bench_srcs]
        kobjs = list(ex.map(lambda s: _compile(s, []), kernel_srcs))
        hobjs = list(ex.map(_compile_host, host_srcs))
        bobjs = [f.result() for f in bobjs_f]
    _run([HIPCC, *DEVICE, "-shared", "-fPIC", "-o", KERNEL_LIB + ".tmp", *kobjs])
    os.replace(KERNEL_LIB + ".tmp", KERNEL_LIB)
    if hobjs:
        _run([CXX, "-shared", "-fPIC", "-o", HOST_LIB + ".tmp", *hobjs,
              "-L", PKG, "-llevo_hip", "-L", os.path.join(ROCM, "lib"), "-lamdhip64", "-Wl,-rpath,$ORIGIN"])
        os.replace(HOST_LIB + ".tmp", HOST_LIB)
    if bobjs:
        _run([HIPCC, *DEVICE, "-shared", "-fPIC", "-o", BENCH_LIB + ".tmp", *bobjs])
        os.replace(BENCH_LIB + ".tmp", BENCH_LIB)
    host_bench = os.path.join(PKG, "bench", "host_dropins.cpp")
    if hobjs and os.path.exists(host_bench):
        _run([CXX, *HOST_FLAGS, "-o", BENCH_HOST + ".tmp", host_bench, "-L", PKG, "-llevo_hip_host", "-llevo_hip",
              "-L", os.path.join(ROCM, "lib"), "-lamdhip64", "-Wl,-rpath,$ORIGIN/.."])
        os.replace(BENCH_HOST + ".tmp", BENCH_HOST)
    if verbose:
        print("built", KERNEL_LIB, HOST_LIB if hobjs else "")


if __name__ == "__main__":
    build(verbose=True)
