"""Build libnq_hip.so (the gfx950 kernels + C ABI) in-tree with hipcc.

    python -m nanoinfer_amd.build          # compile every source, link the library

Objects go to nanoinfer_amd/_build/, the library to nanoinfer_amd/libnq_hip.so.
Every source is compiled on each call (this is the "does it build" check); the
compiles run in parallel processes.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libnq_hip.so")
HOST_LIB = os.path.join(PKG, "libnq_host.so")
HOST_TEST = os.path.join(ROOT, "tests", "cpp", "test_host.bin")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

SOURCES = ["nq_abi.cpp", "nq_quantize.hip", "nq_gemv.hip", "nq_w8a8.hip", "nq_embed.hip", "nq_fused.hip", "nq_wq_gemm.hip", "nq_nit.hip", "nq_rope.hip", "nq_dequant.hip", "nq_ops.hip"]
BENCH_SRC = os.path.join("bench", "nq_probe.hip")  # libnq_bench.so: bench.py's read probe
BENCH_LIB = os.path.join(PKG, "libnq_bench.so")

# -packed-fp32-ops: keep hipcc from forming v_pk_{add,mul,fma}_f32 (the host
# pass prints that it does not know the feature; that is harmless).
# -amdgpu-mfma-vgpr-form: MFMA accumulators in ordinary VGPRs; with AGPR
# accumulators the register allocator shuffled the tiles with v_accvgpr moves
# on every GEMM iteration.
HIP_FLAGS = [
    "-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-I", os.path.join(ROOT, "include"),
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [HIPCC, *HIP_FLAGS, *lang, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def _run(cmd, what):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{r.stderr}")


def _host_artifacts():
    """The C++ host layer, the nicpp pybind11 module and the C++ host test."""
    import sysconfig

    import pybind11

    host_src = os.path.join(CSRC, "host")
    rpath = "-Wl,-rpath,$ORIGIN"
    cxx = [HIPCC, "-std=c++17", "-O2", "-fPIC", "-Wall", "-I", os.path.join(ROOT, "include")]
    _run([*cxx, "-shared", "-o", HOST_LIB + ".tmp", os.path.join(host_src, "nq_host.cpp"),
          os.path.join(host_src, "nq_model.cpp"),
          "-L", PKG, "-lnq_hip", rpath], "libnq_host link")
    os.replace(HOST_LIB + ".tmp", HOST_LIB)
    ext = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    mod = os.path.join(PKG, "nicpp" + ext)
    _run([*cxx, "-shared", "-fvisibility=hidden", "-I", pybind11.get_include(),
          "-I", sysconfig.get_paths()["include"], "-o", mod + ".tmp", os.path.join(host_src, "nicpp.cpp"),
          "-L", PKG, "-lnq_host", "-lnq_hip", rpath], "nicpp module")
    os.replace(mod + ".tmp", mod)
    _run([*cxx, "-o", HOST_TEST + ".tmp", os.path.join(ROOT, "tests", "cpp", "test_host.cpp"),
          "-L", PKG, "-lnq_host", "-lnq_hip", "-Wl,-rpath," + PKG, "-Wl,-rpath,$ORIGIN/../../nanoinfer_amd"],
         "C++ host test")
    os.replace(HOST_TEST + ".tmp", HOST_TEST)
    return [HOST_LIB, mod, HOST_TEST]


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES) + 1)) as ex:
        objs = list(ex.map(_compile, SOURCES + [BENCH_SRC]))
    bench_obj = objs.pop()
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], "libnq_hip link")
    os.replace(tmp, LIB)
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", BENCH_LIB + ".tmp", bench_obj],
         "libnq_bench link")
    os.replace(BENCH_LIB + ".tmp", BENCH_LIB)
    extra = [BENCH_LIB, *_host_artifacts()]
    if verbose:
        for p in [LIB, *extra]:
            print("built", p)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
