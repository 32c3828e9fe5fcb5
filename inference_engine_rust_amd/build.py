"""Build recipe for the native libraries (in-tree, so they travel with the repository snapshot).

* ``libiek.so``        — the product: HIP kernels for gfx950 + the C++ host runtime + C ABI.
* ``libiek.a``         — the same objects as a static archive (link with ``-lamdhip64``).
* ``bin/iek_bench_compare`` — the bench_compare CLI over the C ABI (g++, static libiek.a).
* ``bin/iek_abi_test`` — C++ caller of the C ABI used by the GPU tests (g++, static libiek.a).
* ``libiek_synth.so``  — seeded synthetic GGUF writer / quantisers (host C++).

Objects go to ``inference_engine_rust_amd/_build``; each translation unit compiles in its own
process so the build parallelises across cores.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libiek.so")
LIB_A = os.path.join(PKG, "libiek.a")
BIN = os.path.join(PKG, "bin")
REPO = os.path.dirname(PKG)
ROCM_LIB = "/opt/rocm/lib"
SYNTH_LIB = os.path.join(PKG, "libiek_synth.so")
ARCH = os.environ.get("IEK_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
# Packed-FP32 VALU ops are disabled for all device code: some of their forms have given wrong
# results, without an error, on the MI355X machines this is tested on.
HIP_FLAGS = ["-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops", "-Wall", "-Wno-unused-function", "-Wno-unused-result"]

SOURCES = [
    "kernels/matvec.hip",
    "kernels/ops.hip",
    "kernels/attention.hip",
    "kernels/gemm.hip",
    "kernels/gemm_mfma.hip",
    "kernels/gemm_q.hip",
    "kernels/gemma.hip",
    "kernels/chain.hip",
    "kernels/noalloc.hip",
    "kernels/sampling.hip",
    "model.cpp",
    "session.cpp",
    "api.cpp",
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "unknown target feature" not in l and
                    "warning: feature flag" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        sys.stderr.write(out + "\n")


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, src.replace("/", "_").rsplit(".", 1)[0] + ".o")
    lang = ["-x", "hip"]
    _run([HIPCC, *lang, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def build_synth() -> str:
    _run(["g++", "-std=c++17", "-O2", "-march=x86-64-v3", "-fPIC", "-shared", "-pthread", "-Wall",
          "-Wno-unused-function", "-o", SYNTH_LIB, os.path.join(CSRC, "synth", "gguf_synth.cpp")])
    return SYNTH_LIB


def build_lib(jobs: int | None = None) -> str:
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    tmp_a = LIB_A + ".tmp"
    if os.path.exists(tmp_a):
        os.remove(tmp_a)
    _run(["ar", "rcs", tmp_a, *objs])
    os.replace(tmp_a, LIB_A)
    return LIB


def _link_tool(src: str, out: str) -> str:
    """A C++ caller of include/iek.h built with g++ against the static archive."""
    os.makedirs(BIN, exist_ok=True)
    tmp = out + ".tmp"
    _run(["g++", "-std=c++17", "-O2", "-Wall", "-I", os.path.join(REPO, "include"), src, LIB_A, "-L", ROCM_LIB,
          "-lamdhip64", f"-Wl,-rpath,{ROCM_LIB}", "-pthread", "-o", tmp])
    os.replace(tmp, out)
    return out


def _hip_tool(src: str, out: str) -> str:
    """A stand-alone HIP program (no library)."""
    os.makedirs(BIN, exist_ok=True)
    tmp = out + ".tmp"
    _run([HIPCC, *HIP_FLAGS, src, "-o", tmp])
    os.replace(tmp, out)
    return out


def build_tools() -> None:
    _link_tool(os.path.join(PKG, "cli", "bench_compare.cpp"), os.path.join(BIN, "iek_bench_compare"))
    _link_tool(os.path.join(REPO, "tests", "abi", "iek_abi_test.cpp"), os.path.join(BIN, "iek_abi_test"))
    _hip_tool(os.path.join(PKG, "cli", "calibrate.hip"), os.path.join(BIN, "iek_calibrate"))


def build_all() -> None:
    build_synth()
    build_lib()
    build_tools()


if __name__ == "__main__":
    build_all()
    print(LIB)
