"""Builds the native libraries of the package in-tree (no CMake, no JIT cache).

libgemvq_hip.so    the gfx950 kernels, the command processor, the C ABI of include/gemvq_hip.h and the GGUF reader
                   of include/gemvq_gguf.h (hipcc)
libgemvq_synth.so  the host-only synthetic data generator of include/gemvq_synth.h (g++)
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(PKG, "_build")

HIP_LIB = os.path.join(PKG, "libgemvq_hip.so")
SYNTH_LIB = os.path.join(PKG, "libgemvq_synth.so")

HIP_SOURCES = ["gq_gemv.hip", "gq_gemv_q4_0.hip", "gq_gemv_q4_1.hip", "gq_gemv_q8_0.hip", "gq_gemv_kq.hip",
               "gq_gemv_tok_q4_0.hip", "gq_gemv_tok_q8_0.hip", "gq_gemv_tok_kq.hip", "gq_gemm.hip", "gq_ops.hip", "gq_gdn_out.hip", "gq_ref.hip", "gq_ref_gemv.hip",
               "gq_runtime.hip", "gq_static.hip", "qwen35.cpp", "gguf.cpp", "gq_ggml.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# -ffp-contract=off: no multiply-add is fused unless written as fmaf (results are reproduced bit for bit on the CPU);
# packed FP32 instructions are disabled (they are avoided on this hardware).
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math",
             "-Wno-unused-value", "-Wno-unused-result",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             # leading scalar kernel arguments arrive in SGPRs (kernel argument preloading, gfx940 and later; the
             # code object keeps a prologue that loads them where the firmware does not)
             "-mllvm", "-amdgpu-kernarg-preload-count=16",
             "-I" + INCLUDE, "-I" + CSRC]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(line for line in r.stderr.splitlines() if noise not in line)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{err}\n{r.stdout}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build_hip() -> str:
    os.makedirs(BUILD, exist_ok=True)
    objs = [os.path.join(BUILD, s.rsplit(".", 1)[0] + ".o") for s in HIP_SOURCES]
    with ThreadPoolExecutor(max_workers=len(HIP_SOURCES)) as ex:
        list(ex.map(lambda so: _run([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, so[0]), "-o", so[1]]),
                    zip(HIP_SOURCES, objs)))
    tmp = HIP_LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,-soname,libgemvq_hip.so", *objs, "-o", tmp])
    os.replace(tmp, HIP_LIB)
    return HIP_LIB


def build_synth() -> str:
    tmp = SYNTH_LIB + ".tmp"
    _run(["g++", "-O3", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-pthread",
          "-I" + INCLUDE, os.path.join(CSRC, "synth.cpp"), "-o", tmp])
    os.replace(tmp, SYNTH_LIB)
    return SYNTH_LIB


def build() -> None:
    with ThreadPoolExecutor(max_workers=2) as ex:
        f1 = ex.submit(build_hip)
        f2 = ex.submit(build_synth)
        f1.result()
        f2.result()


if __name__ == "__main__":
    build()
    print("built", HIP_LIB, SYNTH_LIB)
