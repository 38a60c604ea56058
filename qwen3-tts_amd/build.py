"""Build libqwen_tts_hip.so in-tree with hipcc for gfx950 (no JIT cache, no torch).

    python qwen3-tts_amd/build.py            # compiles every source, every time

Device code is compiled with packed-FP32 instructions disabled
(-Xclang -target-feature -Xclang -packed-fp32-ops); the host C file is compiled by
gcc against the HIP runtime headers.  Objects go to qwen3-tts_amd/_build/.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libqwen_tts_hip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = os.environ.get("QWEN_HIP_ARCH", "gfx950")

HIP_SOURCES = ["qt_matvec.hip", "qt_attn.hip", "qt_misc.hip", "qt_pstep.hip", "qt_rstep.hip", "qt_rstep06.hip", "qt_rstep06b.hip", "qt_rstep4.hip", "qt_batch.hip", "qt_prefill.hip", "qt_sample.hip", "qt_sd.hip",
               "qt_noalloc.hip"]
C_SOURCES = ["qwen_tts_hip.c", "qt_load.c", "qt_sd_host.c"]

HIPCC_FLAGS = ["-O3", "-fPIC", "-std=c++17", f"--offload-arch={ARCH}",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-ffp-contract=off",
               "-Wall", "-Wno-unused-function", "-I", CSRC, "-I", os.path.join(ROOT, "include")]
# -ffp-contract=off: every fused multiply-add in the kernels is an explicit fmaf, so two
# kernels that state the same arithmetic round identically (hipcc's default contracts
# a*b+c wherever instruction selection finds it, e.g. an RMSNorm product into the int8
# activation sum, and then the fused step and the per-kernel path disagree by an ulp).
# per-source additions: the q4_0 step's MFMA results feed VALU epilogues right away, and in
# the VGPR form of the instruction they need no copy out of the accumulation registers
# (measured on the phase trace: the q4_0 projections 2.44 -> 2.00 us per layer and role)
HIPCC_FILE_FLAGS = {"qt_rstep4.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}
CC_FLAGS = ["-O2", "-fPIC", "-std=gnu11", "-Wall", "-Wextra", "-Wno-unused-parameter",
            "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"), "-I", CSRC,
            "-I", os.path.join(ROOT, "include")]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r.stderr


def build(verbose=False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    jobs = []
    for s in HIP_SOURCES:
        jobs.append([hipcc, *HIPCC_FLAGS, *HIPCC_FILE_FLAGS.get(s, []), "-c", os.path.join(CSRC, s),
                     "-o", os.path.join(BUILD, s.replace(".hip", ".o"))])
    for s in C_SOURCES:
        jobs.append(["gcc", *CC_FLAGS, "-c", os.path.join(CSRC, s),
                     "-o", os.path.join(BUILD, s.replace(".c", ".o"))])
    with ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        logs = list(ex.map(_run, jobs))
    if verbose:
        for l in logs:
            if l.strip():
                print(l, file=sys.stderr)
    objs = [os.path.join(BUILD, s.replace(".hip", ".o")) for s in HIP_SOURCES] + \
           [os.path.join(BUILD, s.replace(".c", ".o")) for s in C_SOURCES]
    tmp = LIB + ".tmp"
    _run([hipcc, "-shared", f"--offload-arch={ARCH}", "-o", tmp, *objs,
          "-L", os.path.join(ROCM, "lib"), "-lamdhip64", "-Wl,-rpath," + os.path.join(ROCM, "lib")])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
