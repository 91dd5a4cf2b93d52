"""In-tree build of libloractl_rocm.so (the quantized LoRA linear) and
libloractl_mmdit.so (the MMDiT driver's attention-input kernels), hipcc,
gfx950 only.

The library is built next to this file so that it travels with the source
tree; nothing is installed into site-packages.
"""

from __future__ import annotations

import os
import subprocess
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
OBJ = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libloractl_rocm.so")
SOURCES = ["lrq_quant.hip", "lrq_gemm.hip", "lrq_gemm_mid.hip", "lrq_skinny.hip", "lrq_lora.hip", "lrq_api.hip", "lrq_probe.hip"]
MMDIT_LIB = os.path.join(HERE, "libloractl_mmdit.so")
MMDIT_SOURCES = ["mmdit_attn_prep.hip", "mmdit_modulate.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # hand-written kernels only use scalar/float2 code; keep the compiler
    # from forming packed-fp32 instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _compile(src: str) -> str:
    out = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, "-I", INCLUDE, "-c", os.path.join(CSRC, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return out


def _link(lib: str, objs) -> None:
    tmp = lib + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed for {os.path.basename(lib)}:\n{r.stderr}")
    os.replace(tmp, lib)


def build(verbose: bool = False) -> str:
    """Compile every HIP source for gfx950 and link both libraries."""
    os.makedirs(OBJ, exist_ok=True)
    srcs = SOURCES + MMDIT_SOURCES
    with ThreadPoolExecutor(max_workers=len(srcs)) as ex:
        objs = list(ex.map(_compile, srcs))
    _link(LIB, objs[:len(SOURCES)])
    _link(MMDIT_LIB, objs[len(SOURCES):])
    if verbose:
        print(f"built {LIB} and {MMDIT_LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
