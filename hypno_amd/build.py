"""Builds libhypno_hip.so (gfx950) in-tree with hipcc.

    python -m hypno_amd.build        # or hypno_amd.build.build()

Every HIP source is compiled for gfx950 only, with packed FP32 instructions
disabled (-packed-fp32-ops), then linked into one shared library next to this
file.  Object files go to hypno_amd/_build/.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ_DIR = os.path.join(HERE, "_build")
LIB_NAME = "libhypno_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)

SOURCES = ["codec.hip", "gemv_q4_0.hip", "gemv_f16.hip", "gemm.hip", "gemm_q4.hip", "gemm_exact.hip",
           "skinny_q4.hip", "prologue.hip", "gemv_col.hip", "gemm_q8_0.hip", "sample.hip", "api.cpp",
           "model.cpp"]

ARCH = "gfx950"
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    # Packed FP32 (v_pk_{add,mul,fma}_f32) stays off in all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: the fp32 epilogue math reads them directly
    # instead of copying each accumulator out of AGPRs first.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    f"-I{os.path.join(ROOT, 'include')}",
]

# Per-source additions.  The streaming GEMV's leading scalar arguments (the
# first job and the launch shape, 14 SGPRs) are preloaded into SGPRs, so a
# work-group starts its first reads without waiting on kernel-argument
# memory; the compiler keeps a prologue that loads them for firmware that
# does not preload.
FILE_FLAGS = {
    "gemv_q4_0.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=11"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build hypno_amd)")


def _quiet(text: str) -> str:
    # hipcc's host pass does not know the GPU feature flag; that note is noise.
    return "\n".join(l for l in text.splitlines()
                     if "packed-fp32-ops' is not a recognized feature" not in l)


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
    lang = ["-x", "hip"]
    cmd = ([hipcc()] + lang + COMMON_FLAGS + FILE_FLAGS.get(src, []) +
           ["-c", os.path.join(CSRC, src), "-o", obj])
    p = subprocess.run(cmd, capture_output=True, text=True)
    out = _quiet(p.stdout + p.stderr)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{out}")
    if out.strip():
        sys.stderr.write(out + "\n")
    return obj


def build(verbose: bool = False) -> str:
    """Compile every source for gfx950 and link LIB_PATH.  Always rebuilds."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("link failed:\n" + _quiet(p.stdout + p.stderr))
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
