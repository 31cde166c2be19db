"""Builds libcohere_hip.so (the C-ABI library of include/cohere_hip.h) for gfx950 with hipcc, in-tree.

    python cohere-inference_amd/csrc/build.py          # -> cohere-inference_amd/lib/libcohere_hip.so

Flags: -O3; -ffp-contract=off so every fp32 multiply/add the kernels write stays one rounding (the epilogues call
fmaf explicitly where the reference fuses); packed-fp32 instructions disabled; no fast-math.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

CSRC = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(CSRC)
ROOT = os.path.dirname(PKG)
INCLUDE = os.path.join(ROOT, "include")
OUT_DIR = os.path.join(PKG, "lib")
LIB = os.path.join(OUT_DIR, "libcohere_hip.so")
OBJ_DIR = os.path.join(ROOT, "_build")

SOURCES = ["capi.cpp", "gemm_q8.hip", "gemm_q8_dense.hip", "gemm_q8_sparse.hip", "dec_w8.hip", "quant.hip",
           "encoder_ops.hip", "encoder_loop.cpp", "encoder_noalloc.hip", "decoder_ops.hip", "gemm_bf16.hip", "frontend.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
COMMON = ["-O3", "-fPIC", "-std=c++17", "-ffp-contract=off", "-fno-fast-math", f"-I{INCLUDE}", f"-I{CSRC}",
          "-Wall", "-Wno-unused-result"]
# -amdgpu-mfma-vgpr-form: matrix-instruction accumulators in ordinary VGPRs (gfx950 allows either file), so that
# the VALU work on them (the grouped GEMM's per-group fold, the attention's softmax rescale) needs no
# v_accvgpr_read/write copies
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-mllvm", "-amdgpu-mfma-vgpr-form=1", "-x", "hip"]


def _compile(src: str, obj_dir: str = OBJ_DIR, defines=()) -> str:
    obj = os.path.join(obj_dir, src + ".o")
    cmd = [HIPCC, *COMMON, *[f"-D{d}" for d in defines], *DEVICE, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    if err.strip() and os.environ.get("COHERE_BUILD_VERBOSE"):
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = False, out: str = LIB, defines=()) -> str:
    """Compiles every source and links `out`; defines (NAME=VALUE strings) select build options."""
    obj_dir = OBJ_DIR if not defines else os.path.join(OBJ_DIR, "_".join(defines).replace("=", ""))
    os.makedirs(obj_dir, exist_ok=True)
    os.makedirs(os.path.dirname(out), exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(lambda src: _compile(src, obj_dir, defines), SOURCES))
    tmp = out + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, out)
    if verbose:
        print("built", out)
    return out


if __name__ == "__main__":
    # python build.py [OUT DEFINE=VALUE ...]
    if len(sys.argv) > 1:
        build(verbose=True, out=os.path.abspath(sys.argv[1]), defines=tuple(sys.argv[2:]))
    else:
        build(verbose=True)
