"""Builds libmmnb.so (HIP for gfx950) in-tree with hipcc.

    python -m onnx_runtime_dart_amd.build

Packed FP32 instructions are disabled for all device code
(-target-feature -packed-fp32-ops); the host pass warns that it does not
know the feature, which is harmless.
"""
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libmmnb.so"
SOURCES = ["mmnb_runtime.hip", "mmnb_nbits.hip", "mmnb_int8.hip", "mmnb_decoder.hip",
           "mmnb_qlinear.hip", "mmnb_nbits_ex.hip", "mmnb_model.hip"]
ARCH = "gfx950"


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libmmnb)")


def build(verbose=False):
    out_tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
           "-Wall", "-Wno-unused-function",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           # MFMA results in VGPRs, so epilogue FMAs need no v_accvgpr_read
           "-mllvm", "-amdgpu-mfma-vgpr-form",
           "-o", str(out_tmp)] + [str(CSRC / s) for s in SOURCES]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                     if "packed-fp32-ops" not in l and l.strip())
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{msgs}")
    if verbose and msgs:
        print(msgs)
    os.replace(out_tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
    print(LIB)
