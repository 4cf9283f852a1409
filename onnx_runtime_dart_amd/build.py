"""Builds libmmnb.so (HIP for gfx950) in-tree with hipcc.

    python -m onnx_runtime_dart_amd.build

Each translation unit is compiled to an object file in parallel (no device
code crosses translation units, so no relocatable device code is needed),
then the objects are linked into the shared library.

Packed FP32 instructions are disabled for all device code
(-target-feature -packed-fp32-ops); the host pass warns that it does not
know the feature, which is harmless.

Host-only sources (the ONNX reader and MatMulNBits host preparation, which
the CPU fuzz harness also builds under AddressSanitizer) are compiled with
the host C++ compiler.
"""
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libmmnb.so"
SOURCES = ["mmnb_runtime.hip", "mmnb_nbits.hip", "mmnb_int8.hip", "mmnb_decoder.hip",
           "mmnb_qlinear.hip", "mmnb_nbits_ex.hip", "mmnb_model.hip", "mmnb_noalloc.hip",
           "mmnb_nbits_any.hip"]
HOST_SOURCES = ["mmnb_host.cpp"]
ARCH = "gfx950"
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         # MFMA results in VGPRs, so epilogue FMAs need no v_accvgpr_read
         "-mllvm", "-amdgpu-mfma-vgpr-form"]


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libmmnb)")


def host_cxx():
    for cand in (os.environ.get("CXX"), shutil.which("g++"), shutil.which("c++")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("no host C++ compiler (g++) found")


HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra"]


def _filtered(r):
    return "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                     if "packed-fp32-ops" not in l and l.strip())


def build(verbose=False, jobs=None):
    cc = hipcc()
    OBJ.mkdir(exist_ok=True)
    sources = [s for s in SOURCES if (CSRC / s).exists()]

    host_sources = [s for s in HOST_SOURCES if (CSRC / s).exists()]
    cxx = host_cxx() if host_sources else None

    def compile_one(src):
        obj = OBJ / (Path(src).stem + ".o")
        if src in host_sources:
            cmd = [cxx, "-c"] + HOST_FLAGS + ["-o", str(obj), str(CSRC / src)]
        else:
            cmd = [cc, f"--offload-arch={ARCH}", "-c"] + FLAGS + ["-o", str(obj),
                                                                  str(CSRC / src)]
        return src, obj, cmd, subprocess.run(cmd, capture_output=True, text=True)

    units = sources + host_sources
    jobs = jobs or min(len(units), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(compile_one, units))
    for src, _, cmd, r in results:
        if verbose:
            print(" ".join(cmd), flush=True)
        msgs = _filtered(r)
        if r.returncode != 0:
            raise RuntimeError(f"compiler failed on {src} ({r.returncode}):\n{msgs}")
        if verbose and msgs:
            print(msgs)
    out_tmp = LIB.with_suffix(".so.tmp")
    link = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(out_tmp)] + \
        [str(o) for _, o, _, _ in results]
    if verbose:
        print(" ".join(link), flush=True)
    r = subprocess.run(link, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed ({r.returncode}):\n{_filtered(r)}")
    os.replace(out_tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
    print(LIB)
