"""Builds liblsfa_gfx950.so (the HIP kernels plus the C ABI) in-tree.

    python -m lightserve_amd.csrc.build          # or: python lightserve_amd/csrc/build.py

Every source is compiled for gfx950 only, in parallel, with packed-fp32 VALU
instructions disabled, then linked into lightserve_amd/liblsfa_gfx950.so next
to the Python package that loads it; the linker's version script
(exports.map) exports the lsfa_* C ABI and nothing else.
"""
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
REPO = os.path.dirname(PKG)
OUT = os.path.join(PKG, "liblsfa_gfx950.so")
BUILD_DIR = os.path.join(HERE, "_build")
SOURCES = ["fa_fwd.hip", "fa_bwd.hip", "fa_f32.hip", "fa_decode.hip", "fa_rope.hip", "fa_norm.hip", "fa_gemv.hip", "fa_gemv_mfma.hip", "fa_sample.hip", "fa_api.hip"]
HEADERS = ["fa_common.hpp", os.path.join("..", "..", "include", "lightserve_fa.h")]

ARCH = "gfx950"
CXXFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 VALU ops are kept out of every code object
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-source additions. fa_bwd.hip: MFMA results in VGPRs. The dK/dV kernel
# runs one wave per SIMD, where the compiler would otherwise put every MFMA
# accumulator in AGPRs and copy S and dP back to VGPRs for the softmax (one
# v_accvgpr_read per element); with VGPR results only the long-lived dK/dV
# sums spill to AGPRs.
EXTRA_FLAGS = {"fa_bwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the gfx950 kernels need ROCm's hipcc to build")


def _compile(src):
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [_hipcc(), *CXXFLAGS, *EXTRA_FLAGS.get(src, []), "-c", os.path.join(HERE, src), "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"compiling {src} failed:\n{' '.join(cmd)}\n{err}")
    return obj, err


def build(verbose=False):
    os.makedirs(BUILD_DIR, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        results = list(ex.map(_compile, SOURCES))
    for _, err in results:
        if verbose and err.strip():
            print(err, file=sys.stderr)
    objs = [o for o, _ in results]
    tmp = OUT + ".tmp"
    # exports.map keeps the dynamic symbol table to the lsfa_* C ABI
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC",
           f"-Wl,--version-script={os.path.join(HERE, 'exports.map')}", *objs, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"linking failed:\n{' '.join(cmd)}\n{proc.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
