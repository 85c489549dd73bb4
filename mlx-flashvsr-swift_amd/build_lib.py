"""Build recipe for libfvsr_lcsa.so (gfx950) and the C++ host probe.

Run as `python mlx-flashvsr-swift_amd/build_lib.py` or call `build()`. hipcc cross-compiles for gfx950 without a
GPU. Output goes in-tree (mlx-flashvsr-swift_amd/lib/) so it travels with the repository snapshot.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
HOST = os.path.join(PKG, "host")
LIB_DIR = os.path.join(PKG, "lib")
LIB = os.path.join(LIB_DIR, "libfvsr_lcsa.so")
PROBE = os.path.join(LIB_DIR, "fvsr_probe_attn")

SOURCES = ["api.hip", "lcsa_attn.hip", "lcsa_select.hip", "kv_ring.hip", "qkv_epilogue.hip", "dit_block.hip"]
# Packed-FP32 VALU forms are disabled: hipcc -O3 would otherwise emit v_pk_{add,mul,fma}_f32 from float code.
# MFMA builtins get the VGPR form (results in VGPRs, where the VALU reads them without v_accvgpr_read); every MFMA
# of the attention kernels, the output accumulation included, is a compiler builtin.
HIP_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang",
             "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libfvsr_lcsa)")


def _run(cmd, verbose: bool):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build failed ({res.returncode}):\n{out}")
    if verbose and out.strip():
        print(out)


def build(verbose: bool = False) -> str:
    """Compile every HIP source into lib/libfvsr_lcsa.so (always rebuilds) and the host probe; returns the .so path."""
    os.makedirs(LIB_DIR, exist_ok=True)
    hipcc = _hipcc()
    tmp = LIB + ".tmp"
    # hipBLASLt for the DiT block's GEMMs (fvsr_linear / fvsr_dit_block)
    _run([hipcc, *HIP_FLAGS, "-shared", *[os.path.join(CSRC, s) for s in SOURCES], "-o", tmp, "-lhipblaslt"], verbose)
    os.replace(tmp, LIB)
    probe_src = os.path.join(HOST, "probe_attn.cpp")
    if os.path.exists(probe_src):
        ptmp = PROBE + ".tmp"
        _run([hipcc, *HIP_FLAGS, "-x", "hip", f"-I{os.path.join(ROOT, 'include')}", f"-I{HOST}", probe_src,
              f"-L{LIB_DIR}", "-lfvsr_lcsa", f"-Wl,-rpath,$ORIGIN", "-o", ptmp], verbose)
        os.replace(ptmp, PROBE)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
