"""Build ``libtkv_hip.so`` (the gfx950 kernels + C ABI) in-tree with hipcc.

    python -m tritonkv_amd.build          # or: __graft_entry__.build()

Each ``.hip`` source is compiled to an object in parallel (the quantized split
kernel's instantiations are spread over one file per K/V bit-width pair and
head-column width), then
linked into ``tritonkv_amd/libtkv_hip.so``.  Flags:

* ``--offload-arch=gfx950`` only -- no other targets, no host fallback;
* ``-O3`` without fast-math: the quantizer needs IEEE binary32 division and
  ``rintf`` for bit-exact parity with the reference;
* ``-Xclang -target-feature -Xclang -packed-fp32-ops`` keeps the compiler from
  emitting packed-fp32 VALU instructions;
* ``-mllvm -amdgpu-mfma-vgpr-form`` keeps MFMA accumulators in the unified
  VGPR file: without it the decode loop shuttled every accumulator through
  AGPRs around each MFMA (~100 extra moves per 32-token chunk) and serialised
  the per-group score MFMAs through one AGPR quad;
* ``-mllvm -amdgpu-kernarg-preload-count=16`` has the command processor load
  up to 16 leading argument dwords into SGPRs before a wave starts (the
  kernels taking scalar arguments: combine, quantize, window kernels; a struct
  passed by value is not preloaded).  The combine then starts without waiting
  on its argument loads: 0.1-0.2 us per cold Qwen-shape decode step with
  splits.  The kernel keeps a prologue that loads them itself where the
  firmware does not preload.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libtkv_hip.so")
SOURCES = ["decode_attention.hip", "quant_pack.hip", "runtime.hip"] + [
    f"quant_split_{bits}{hc}.hip" for bits in ("k4v4", "k2v2", "k4v2", "k2v4") for hc in ("", "_h4", "_h8")]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-mllvm", "-amdgpu-mfma-vgpr-form",
        "-mllvm", "-amdgpu-kernarg-preload-count=16",
        "-I", os.path.join(ROOT, "include"),
        "-Wno-unused-result",
    ]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *_flags(), "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr[-6000:]}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile every HIP source for gfx950 and link the shared library."""
    os.makedirs(OBJ, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-6000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
