"""Build libheatkv.so (gfx950) in-tree from the HIP sources in this directory.

Usage: ``python heatkv_amd/csrc/build.py`` or ``heatkv_amd.csrc.build.build()``.
Each source compiles to an object in ``_build/`` in parallel, then one link
writes ``heatkv_amd/libheatkv.so``.  Always recompiles (it is the build check).
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
SOURCES = ("abi.hip", "pack.hip", "produce.hip", "plan.hip", "seg_attn.hip", "seg_attn_split.hip",
           "seg_attn_staged.hip", "seg_attn_direct.hip")
ARCH = "gfx950"
LIB = os.path.join(PKG, "libheatkv.so")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed-fp32 VALU ops are not generated (this target has given wrong
    # results with some of their forms).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{os.path.join(ROOT, 'include')}",
]

# Per-source flags.  The 16-bit and split-row attention kernels take their
# work plan's pointer and unit count as their first two arguments, preloaded
# into SGPRs at wave launch, so the unit's load needs no kernel-argument load
# first.  The 16-bit kernel keeps the pre-register-allocation schedule (no
# post-RA machine scheduler): 0.3-1 % faster on every measured launch shape.
EXTRA = {
    "seg_attn_direct.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=2", "-mllvm", "-enable-post-misched=0"],
    "seg_attn_split.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=2"],
}


def _hipcc():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = os.path.join(rocm, "bin", "hipcc")
    return cand if os.path.exists(cand) else "hipcc"


def _run(cmd):
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so.
    err = "\n".join(l for l in proc.stderr.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    return err


def build(verbose: bool = False) -> str:
    out_dir = os.path.join(ROOT, "_build")
    os.makedirs(out_dir, exist_ok=True)
    hipcc = _hipcc()
    objs = []
    cmds = []
    for src in SOURCES:
        obj = os.path.join(out_dir, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([hipcc, *FLAGS, *EXTRA.get(src, []), "-c", os.path.join(HERE, src), "-o", obj])
    with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        for msg in ex.map(_run, cmds):
            if verbose and msg.strip():
                print(msg, file=sys.stderr)
    tmp = LIB + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
