"""Checks on the generated gfx950 code (host-side compile, no GPU needed).

The direct-to-LDS attention kernel and the split-row kernel write M0 inside
their DMA inline assembly and declare it clobbered; that is only sound while
no compiler-generated instruction relies on M0.  This compiles the kernels
to assembly with the library build's own flags (heatkv_amd/csrc/build.py:
FLAGS plus the per-file EXTRA, e.g. the kernel-argument preload) and checks
that every M0 reference sits inside an inline-assembly block, that no kernel
spills registers to scratch, and that operand loads stay 16-byte vectors.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

from heatkv_amd.csrc import build as _build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "heatkv_amd", "csrc")


def _hipcc():
    cand = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")
    return cand if os.path.exists(cand) else shutil.which("hipcc")


def _asm(src, tmp_path):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    out = tmp_path / "k.s"
    cmd = [hipcc, *_build.FLAGS, *_build.EXTRA.get(src, []), "-S", "--cuda-device-only",
           os.path.join(CSRC, src), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    return out.read_text()


@pytest.mark.parametrize("src", ["seg_attn_direct.hip", "seg_attn_split.hip"])
def test_m0_only_inside_inline_asm(src, tmp_path):
    text = _asm(src, tmp_path)
    inside = False
    for line in text.splitlines():
        s = line.strip()
        if s.startswith(";;#ASMSTART"):
            inside = True
        elif s.startswith(";;#ASMEND"):
            inside = False
        elif not inside and not s.startswith(";") and re.search(r"\bm0\b", s):
            pytest.fail(f"compiler-generated M0 use outside the DMA asm: {s}")


@pytest.mark.parametrize("src", ["seg_attn_direct.hip", "seg_attn_split.hip", "seg_attn_staged.hip", "pack.hip"])
def test_no_scratch_spills(src, tmp_path):
    text = _asm(src, tmp_path)
    assert "scratch_store" not in text and "scratch_load" not in text


@pytest.mark.parametrize("src", ["seg_attn_direct.hip", "seg_attn_split.hip", "seg_attn_staged.hip"])
def test_operand_loads_stay_16_byte_vectors(src, tmp_path):
    """Every buffer load of the attention kernels moves 16 bytes per lane.  A
    single-dword buffer load here is the toolchain's miscompile of a 16-byte
    load whose elements are extracted and cast one by one (one dword loaded
    and replicated), which corrupts fp32 q / k / v."""
    text = _asm(src, tmp_path)
    assert not re.search(r"\bbuffer_load_dword\b", text)
