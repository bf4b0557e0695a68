"""The LDS copies of the attention and tiled GEMM kernels are issued from
inline assembly (`copy_to_lds`, `copy_to_lds_so` in attn_common.h), where the
compiler's hazard pass does not look.  A VALU write of an SGPR
(v_readfirstlane / v_readlane) must be at least 5 wait states before a VMEM
instruction that reads that SGPR; a copy that reads its buffer descriptor (or
its SGPR offset) too early reads a stale range, and its padding lanes (offset
2^31, meant to fall out of range) then touch memory 2 GB past the tile.  The
M0 write that sets a copy's LDS address needs one wait state before the copy.
These tests compile the kernels to gfx950 assembly on the CPU, with the flags
the library is built with, and check every copy.  No GPU needed."""

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KDIR = os.path.join(ROOT, "mccl-jax_amd", "src", "kernels")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

_COPY = re.compile(r"^buffer_load_dwordx4\s+\S+,\s+s\[(\d+):(\d+)\],\s+(s\d+|\S+)\b.*\blds\b")
_VALU_SGPR_WRITE = re.compile(r"^(v_readfirstlane_b32|v_readlane_b32)\s+(s\d+)\b")
_M0_WRITE = re.compile(r"^\S+\s+m0\b")


def hazards(asm: str, window: int = 5):
    """Copies whose descriptor or SGPR-offset registers were written by a
    VALU op fewer than `window` wait states earlier, or whose M0 was written
    by the instruction right before them (s_nop N counts N + 1 wait states,
    any other instruction 1; labels, comments and directives count 0)."""
    lines = [l.strip() for l in asm.splitlines()]
    found = []
    for i, line in enumerate(lines):
        m = _COPY.match(line)
        if not m:
            continue
        regs = {f"s{k}" for k in range(int(m.group(1)), int(m.group(2)) + 1)}
        if m.group(3).startswith("s"):
            regs.add(m.group(3))
        dist, j = 0, i - 1
        while j >= 0 and dist < window:
            t = lines[j]
            j -= 1
            if not t or t.startswith((";", ".")) or t.endswith(":"):
                continue
            if t.startswith("s_nop"):
                dist += int(t.split()[1]) + 1
                continue
            if dist == 0 and _M0_WRITE.match(t):
                found.append((i, t, line))
                break
            w = _VALU_SGPR_WRITE.match(t)
            if w and w.group(2) in regs:
                found.append((i, t, line))
                break
            dist += 1
    return found


def test_checker_flags_a_short_window():
    bad = "v_readfirstlane_b32 s10, v3\ns_mov_b32 m0, s4\ns_nop 0\nbuffer_load_dwordx4 v1, s[8:11], 0 offen lds\n"
    good = "v_readfirstlane_b32 s10, v3\ns_mov_b32 m0, s4\ns_nop 4\nbuffer_load_dwordx4 v1, s[8:11], 0 offen lds\n"
    other = "v_readfirstlane_b32 s12, v3\ns_nop 0\nbuffer_load_dwordx4 v1, s[8:11], 0 offen lds\n"
    assert len(hazards(bad)) == 1
    assert hazards(good) == []
    assert hazards(other) == []
    # the SGPR offset of copy_to_lds_so is checked like the descriptor
    soff_bad = "v_readfirstlane_b32 s7, v3\ns_nop 0\nbuffer_load_dwordx4 v1, s[8:11], s7 offen lds\n"
    soff_good = "v_readfirstlane_b32 s7, v3\ns_nop 4\nbuffer_load_dwordx4 v1, s[8:11], s7 offen lds\n"
    assert len(hazards(soff_bad)) == 1
    assert hazards(soff_good) == []
    # M0 written by the instruction right before the copy
    m0_bad = "s_mov_b32 m0, s5\nbuffer_load_dwordx4 v1, s[8:11], s7 offen lds\n"
    m0_good = "s_mov_b32 m0, s5\ns_nop 0\nbuffer_load_dwordx4 v1, s[8:11], s7 offen lds\n"
    assert len(hazards(m0_bad)) == 1
    assert hazards(m0_good) == []


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC), reason="hipcc not available")
@pytest.mark.parametrize("src", ["attention.hip", "attention_bwd.hip", "gemm_tiled.hip"])
def test_lds_copies_have_no_sgpr_hazard(src, tmp_path):
    out = tmp_path / (src + ".s")
    # per-file flags as in mccl-jax_amd/Makefile
    extra = ["-mllvm", "-amdgpu-mfma-vgpr-form"] if src == "attention.hip" else []
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", *extra, "-I" + os.path.join(ROOT, "include"), "-I" + KDIR, "--cuda-device-only",
           "-S", os.path.join(KDIR, src), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=300)
    asm = out.read_text()
    n_copies = sum(1 for l in asm.splitlines() if _COPY.match(l.strip()))
    assert n_copies > 0, "no LDS copies found: the pattern no longer matches the kernels"
    assert hazards(asm) == []
