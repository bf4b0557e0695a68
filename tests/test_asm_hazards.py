"""The LDS copies of the attention kernels are issued from inline assembly
(`copy_to_lds` in attn_common.h), where the compiler's hazard pass does not
look.  A VALU write of an SGPR (v_readfirstlane / v_readlane) must be at least
5 wait states before a VMEM instruction that reads that SGPR; a copy that
reads its buffer descriptor too early reads a stale range, and its padding
lanes (offset 2^31, meant to fall out of range) then touch memory 2 GB past
the tile.  These tests compile the kernels to gfx950 assembly on the CPU and
check every copy.  No GPU needed."""

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KDIR = os.path.join(ROOT, "mccl-jax_amd", "src", "kernels")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

_COPY = re.compile(r"^buffer_load_dwordx4\s+\S+,\s+s\[(\d+):(\d+)\].*\blds\b")
_VALU_SGPR_WRITE = re.compile(r"^(v_readfirstlane_b32|v_readlane_b32)\s+(s\d+)\b")


def hazards(asm: str, window: int = 5):
    """Copies whose descriptor SGPRs were written by a VALU op fewer than
    `window` wait states earlier (s_nop N counts N + 1, any other
    instruction 1; labels, comments and directives count 0)."""
    lines = [l.strip() for l in asm.splitlines()]
    found = []
    for i, line in enumerate(lines):
        m = _COPY.match(line)
        if not m:
            continue
        regs = {f"s{k}" for k in range(int(m.group(1)), int(m.group(2)) + 1)}
        dist, j = 0, i - 1
        while j >= 0 and dist < window:
            t = lines[j]
            j -= 1
            if not t or t.startswith((";", ".")) or t.endswith(":"):
                continue
            if t.startswith("s_nop"):
                dist += int(t.split()[1]) + 1
                continue
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


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC), reason="hipcc not available")
@pytest.mark.parametrize("src", ["attention.hip", "attention_bwd.hip"])
def test_lds_copies_have_no_sgpr_hazard(src, tmp_path):
    out = tmp_path / (src + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-I" + os.path.join(ROOT, "include"), "-I" + KDIR, "--cuda-device-only", "-S",
           os.path.join(KDIR, src), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=300)
    asm = out.read_text()
    n_copies = sum(1 for l in asm.splitlines() if _COPY.match(l.strip()))
    assert n_copies > 0, "no LDS copies found: the pattern no longer matches the kernels"
    assert hazards(asm) == []
