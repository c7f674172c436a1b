"""Inline asm in the kernels is not covered by the compiler's MFMA hazard
checks: an asm instruction that writes a VGPR which an MFMA still in flight
will write can have its result overwritten when the MFMA completes (a wrong
value, no fault).  The attention kernels hold the only VALU inline asm
(v_sad_u32 in the scan); this compiles them to gfx950 assembly and checks
that no inline-asm write lands in the destination registers of an MFMA
issued shortly before it."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "compress-zip_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"
WINDOW = 40  # instructions back: more than an MFMA's latency in issue slots


def _regs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def _hazards(asm_text):
    """(inline-asm instruction, MFMA) pairs where the asm writes a register of
    the MFMA's destination within WINDOW instructions after it."""
    found, hist, in_asm, n_asm = [], [], False, 0
    for line in asm_text.split("\n"):
        t = line.strip()
        if t.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if t.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if t.startswith(".Lfunc_end"):
            hist = []
        if not t or t.startswith((";", ".")) or t.endswith(":"):
            continue
        parts = t.replace(",", " ").split()
        op = parts[0]
        dst = _regs(parts[1]) if len(parts) > 1 else set()
        if in_asm and op.startswith("v_"):
            n_asm += 1
            for hop, hdst in hist[-WINDOW:]:
                if hop.startswith("v_mfma") and dst & hdst:
                    found.append((t, hop))
                    break
        if op.startswith(("v_", "s_")):
            hist.append((op, dst))
    return found, n_asm


def test_checker_flags_a_write_into_an_mfma_destination():
    text = "\n".join([
        "\tv_mfma_i32_16x16x64_i8 v[24:27], v[0:3], v[4:7], 0",
        "\tv_add_u32_e32 v8, v9, v10",
        ";;#ASMSTART",
        "\tv_ffbl_b32 v25, v55",
        ";;#ASMEND",
    ])
    found, n = _hazards(text)
    assert n == 1 and len(found) == 1


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
@pytest.mark.parametrize("src", ["czip_attention.hip", "czip_decode.hip"])
def test_no_inline_asm_write_into_an_mfma_destination(tmp_path, src):
    out = tmp_path / (src + ".s")
    cmd = [HIPCC, "-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "-I", os.path.join(ROOT, "include"), "-I", CSRC, "-x", "hip", "-S",
           "--offload-device-only", os.path.join(CSRC, src), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    found, n_asm = _hazards(out.read_text())
    assert n_asm > 0  # the scan's v_sad_u32 is there to check
    assert not found, found[:3]
