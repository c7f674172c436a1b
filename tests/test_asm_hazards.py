"""Inline asm in the kernels is not covered by the compiler's MFMA hazard
checks.  Two cases are checked over the gfx950 assembly of the attention
kernels, which hold the only VALU inline asm (v_sad_u32 in the scan):
  * write after write: an asm instruction that writes a VGPR which an MFMA
    still in flight will write can have its result overwritten when the MFMA
    completes (a wrong value, no fault);
  * read after write: an asm instruction that reads a VGPR whose latest writer
    is an MFMA issued shortly before it may read the register before the
    MFMA's result lands, since no wait states are placed for it.
Both are flagged within a window of instructions longer than an MFMA's
latency in issue slots."""
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


def _writes_vgpr(op):
    """Instructions whose first operand is a VGPR they write (the rest read)."""
    return (op.startswith("v_") and not op.startswith(("v_cmp", "v_readlane", "v_readfirstlane"))) or \
        op.startswith(("ds_read", "ds_bpermute", "ds_permute", "ds_swizzle")) or "_load" in op


def _hazards(asm_text):
    """(inline-asm instruction, MFMA, kind) triples: the asm writes a register
    of the destination of an MFMA issued within WINDOW instructions before it
    ("waw"), or reads a register whose latest writer is such an MFMA
    ("raw")."""
    found, hist, in_asm, n_asm = [], [], False, 0
    last = {}  # VGPR -> (instruction index, op) of its latest writer
    idx = 0
    for line in asm_text.split("\n"):
        t = line.strip()
        if t.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if t.startswith(";;#ASMEND"):
            in_asm = False
            continue
        if t.startswith(".Lfunc_end"):
            hist, last = [], {}
        if not t or t.startswith((";", ".")) or t.endswith(":"):
            continue
        parts = t.replace(",", " ").split()
        op = parts[0]
        dst = _regs(parts[1]) if len(parts) > 1 and _writes_vgpr(op) else set()
        src = set()
        for tok in parts[2 if dst else 1:]:
            src |= _regs(tok)
        if in_asm and op.startswith("v_"):
            n_asm += 1
            for hop, hdst in hist[-WINDOW:]:
                if hop.startswith("v_mfma") and dst & hdst:
                    found.append((t, hop, "waw"))
                    break
            for r in sorted(src):
                w = last.get(r)
                if w and w[1].startswith("v_mfma") and idx - w[0] <= WINDOW:
                    found.append((t, w[1], "raw"))
                    break
        if op.startswith(("v_", "s_")):
            hist.append((op, dst))
        for r in dst:
            last[r] = (idx, op)
        idx += 1
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
    assert n == 1 and [k for _, _, k in found] == ["waw"]


def test_checker_flags_a_read_of_an_mfma_result():
    text = "\n".join([
        "\tv_mfma_i32_16x16x64_i8 v[24:27], v[0:3], v[4:7], 0",
        "\tv_add_u32_e32 v8, v9, v10",
        ";;#ASMSTART",
        "\tv_sad_u32 v40, v26, v8, 0",
        ";;#ASMEND",
    ])
    found, n = _hazards(text)
    assert n == 1 and [k for _, _, k in found] == ["raw"]


def test_checker_passes_a_read_of_a_rewritten_register():
    # v26 was an MFMA destination, but a later VALU instruction wrote it: the
    # asm reads that value, not the MFMA's
    text = "\n".join([
        "\tv_mfma_i32_16x16x64_i8 v[24:27], v[0:3], v[4:7], 0",
        "\ts_nop 7",
        "\tv_add_u32_e32 v26, v24, v10",
        ";;#ASMSTART",
        "\tv_sad_u32 v40, v26, v8, 0",
        ";;#ASMEND",
    ])
    found, n = _hazards(text)
    assert n == 1 and not found


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
