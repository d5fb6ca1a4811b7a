"""The MLA fast pass issues its S^T MFMAs as inline asm, so the compiler cannot see their latency:
no instruction may read the accumulator until the MFMA's result is ready (18 wait states for a
16-pass 32x32 MFMA; back-to-back MFMAs that accumulate into the same registers are exempt). The
waits are written as nops tied to the accumulator; this test compiles the kernel for gfx950 and
checks the emitted schedule, since a change elsewhere can make the compiler move a read."""
import os
import re
import shutil
import subprocess
from pathlib import Path

import pytest

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
SRC = Path(__file__).resolve().parent.parent / "torchair_amd" / "csrc" / "attention.hip"
KERNEL = "_ZN3tai12_GLOBAL__N_117mla_decode_kernelILi512ELi64ELb0EEEvNS0_7MlaArgsE"
WAIT_STATES = 18


def _regs(text):
    out = set()
    for m in re.finditer(r"\bv(\d+)\b", text):
        out.add(int(m.group(1)))
    for m in re.finditer(r"\bv\[(\d+):(\d+)\]", text):
        out |= set(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def hazards(asm_lines):
    """(line, text) of every instruction that reads a VGPR MFMA destination too early."""
    found, pending, dst, waits = [], False, set(), 0
    for i, line in enumerate(asm_lines):
        t = line.strip()
        if not t or t.startswith((";", ".")):
            continue
        m = re.match(r"v_mfma\w*\s+v\[(\d+):(\d+)\]", t)
        if m:
            pending, dst, waits = True, set(range(int(m.group(1)), int(m.group(2)) + 1)), 0
            continue
        if not pending:
            continue
        if t.startswith("v_mfma"):  # an MFMA into AGPRs: does not read the VGPR accumulator
            continue
        nop = re.match(r"s_nop (\d+)", t)
        if nop:
            waits += int(nop.group(1)) + 1
        else:
            if _regs(t) & dst:
                found.append((i, t))
            waits += 1
        if waits >= WAIT_STATES:
            pending = False
    return found


def test_hazard_checker_flags_an_early_read():
    lines = ["v_mfma_f32_32x32x16_bf16 v[2:17], v[20:23], v[24:27], v[2:17]", "s_nop 3",
             "v_mul_f32_e32 v2, s31, v2"]
    assert hazards(lines) == [(2, "v_mul_f32_e32 v2, s31, v2")]
    assert hazards(lines[:1] + ["s_nop 15", "s_nop 7"] + lines[2:]) == []


@pytest.mark.skipif(not shutil.which(HIPCC) and not Path(HIPCC).exists(), reason="hipcc not available")
def test_mla_fast_pass_reads_no_mfma_result_early(tmp_path):
    out = tmp_path / "attention.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fhip-fp32-correctly-rounded-divide-sqrt",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-result",
           "--cuda-device-only", "-S", str(SRC), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    text = out.read_text()
    start = text.index(KERNEL + ":")
    body = text[start:text.index("s_endpgm", start)].splitlines()
    assert any("v_mfma_f32_32x32x16_bf16 v[" in l for l in body), "expected VGPR-destination MFMAs"
    assert hazards(body) == []


def test_no_inline_asm_vector_memory_stores():
    """A vector-memory store written as inline asm hides its data registers from the compiler's hazard
    recognizer: the next VALU may overwrite them before the store has read them (a >8-byte store
    reads its data over several cycles), which corrupted grouped-GEMM output rows. Stores with a
    cache policy use the compiler's non-temporal store on a global-address-space pointer instead."""
    csrc = SRC.parent
    pat = re.compile(r'asm\s+volatile\(\s*"\s*(global|buffer|flat|scratch)_store')
    offenders = [f"{p.name}:{i + 1}" for p in sorted(csrc.glob("*.hip"))
                 for i, line in enumerate(p.read_text().splitlines()) if pat.search(line)]
    assert offenders == []
