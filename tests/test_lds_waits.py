"""No compiler-inserted wait for in-flight copies before an LDS read.

The ring kernels copy their next stage into LDS with buffer_load ... lds
while they compute on the current one.  Before an LDS load that carries no
alias information, the compiler waits for every outstanding copy
(s_waitcnt vmcnt), which would make each stage's math wait for the next
stage's copies.  The kernels read such data through settled loads or typed
field loads instead (common.hpp, qformats.hpp).  This test compiles the
sources to gfx950 assembly (no GPU needed) and checks that no kernel has a
compiler-emitted vmcnt wait directly before an LDS read, except the two
known ones outside any loop.
"""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from ane_amd.build import HIP_FLAGS, hipcc

ROOT = Path(__file__).resolve().parents[1]
SOURCES = ["q8_0.hip", "q8_0_mmv.hip", "gemm_i8_tile256.hip", "gemm_i8_tile128d.hip", "decode.hip",
           "qformats.hip"]
# waits that are not in a loop: the skinny contraction's epilogue
ALLOWED = ("k_gemm_skinny",)


def lds_read_waits(asm: str) -> dict:
    """kernel symbol -> number of compiler-emitted vmcnt waits whose next
    instruction is an LDS read (waits inside inline asm excluded)."""
    out = {}
    kernel = None
    in_asm = False
    lines = asm.split("\n")
    for i, line in enumerate(lines):
        m = re.match(r"^(_Z\S+):", line)
        if m:
            kernel = m.group(1)
            out.setdefault(kernel, 0)
            continue
        s = line.strip()
        if "ASMSTART" in s:
            in_asm = True
            continue
        if "ASMEND" in s:
            in_asm = False
            continue
        if kernel is None or in_asm:
            continue
        if s == "s_endpgm":
            kernel = None
            continue
        if s.startswith("s_waitcnt") and "vmcnt(" in s:
            j = i + 1
            while j < len(lines) and (not lines[j].strip() or lines[j].strip().startswith((";", "s_waitcnt"))):
                j += 1
            if j < len(lines) and lines[j].strip().startswith("ds_read"):
                out[kernel] += 1
    return out


def test_parser_counts_a_wait_before_an_lds_read():
    asm = "\n".join([
        "_ZN3ane1kEv:", "\tbuffer_load_dwordx4 v0, s[0:3], 0 offen lds", "\ts_waitcnt vmcnt(0)",
        "\tds_read_b128 v[0:3], v4", "\t;;#ASMSTART", "\ts_waitcnt vmcnt(0)", "\tds_read_b32 v1, v2",
        "\t;;#ASMEND", "\ts_waitcnt vmcnt(3)", "\tv_add_f32 v0, v1, v2", "\ts_endpgm"])
    assert lds_read_waits(asm) == {"_ZN3ane1kEv": 1}


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not available")
@pytest.mark.parametrize("src", SOURCES)
def test_no_wait_for_copies_before_lds_reads(src, tmp_path):
    flags = [f for f in HIP_FLAGS if f != "-fPIC"]
    out = tmp_path / (Path(src).stem + ".s")
    subprocess.run([hipcc(), *flags, "--cuda-device-only", "-S", str(ROOT / "ane_amd" / "csrc" / src),
                    "-o", str(out)], check=True, capture_output=True)
    bad = {k: n for k, n in lds_read_waits(out.read_text()).items()
           if n and not any(a in k for a in ALLOWED)}
    assert not bad, f"compiler vmcnt waits before LDS reads: {bad}"
