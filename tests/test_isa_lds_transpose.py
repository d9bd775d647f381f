"""The prefill and balanced decode / verify kernels issue their LDS transpose reads
(ds_read_b64_tr_b16) from inline assembly, so
the compiler neither waits for them nor knows that their destination registers are still being
written until the explicit `s_waitcnt lgkmcnt(0)` that follows.  This test compiles
pkv_attention.hip for gfx950 to assembly and checks, for every such read in every kernel, that no
instruction between the read and that wait touches a register the read is filling, and that the
wait comes before the end of the program.  Needs hipcc (no GPU)."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from prism_amd import build as pbuild

SRC = pbuild.CSRC / "pkv_attention.hip"


def _regs(operand: str) -> set[int]:
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", operand)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"v(\d+)", operand)
    return {int(m.group(1))} if m else set()


def _operand_regs(line: str) -> set[int]:
    out: set[int] = set()
    for tok in re.findall(r"v\[\d+:\d+\]|\bv\d+\b", line):
        out |= _regs(tok)
    return out


@pytest.fixture(scope="module")
def asm(tmp_path_factory) -> str:
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa") / "attn.s"
    flags = [f for f in pbuild.HIPCC_FLAGS if f != "-fPIC"]
    subprocess.run([hipcc, *flags, "--cuda-device-only", "-S", str(SRC), "-o", str(out)], check=True,
                   stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    return out.read_text()


def test_transpose_reads_are_waited_for_before_use(asm):
    lines = asm.splitlines()
    n_reads = 0
    i = 0
    while i < len(lines):
        line = lines[i].strip()
        if not line.startswith("ds_read_b64_tr_b16"):
            i += 1
            continue
        # a run of reads, then the instructions up to the explicit wait
        pending: set[int] = set()
        j = i
        while j < len(lines):
            cur = lines[j].split(";")[0].strip()
            if cur.startswith("ds_read_b64_tr_b16"):
                dst, addr = [t.strip() for t in cur.split(None, 1)[1].split(",")[:2]]
                assert not (_regs(dst) & pending), f"line {j + 1}: a transpose read overwrites a pending one: {cur}"
                assert not (_regs(addr) & pending), f"line {j + 1}: address from a pending read: {cur}"
                pending |= _regs(dst)
                n_reads += 1
            elif cur == "s_waitcnt lgkmcnt(0)":
                break
            elif cur and not cur.startswith((".", "s_", ";")) and not cur.endswith(":"):
                touched = _operand_regs(cur) & pending
                assert not touched, f"line {j + 1}: {cur!r} touches v{sorted(touched)} before the wait"
            elif cur.startswith(("s_endpgm", "s_setpc")):
                raise AssertionError(f"line {j + 1}: program ends with transpose reads outstanding")
            j += 1
        assert j < len(lines), "no wait after the transpose reads"
        i = j + 1
    assert n_reads >= 16, "the prefill kernel's transpose reads were not found"
