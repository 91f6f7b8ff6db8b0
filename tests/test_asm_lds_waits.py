"""The kernels that read LDS through inline asm (ds_read_b128 / ds_read_b64_tr_b16 with explicit
lgkmcnt waits: the MFMA mainloop of mfma_gemm.h, in the lm_head kernels and the split-K product)
must not touch a loaded register before its wait. The compiler treats an asm read's output as ready at once, so a move or an
operand it places between the read and the wait reads a register the LDS has not filled yet:
a data race that shows up as a wrong 64 x 64 block now and then, not as a fault. This test
compiles those sources to gfx950 assembly (the library's own flags) and scans every kernel
linearly: from an asm LDS read until the next lgkmcnt(0), no other instruction may read its
destination registers. CPU only (hipcc cross-compiles); skipped without hipcc.
"""

from __future__ import annotations

import re
import shutil
import subprocess

import pytest

from rus_amd import build

SOURCES = ("gemm.hip", "lmhead.hip")
_VREG = re.compile(r"v\[(\d+):(\d+)\]|\bv(\d+)\b")
_STORE = ("global_store", "ds_write", "buffer_store", "flat_store")


def _regs(text: str) -> set[int]:
    out: set[int] = set()
    for m in _VREG.finditer(text):
        if m.group(3):
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def early_reads(asm: str) -> dict[str, list[tuple[int, str]]]:
    """{kernel: [(line, instruction)]} of instructions reading a register that an inline-asm LDS
    read wrote and no lgkmcnt(0) wait has covered yet (linear scan of each kernel body)."""
    lines = asm.split("\n")
    kernels = re.findall(r"^\s+\.type\s+(\w+),@function", asm, re.M)
    found: dict[str, list[tuple[int, str]]] = {}
    for fn in kernels:
        start = next(i for i, l in enumerate(lines) if l.startswith(fn + ":"))
        pending: set[int] = set()
        in_asm = False
        bad = []
        for i in range(start + 1, len(lines)):
            s = lines[i].strip()
            if s.startswith("s_endpgm"):
                break
            if s == ";;#ASMSTART":
                in_asm = True
                continue
            if s == ";;#ASMEND":
                in_asm = False
                continue
            if not s or s.startswith((";", ".")):
                continue
            op = s.split()[0]
            if op == "s_waitcnt" and "lgkmcnt(0)" in s:
                pending.clear()
                continue
            if in_asm:
                if op.startswith("ds_read"):
                    pending |= _regs(s.split()[1].rstrip(","))
                continue
            parts = [p.strip() for p in s[len(op):].split(",")]
            used: set[int] = set()
            for p in parts if op.startswith(_STORE) else parts[1:]:
                used |= _regs(p)
            if pending & used:
                bad.append((i + 1, s))
            if parts and not op.startswith(_STORE + ("s_",)):
                pending -= _regs(parts[0])
        if bad:
            found[fn] = bad
    return found


def test_checker_flags_an_early_move():
    asm = "\n".join([
        "\t.type\t_Zk,@function", "_Zk:", ";;#ASMSTART", "ds_read_b64_tr_b16 v[10:11], v2 offset:0",
        ";;#ASMEND", "v_mov_b32_e32 v20, v11", ";;#ASMSTART", "s_waitcnt lgkmcnt(0)", ";;#ASMEND",
        "v_mov_b32_e32 v21, v10", "s_endpgm"])
    got = early_reads(asm)
    assert list(got) == ["_Zk"] and len(got["_Zk"]) == 1 and "v20, v11" in got["_Zk"][0][1]


@pytest.mark.skipif(shutil.which("hipcc") is None and not build.Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not available")
@pytest.mark.parametrize("src", SOURCES)
def test_no_register_read_before_its_lds_wait(src, tmp_path):
    out = tmp_path / (src + ".s")
    cmd = [build.hipcc(), *build.HIPCC_FLAGS, "--offload-device-only", "-S",
           str(build.CSRC_DIR / src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    assert early_reads(out.read_text()) == {}
