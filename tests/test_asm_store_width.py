"""The bandwidth-bound kernels move 16-byte packs, and each pack must leave as one 16-byte access.
Where two branches stored the same pack, the compiler once merged the stores and split them into
2-, 4- and 8-byte pieces at odd offsets (a 16-byte store as short + dwordx2 + dword + short): the
RoPE forward then issued 2.5x the write requests its output needs. This test compiles those
sources to gfx950 assembly (the library's own flags) and fails on any global store of a split
pack in the kernels that are meant to have none. CPU only (hipcc cross-compiles); skipped
without hipcc.
"""

from __future__ import annotations

import re
import shutil
import subprocess

import pytest

from rus_amd import build

# A piece of a split pack: a 2-byte store, or a 4 / 8 / 12-byte store at an offset that is not a
# multiple of its own width within the 16-byte pack.
_SPLIT = re.compile(
    r"global_store_short\b|global_store_byte\b"
    r"|global_store_dword\s+v\[\d+:\d+\],\s*v\d+,\s*off\s+offset:(?:2|6|10|14)\b"
    r"|global_store_dwordx[23]\s+v\[\d+:\d+\],\s*v\[\d+:\d+\],\s*off\s+offset:(?:2|4|6|10)\b")

# kernels (mangled-name fragments) that write only whole 16-byte packs, per source; scalar
# stores of single values are legitimate elsewhere (fp16 LoRA mid values, counters, flags).
PACK_ONLY = {
    "rope.hip": ("rope_fwd_kernel", "rope_bwd_kernelIDF16"),
    "swiglu.hip": ("swiglu_fwd_kernelIDF16_Li8", "swiglu_bwd_kernelIDF16_Li8"),
    "rmsnorm.hip": ("rmsnorm_fwd_wide", "rmsnorm_bwd_wide"),
    "nf4_dequant.hip": ("nf4_dequant_multi_kernel", "nf4_dequant_norm_kernel"),
}


def split_stores(asm: str, fragments: tuple[str, ...]) -> dict[str, list[str]]:
    """{kernel: [store]} of split-pack stores in the kernels whose names contain a fragment."""
    found: dict[str, list[str]] = {}
    cur = None
    for line in asm.split("\n"):
        m = re.match(r"^(_Z\w+):\s*(;.*)?$", line)
        if m:
            cur = m.group(1) if any(f in m.group(1) for f in fragments) else None
            continue
        if cur and _SPLIT.search(line):
            found.setdefault(cur, []).append(line.strip())
    return found


def test_checker_flags_a_split_pack():
    asm = "\n".join(["_ZN3rus12rope_fwd_kernelE:", "\tglobal_store_dwordx4 v[0:1], v[2:5], off",
                     "\tglobal_store_short v[0:1], v8, off offset:14",
                     "\tglobal_store_dword v[0:1], v2, off offset:10",
                     "\tglobal_store_dwordx2 v[0:1], v[4:5], off offset:2", "\ts_endpgm",
                     "_ZN3rus12other_kernelE:", "\tglobal_store_short v[0:1], v8, off"])
    got = split_stores(asm, ("rope_fwd_kernel",))
    assert list(got) == ["_ZN3rus12rope_fwd_kernelE"] and len(got["_ZN3rus12rope_fwd_kernelE"]) == 3


@pytest.mark.skipif(shutil.which("hipcc") is None and not build.Path("/opt/rocm/bin/hipcc").exists(),
                    reason="hipcc not available")
@pytest.mark.parametrize("src", sorted(PACK_ONLY))
def test_packs_leave_as_whole_16_byte_stores(src, tmp_path):
    out = tmp_path / (src + ".s")
    cmd = [build.hipcc(), *build.HIPCC_FLAGS, "--offload-device-only", "-S",
           str(build.CSRC_DIR / src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    asm = out.read_text()
    # the kernels exist under these names (a rename would otherwise pass silently)
    for frag in PACK_ONLY[src]:
        assert re.search(rf"^_Z\w*{frag}\w*:", asm, re.M), frag
    assert split_stores(asm, PACK_ONLY[src]) == {}
