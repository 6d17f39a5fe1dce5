"""The direct-to-LDS tile loads (dma_load16_lds and dma_load16_lds_nt in pasa_amd/csrc/common.h) write m0
inside inline assembly, which the compiler cannot see.  That is safe only while no
kernel also contains a compiler-generated m0 user (whose m0 value the compiler may
set once and hoist).  This compiles the kernels that use the load to gfx950
assembly and checks that every m0 access is the load's own s_mov_b32 m0 / s_nop 0 /
buffer_load_dwordx4 ... lds sequence.  CPU only (hipcc cross-compiles)."""
import os
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "pasa_amd" / "csrc"
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not available")
@pytest.mark.parametrize("src", ["sparse_attn.hip", "block_stats.hip", "select.hip"])
def test_only_the_dma_load_touches_m0(src, tmp_path):
    out = tmp_path / (src + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", str(CSRC / src), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    lines = [l.split(";")[0].strip() for l in out.read_text().splitlines()]
    lines = [l for l in lines if l and not l.startswith(".")]
    n_loads = 0
    for i, l in enumerate(lines):
        if not re.search(r"\bm0\b", l):
            continue
        assert re.fullmatch(r"s_mov_b32 m0, s\d+", l), f"{src}: unexpected m0 access: {l}"
        assert lines[i + 1] == "s_nop 0", f"{src}: m0 write not followed by the wait state: {lines[i + 1]}"
        assert lines[i + 2].startswith("buffer_load_dwordx4") and lines[i + 2].endswith(" lds"), \
            f"{src}: m0 write not followed by an LDS-direct load: {lines[i + 2]}"
        n_loads += 1
    assert n_loads > 0, f"{src}: no direct-to-LDS loads found"
