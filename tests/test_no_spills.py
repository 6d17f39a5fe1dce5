"""The MFMA kernels run at two waves per SIMD with 230-256 VGPRs per lane, at the edge of the
register file: a small source change can make the compiler spill to scratch memory, which
costs far more than the change saves and shows up only as a slower kernel.  This compiles
the tuned kernels to gfx950 assembly and checks that none of them spills a VGPR, that the
attention kernels spill no SGPR either (SGPR spills go to VGPR lanes, a few instructions
each; K2's placed fp16 instantiation has two, outside its block loop), and that each keeps
the occupancy it is launched for.  CPU only (hipcc cross-compiles)."""
import os
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "pasa_amd" / "csrc"
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# kernel name prefix (after "pasa::") -> (most VGPRs per lane its occupancy allows, SGPR spills allowed)
KERNELS = {
    "sparse_attn.hip": {"k4_sparse_attn_dma": (256, False), "k4_sparse_attn": (256, False)},
    "block_stats.hip": {"k2_block_stats_dma": (512, True)},
    "select.hip": {"k3_scores": (512, False)},
}


def _kernels(asm: str):
    """(name, vgpr_count, vgpr_spill_count, sgpr_spill_count) per kernel from the metadata."""
    out = []
    for block in re.split(r"\n\s+- \.", asm):
        m = re.search(r"\.name:\s+(\S+)", block)
        if not m:
            continue
        def num(key):
            k = re.search(r"\.%s:\s+(\d+)" % key, block)
            return int(k.group(1)) if k else None
        out.append((m.group(1), num("vgpr_count"), num("vgpr_spill_count"), num("sgpr_spill_count")))
    return out


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not available")
@pytest.mark.parametrize("src", sorted(KERNELS))
def test_mfma_kernels_do_not_spill(src, tmp_path):
    out = tmp_path / (src + ".s")
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", str(CSRC / src), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    seen = {p: 0 for p in KERNELS[src]}
    for name, vgprs, vspill, sspill in _kernels(out.read_text()):
        for prefix, (limit, sgpr_ok) in KERNELS[src].items():
            # mangled: _ZN4pasa<len><name>I... ; match the exact kernel name
            if re.match(r"_ZN4pasa%d%sI" % (len(prefix), prefix), name):
                seen[prefix] += 1
                assert vspill == 0, f"{src}: {name} spills {vspill} VGPRs"
                assert sgpr_ok or sspill == 0, f"{src}: {name} spills {sspill} SGPRs"
                assert vgprs is not None and vgprs <= limit, f"{src}: {name} uses {vgprs} VGPRs (limit {limit})"
    assert all(seen.values()), f"{src}: kernels not found: {[p for p, n in seen.items() if not n]}"
