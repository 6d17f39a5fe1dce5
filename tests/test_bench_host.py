"""The bench contract on the CPU: a multi-GPU request exits with a message (this build
measures one GPU), and the algorithmic K4 FLOP count behind ``value`` matches the count
of work the kernel issues."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

from pasa_amd.workloads import WORKLOADS

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.parametrize("argv, env", [(["--gpus", "2"], {}), (["--gpus", "8"], {}), ([], {"WORLD_SIZE": "2"})])
def test_more_than_one_gpu_exits_with_a_message(argv, env):
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), *argv], capture_output=True, text=True,
                       env={**os.environ, **env}, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_c2_flops_equal_the_mfma_work():
    """c2 at block 128: every (query block, selected block) pair is one 128 x 128 x 128 tile
    of S = QK^T and one of P.V (4 D BT^2 FLOP), and every (query block, group) pair one
    32-block score tile, one P-bar.V-hat and one Q.H-bar product.  K4 issues
    886,594,560 16x16x32 MFMAs per launch at c2 (rocprofv3 SQ_INSTS_MFMA, every dispatch), each
    16,384 FLOP: the count below is that number of MFMAs exactly.  A wave owns 32 query rows,
    two 16-row tiles; each product is (output tiles of 16 x 16) x (k-steps of 32)."""
    wl = WORKLOADS["c2"]
    BH, D, BT, G = 40, 128, 128, 32
    NT = -(-75600 // BT)
    NS, NG = int(0.1 * NT), -(-NT // G)
    assert (NT, NS, NG) == (591, 59, 19)
    qt = 2                                                                   # 16-row query tiles per wave
    per_wave_mfma_tile = (BT // 16) * qt * (D // 32) + (D // 16) * qt * (BT // 32)   # S and P.V
    per_wave_mfma_group = (G // 16) * qt * (D // 32) + (D // 16) * qt * (G // 32) + (D // 16) * qt * (D // 32)
    waves = BH * NT * (BT // 32)
    mfma = waves * (NS * per_wave_mfma_tile + NG * per_wave_mfma_group)
    assert mfma == 886_594_560
    assert wl.k4_flops(G, NS) == mfma * 16 * 16 * 32 * 2


def test_c3_text_flops():
    """c3 adds the text segment: video rows x text keys and dense text rows, 4 D per pair."""
    wl = WORKLOADS["c3"]
    no_text = wl.__class__(**{**wl.__dict__, "text_tokens": 0})
    Tv, X, BH, D = 118800, 256, 24, 128
    assert wl.k4_flops() - no_text.k4_flops() == 4 * D * (Tv * X + X * (Tv + X)) * BH
