"""The allocation-free attention entry (pasa_sparse_attn_noalloc) against the
workspace entry (pasa_sparse_attn): the same kernels on the same inputs, so the
outputs must be bitwise equal.  Two calls in a row on one device, the second on a
smaller input (fewer slices and groups, block size 64, a padded text segment), so
the second call runs on the first call's leftover pack in the static scratch."""
import sys

import pytest
import torch

from pasa_amd import _lib, ops
from pasa_amd.workloads import WORKLOADS, make_inputs, small_workload

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def run_both(wl, text_valid=None, gamma="literal", seed=0):
    dev = torch.device("cuda:0")
    q, k, v = (t.to(dev) for t in make_inputs(wl, seed=seed, dtype=torch.bfloat16))
    BT, text = wl.block_size, wl.text_tokens
    st = ops.block_stats(q, k, v, BT, 32, text_tokens=text)
    sel = ops.select_blocks(st, wl.density, wl.op_scale)
    ref = ops.sparse_attn(q, k, v, st, sel, wl.op_scale, BT, gamma, text_tokens=text, text_valid=text_valid)
    out = torch.full_like(v, float("nan"))  # every row must be written
    got = ops.sparse_attn_noalloc(q, k, v, st, sel, wl.op_scale, BT, gamma, out=out, text_tokens=text,
                                  text_valid=text_valid)
    torch.cuda.synchronize()
    assert got.data_ptr() == out.data_ptr()
    return ref.cpu(), got.cpu()


def test_noalloc_equals_workspace_entry_two_calls(device):
    lib = _lib.load()
    big = small_workload(WORKLOADS["c1"], heads=3, grid=WORKLOADS["c1"].grid)   # 3 x 32760, BT 128, NG 8
    need = lib.pasa_sparse_attn_workspace_bytes(big.heads, big.seq_len, 0, 128, big.block_size, 32)
    say(f"[noalloc] call 1: {big.heads} heads x {big.seq_len} tokens, BT {big.block_size}, pack {need} bytes")
    ref, got = run_both(big)
    assert torch.equal(ref.view(torch.int16), got.view(torch.int16)), "call 1 differs from pasa_sparse_attn"

    small = small_workload(WORKLOADS["c3"], heads=1, grid=(3, 10, 20), block_size=64, density=0.3,
                           text_tokens=40, prescale=1.0, scale=None)
    need2 = lib.pasa_sparse_attn_workspace_bytes(1, small.seq_len, 40, 128, 64, 32)
    assert need2 < need
    say(f"[noalloc] call 2: 1 head x {small.seq_len} tokens (40 text, 37 valid), BT 64, pack {need2} bytes")
    ref2, got2 = run_both(small, text_valid=37, gamma="consistent", seed=1)
    assert torch.equal(ref2.view(torch.int16), got2.view(torch.int16)), "call 2 differs from pasa_sparse_attn"
    assert not torch.isnan(got2.float()).any()
