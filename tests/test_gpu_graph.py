"""The operator under HIP graph capture.

Each case captures one call (K2, the phase-2 pack, K3 and K4, or the dense kernel, all
launched on torch's current stream, which is the capture stream inside
``torch.cuda.graph``) and replays it three times, with eager calls on other inputs and
device synchronisations between the replays.  Every replay must equal the eager call on
the same inputs bit for bit (the kernels use no atomics, so a call is deterministic).
Then new values are copied into the captured inputs, and one more replay must equal the
eager call on those values.  None of these calls records a memset: the library clears
nothing, and torch's allocations inside the capture come from the graph's private pool.
"""
import sys

import pytest
import torch

from pasa_amd import ops
from pasa_amd.workloads import WORKLOADS, make_inputs, small_workload

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def bits(t):
    return t.view(torch.int32) if t.dtype == torch.float32 else t.view(torch.int16)


def capture(fn):
    """Warm ``fn`` up on a side stream (default priority), then capture one call of it."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    torch.cuda.synchronize()
    return g, out


def check_replays(name, wl, call, dtype, seed=0):
    """call(q, k, v) -> o.  Captured on static q, k, v; checked as the module docstring says."""
    dev = torch.device("cuda:0")
    q, k, v = (t.to(dev) for t in make_inputs(wl, seed=seed, dtype=dtype))
    q2, k2, v2 = (t.to(dev) for t in make_inputs(wl, seed=seed + 1, dtype=dtype))
    say(f"[graph] {name}: eager reference, {tuple(q.shape)} {dtype}")
    ref = call(q, k, v).clone()
    ref2 = call(q2, k2, v2).clone()
    torch.cuda.synchronize()
    assert not torch.equal(bits(ref), bits(ref2)), "the two input sets must give different outputs"
    say(f"[graph] {name}: capture")
    g, out = capture(lambda: call(q, k, v))
    for r in range(3):
        other = call(q2, k2, v2)  # eager work between replays, reusing the caching allocator's memory
        torch.cuda.synchronize()
        assert torch.equal(bits(other), bits(ref2)), f"eager call between replays differs ({name})"
        g.replay()
        torch.cuda.synchronize()
        say(f"[graph] {name}: replay {r}")
        assert torch.equal(bits(out), bits(ref)), f"replay {r} differs from the eager call ({name})"
    for dst, src in zip((q, k, v), (q2, k2, v2)):
        dst.copy_(src)
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(bits(out), bits(ref2)), f"replay on new inputs differs from the eager call ({name})"
    del g


C1 = WORKLOADS["c1"]
C3 = WORKLOADS["c3"]


def test_graph_operator_block128(device):
    wl = small_workload(C1, heads=2, grid=(5, 30, 52))  # T 7,800, NT 61
    check_replays("operator bf16 BT 128", wl,
                  lambda q, k, v: ops.pisa_pg_attention(q, k, v, wl.density, block_size=128, scale=wl.op_scale),
                  torch.bfloat16)


def test_graph_operator_block64_text(device):
    wl = small_workload(C3, heads=2, grid=(3, 10, 20), block_size=64, density=0.3, text_tokens=40,
                        prescale=1.0, scale=None)
    check_replays("operator bf16 BT 64, 40 text tokens (37 valid)", wl,
                  lambda q, k, v: ops.pisa_pg_attention(q, k, v, wl.density, block_size=64, scale=wl.op_scale,
                                                        text_tokens=40, text_valid=37),
                  torch.bfloat16)


def test_graph_operator_placed(device):
    wl = small_workload(C1, heads=2, grid=(6, 20, 30))  # F 6, P 600, T 3,600
    # The flags live on the device already: a host-to-device copy cannot be captured.
    flags = torch.tensor([1, 0], dtype=torch.int32, device=device)
    pl = ops.Placement(num_frame=6, frame_size=600, head_is_temporal=flags)
    check_replays("operator bf16 BT 128, placement folded in", wl,
                  lambda q, k, v: ops.pisa_pg_attention(q, k, v, wl.density, block_size=128, scale=wl.op_scale,
                                                        placement=pl),
                  torch.bfloat16)


def test_graph_operator_any_shape_fp32(device):
    wl = small_workload(C1, heads=1, grid=(2, 16, 32), head_dim=96, block_size=64, density=0.25,
                        dtype=torch.float32, prescale=1.0, scale=None)
    assert not ops.tuned_shape(torch.float32, 96, 64, 16)
    check_replays("operator fp32 D 96 BT 64 G 16 (any-shape kernels)", wl,
                  lambda q, k, v: ops.pisa_pg_attention(q, k, v, wl.density, block_size=64, group_size=16,
                                                        scale=wl.op_scale),
                  torch.float32)


def test_graph_dense(device):
    wl = small_workload(C3, heads=2, grid=(2, 16, 32), text_tokens=64, prescale=1.0, scale=None)
    check_replays("dense bf16 with a padded text segment", wl,
                  lambda q, k, v: ops.dense_attention(q, k, v, text_tokens=64, text_valid=50),
                  torch.bfloat16)


def test_graph_noalloc_entry(device):
    """The allocation-free entry, the one meant for captured code: statistics and selection
    computed eagerly, the attention call alone captured, its output buffer given."""
    wl = small_workload(C1, heads=2, grid=(5, 30, 52))
    dev = torch.device("cuda:0")
    q, k, v = (t.to(dev) for t in make_inputs(wl, seed=3, dtype=torch.bfloat16))
    st = ops.block_stats(q, k, v, 128, 32)
    sel = ops.select_blocks(st, wl.density, wl.op_scale, indices=False)
    out = torch.empty_like(v)
    run = lambda: ops.sparse_attn_noalloc(q, k, v, st, sel, wl.op_scale, 128, out=out)
    ref = ops.sparse_attn(q, k, v, st, sel, wl.op_scale, 128).clone()
    run()  # the first call on the device looks up the static scratch's address
    torch.cuda.synchronize()
    assert torch.equal(bits(out), bits(ref))
    say("[graph] noalloc entry: capture")
    g, o = capture(run)
    assert o.data_ptr() == out.data_ptr()
    for r in range(3):
        out.fill_(float("nan"))  # a fill kernel, outside the graph
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        say(f"[graph] noalloc entry: replay {r}")
        assert torch.equal(bits(out), bits(ref)), f"replay {r} differs"
    del g
