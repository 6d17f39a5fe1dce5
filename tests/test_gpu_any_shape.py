"""GPU parity of the any-shape kernels (pasa_amd/csrc/any_shape.hip) against the CPU oracle.

These serve the calls the tuned kernels do not take, as the reference does
(svg/kernels/triton/group_pisa_attention.py:307-398 accepts any float dtype, any group size
and any power-of-two block size): fp32 q, k, v; head dims 1 .. 128; group sizes other than
32; block sizes 16 .. 256.  Every call here goes through the C ABI of libpasa_amd.so.

  * fp32: the north_star criterion literally -- cosine >= 0.999 and max|err| <= 2e-2 x
    RMS against the oracle's fp32 evaluation (no output rounding to allow for).
  * bf16 / fp16: as the tuned kernels are held, to the oracle run at the reference's own
    roundings in that type (kc, vc, Hbar, P and the output stored in it): max|err| within
    1.5x that floor's (+ one ulp), and the error beyond one ulp within the north_star bound.
  * statistics: against the fp64 oracle to fp32 tolerance."""
import math
import sys

import pytest
import torch

from oracle import pisa_oracle as O
from pasa_amd import ops
from pasa_amd.workloads import WORKLOADS, Workload, make_inputs, small_workload

pytestmark = pytest.mark.gpu

COS_MIN = 0.999
BOUND = 2e-2


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def inputs(heads, T, D, dtype, seed, text=0):
    """Q, K, V = N(0,1) plus a shared smooth positional component (attention mass local),
    the c0 recipe at an arbitrary size; text rows pure N(0,1)."""
    g = torch.Generator().manual_seed(seed)
    pos = torch.arange(T - text, dtype=torch.float32)[:, None]
    lam = torch.rand(D, generator=g) * 6 + 2
    phi = torch.rand(D, generator=g) * 2 * math.pi
    wave = torch.sin(2 * math.pi * pos / lam + phi)
    q, k, v = (torch.randn(1, heads, T, D, generator=g) for _ in range(3))
    q[..., : T - text, :] += wave
    k[..., : T - text, :] += wave
    return q.to(dtype), k.to(dtype), v.to(dtype)


def check(out, ref, what, dtype, floor=None):
    m = O.parity_metrics(out, ref, torch.bfloat16 if dtype == torch.float32 else dtype)
    say(f"[any] {what}: cos={m['cos']:.7f} max_abs/rms={m['max_abs_over_rms']:.3e} "
        f"excess/rms={m['excess_over_rms']:.3e}"
        + ("" if floor is None else f" floor max_abs/rms={floor['max_abs_over_rms']:.3e}"))
    assert m["cos"] >= COS_MIN, (what, m)
    if dtype == torch.float32:
        assert m["max_abs_over_rms"] <= BOUND, (what, m)      # the north_star bound, literally
    else:
        assert m["excess_over_rms"] <= max(BOUND, 1.5 * floor["excess_over_rms"]), (what, m, floor)
        ulp = float(O.ulp(torch.tensor(ref.abs().max().item()), dtype))
        assert m["max_abs"] <= 1.5 * floor["max_abs"] + ulp, (what, m, floor)
    return m


def test_c0_fp32_end_to_end(device):
    """Config c0 as BASELINE.json states it, one PISA call in fp32 (B1 H2 D64, 1024 tokens,
    block 64, 25% density): the whole operator on the GPU against the oracle's fp32 pipeline."""
    wl = WORKLOADS["c0"]
    q, k, v = make_inputs(wl, seed=0)
    assert q.dtype == torch.float32
    say(f"[any] c0 fp32: {wl.heads} heads x {wl.seq_len} tokens, D {wl.head_dim}, block {wl.block_size}")
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    o = ops.pisa_pg_attention(qd, kd, vd, density=wl.density, block_size=wl.block_size, scale=wl.op_scale)
    assert o.dtype == torch.float32
    st = ops.block_stats(qd, kd, vd, wl.block_size, 32)
    sel = ops.select_blocks(st, wl.density, wl.op_scale)
    # the GPU's selection: the attention stage alone
    ref_sel = O.pisa_pg_attention(q, k, v, wl.density, wl.block_size, 32, wl.op_scale, indices=sel.idx.cpu())
    check(o.cpu(), ref_sel, "c0 fp32 (GPU selection)", torch.float32)
    # the oracle's own pipeline: at c0 the selections agree, so the whole operator meets the bound
    ref, aux = O.pisa_pg_attention(q, k, v, wl.density, wl.block_size, 32, wl.op_scale, return_aux=True)
    same = torch.equal(torch.sort(aux["idx"].reshape(sel.idx.shape), -1).values,
                       torch.sort(sel.idx.cpu(), -1).values)
    say(f"[any] c0 fp32: selection equal to the oracle's: {same}")
    assert same
    check(o.cpu(), ref, "c0 fp32 (end to end)", torch.float32)


STAT_CASES = [  # heads, T, D, BT, G, dtype
    (2, 1024, 64, 64, 32, torch.float32),
    (1, 1000, 96, 32, 16, torch.bfloat16),
    (2, 777, 128, 256, 4, torch.float16),
    (1, 500, 48, 16, 7, torch.float32),
    (1, 2100, 128, 128, 64, torch.bfloat16),
]


@pytest.mark.parametrize("heads,T,D,BT,G,dtype", STAT_CASES)
def test_block_stats_any(device, heads, T, D, BT, G, dtype):
    q, k, v = inputs(heads, T, D, dtype, seed=T + D)
    say(f"[any K2] heads={heads} T={T} D={D} BT={BT} G={G} {dtype}")
    st = ops.block_stats(q.to(device), k.to(device), v.to(device), BT, G)
    ref = O.block_stats(*(t.reshape(heads, T, D) for t in (q, k, v)), BT, dtype=torch.float64)
    hg = O.group_moment(ref.hc, G)
    for name, got, exp, rtol in (("qc", st.qc, ref.qc, 2e-5), ("kc", st.kc, ref.kc, 2e-5), ("vc", st.vc, ref.vc, 2e-5),
                                 ("hnorm", st.hnorm, ref.hnorm, 1e-4), ("hgroup", st.hgroup, hg, 1e-4)):
        got = got.cpu().double().reshape(exp.shape)
        tol = rtol * float(exp.abs().max()) + 1e-6
        err = float((got - exp).abs().max())
        say(f"[any K2]   {name}: max err {err:.3e} (tol {tol:.3e})")
        assert err <= tol, name


ATTN_CASES = [  # heads, T, D, BT, G, density, dtype, gamma, text, text_valid
    (2, 1024, 64, 64, 32, 0.25, torch.float32, "literal", 0, None),
    (1, 3000, 128, 128, 16, 0.15, torch.bfloat16, "literal", 0, None),     # group size 16
    (2, 1500, 80, 32, 8, 0.2, torch.bfloat16, "consistent", 0, None),      # D 80, block 32
    (1, 2000, 64, 256, 4, 0.3, torch.float16, "literal", 100, 37),         # block 256, text + padding
    (2, 900, 128, 16, 64, 0.1, torch.float32, "literal", 60, None),        # block 16, fp32 text
    (1, 2600, 128, 128, 64, 0.1, torch.bfloat16, "literal", 0, None),      # group size 64
    (1, 1200, 96, 64, 32, 0.25, torch.float32, "consistent", 0, None),
    (2, 1100, 64, 64, 32, 0.2, torch.bfloat16, "literal", 50, 20),         # a text segment at head_dim 64
]


@pytest.mark.parametrize("heads,T,D,BT,G,density,dtype,gamma,text,valid", ATTN_CASES)
def test_sparse_attn_any_shared_selection(device, heads, T, D, BT, G, density, dtype, gamma, text, valid):
    """The any-shape K4 on the GPU's own statistics and selection against the oracle's
    attention stage on that selection."""
    q, k, v = inputs(heads, T, D, dtype, seed=7 * T + BT, text=text)
    say(f"[any K4] heads={heads} T={T} D={D} BT={BT} G={G} density={density} {dtype} {gamma} text={text} "
        f"valid={valid}")
    assert not ops.tuned_shape(dtype, D, BT, G, text)
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    scale = D ** -0.5
    st = ops.block_stats(qd, kd, vd, BT, G, text_tokens=text)
    sel = ops.select_blocks(st, density, scale)
    o = ops.sparse_attn(qd, kd, vd, st, sel, scale, BT, gamma, text_tokens=text, text_valid=valid, group_size=G)
    assert o.dtype == dtype
    kw = dict(gamma=gamma, indices=sel.idx.cpu(), text_tokens=text, text_valid=valid)
    ref = O.pisa_pg_attention(q, k, v, density, BT, G, scale, **kw)
    floor = None
    if dtype != torch.float32:
        rp = O.pisa_pg_attention(q, k, v, density, BT, G, scale, ref_precision=dtype, **kw)
        floor = O.parity_metrics(rp, ref, dtype)
    check(o.cpu(), ref, f"K4 T={T} D={D} BT={BT} G={G} {dtype}", dtype, floor)
    # the allocation-free entry takes the same route and gives the same bits
    o2 = ops.sparse_attn_noalloc(qd, kd, vd, st, sel, scale, BT, gamma, text_tokens=text, text_valid=valid,
                                 group_size=G)
    torch.cuda.synchronize()
    assert torch.equal(o.view(torch.uint8), o2.view(torch.uint8))


@pytest.mark.parametrize("G,BT,dtype", [(16, 64, torch.bfloat16), (8, 128, torch.float16), (32, 64, torch.float32)])
def test_operator_any_group_block_dtype(device, G, BT, dtype):
    """pisa_pg_attention itself with a group size, block size or dtype the tuned kernels do not
    take (reference :307-318 signature), at the Wan2.1-1.3B grid on one head: run-to-run
    bitwise determinism, and the oracle's attention stage on the GPU selection."""
    wl = small_workload(WORKLOADS["c1"], heads=1, grid=(7, 30, 52), block_size=BT, density=0.15)
    q, k, v = make_inputs(wl, seed=3, dtype=dtype)
    say(f"[any op] T={wl.seq_len} G={G} BT={BT} {dtype}")
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    o = ops.pisa_pg_attention(qd, kd, vd, density=wl.density, block_size=BT, group_size=G, scale=wl.op_scale)
    o2 = ops.pisa_pg_attention(qd, kd, vd, density=wl.density, block_size=BT, group_size=G, scale=wl.op_scale)
    assert torch.equal(o.view(torch.uint8), o2.view(torch.uint8)), "run-to-run bitwise determinism"
    st = ops.block_stats(qd, kd, vd, BT, G)
    sel = ops.select_blocks(st, wl.density, wl.op_scale)
    ref = O.pisa_pg_attention(q, k, v, wl.density, BT, G, wl.op_scale, indices=sel.idx.cpu())
    floor = None
    if dtype != torch.float32:
        rp = O.pisa_pg_attention(q, k, v, wl.density, BT, G, wl.op_scale, indices=sel.idx.cpu(),
                                 ref_precision=dtype)
        floor = O.parity_metrics(rp, ref, dtype)
    check(o.cpu(), ref, f"operator G={G} BT={BT} {dtype}", dtype, floor)


@pytest.mark.parametrize("heads,T,D,dtype,text,valid", [(2, 700, 64, torch.float32, 0, None),
                                                        (1, 1000, 128, torch.float32, 100, 37),
                                                        (2, 600, 96, torch.bfloat16, 40, 40)])
def test_dense_attention_any(device, heads, T, D, dtype, text, valid):
    """Dense attention (the processors' warm-up layers) for fp32 or a head dim other than 128:
    softmax(scale q k^T) v in fp64, block-diagonal over the text segments."""
    g = torch.Generator().manual_seed(T + D)
    q, k, v = (torch.randn(1, heads, T, D, generator=g).to(dtype) for _ in range(3))
    o = ops.dense_attention(q.to(device), k.to(device), v.to(device), text_tokens=text, text_valid=valid).cpu()
    assert o.dtype == dtype
    es = O.effective_scale(D ** -0.5)
    seg = T - text + (text if valid is None else valid)
    qd, kd, vd = q.double(), k.double(), v.double()
    ref = torch.empty(1, heads, T, D, dtype=torch.float64)
    ref[..., :seg, :] = O.dense_attention(qd[..., :seg, :], kd[..., :seg, :], vd[..., :seg, :], es)
    if seg < T:
        ref[..., seg:, :] = O.dense_attention(qd[..., seg:, :], kd[..., seg:, :], vd[..., seg:, :], es)
    floor = None
    if dtype != torch.float32:
        rp = O.pisa_pg_attention(q.float(), k.float(), v.float(), 1.0, 64, 32, D ** -0.5, ref_precision=dtype,
                                 text_tokens=text, text_valid=valid)
        floor = O.parity_metrics(rp, ref, dtype)
    check(o, ref, f"dense T={T} D={D} {dtype} text={text}", dtype, floor)
