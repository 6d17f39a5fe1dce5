"""GPU parity of the gfx950 kernels against the CPU oracle (run with -m gpu).

K1 (permutation) and K3's top-k are compared bit-exactly; K2 statistics and K3
scores to fp32 tolerance.  K4 and the whole op are compared with the oracle's fp32
evaluation of the same bf16 inputs:
  * cosine >= 0.999 (north_star);
  * max|err| <= 2e-2 * RMS(ref) after allowing one bf16 ulp of each reference
    element.  The north_star's plain max|err| <= 2e-2 * RMS cannot hold for bf16
    outputs here: the outputs are heavy-tailed (max|o| ~ 50 x RMS), so the bf16
    rounding of the largest elements alone is ~0.2 x RMS.  The plain figure is
    printed for every case;
  * K4's error is at most 1.5x (+ one ulp) that of the oracle run at the
    reference's own precision (bf16 P, kc/vc/h_group and output), i.e. the
    kernel adds no error beyond what the reference's design has.  Where that
    reference-precision error itself exceeds the 2e-2 * RMS excess bound (the
    HunyuanVideo shape), the excess bound becomes 1.5x the floor's.
End to end, GPU and CPU fp32 scores differ in the last ulp, so a query block may
pick a different block at an exact or near tie; the test proves every such
difference is a near tie and checks the other query blocks elementwise."""
import dataclasses
import math
import os
import sys

import numpy as np
import pytest
import torch

from oracle import pisa_oracle as O
from pasa_amd import _lib, ops, placement
from pasa_amd.workloads import WORKLOADS, Workload, make_inputs, small_workload

pytestmark = pytest.mark.gpu

COS_MIN = 0.999
EXCESS_OVER_RMS = 2e-2


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def check_parity(out, ref, what, floor=None, dtype=torch.bfloat16):
    """cos >= 0.999, and the error beyond one ulp of the output type ``dtype`` (bf16 or
    fp16) <= 2e-2 * RMS.  With ``floor`` (the metrics of the reference-precision oracle
    against the same fp32 reference): max|err| <= 1.5 x the floor's + one ulp, and the
    excess bound is max(2e-2, 1.5 x the floor's excess) * RMS -- where the reference's own
    roundings already exceed 2e-2 * RMS beyond one ulp (at the HunyuanVideo shape,
    near-zero outputs that come from cancelling sums), the kernel is held to that floor
    instead."""
    m = O.parity_metrics(out, ref, dtype)
    say(f"[parity] {what}: cos={m['cos']:.7f} max_abs/rms={m['max_abs_over_rms']:.3e} "
        f"excess/rms={m['excess_over_rms']:.3e}"
        + ("" if floor is None else f" floor max_abs/rms={floor['max_abs_over_rms']:.3e} "
                                    f"floor excess/rms={floor['excess_over_rms']:.3e}"))
    assert m["cos"] >= COS_MIN, (what, m)
    bound = EXCESS_OVER_RMS if floor is None else max(EXCESS_OVER_RMS, 1.5 * floor["excess_over_rms"])
    assert m["excess_over_rms"] <= bound, (what, m, floor)
    if floor is not None:
        ulp = float(O.ulp(torch.tensor(ref.abs().max().item()), dtype))
        assert m["max_abs"] <= 1.5 * floor["max_abs"] + ulp, (what, m, floor)
    return m


def test_native_library_loaded(device):
    lib = _lib.load()
    assert lib.pasa_abi_version() == _lib.ABI_VERSION
    maps = open("/proc/self/maps").read()
    assert str(_lib.LIB_PATH) in maps


# ---------------------------------------------------------------- K1 --------

def random_bits(shape, device, dtype=torch.bfloat16, seed=0):
    g = torch.Generator(device=device).manual_seed(seed)
    if dtype == torch.float32:
        return torch.randint(-2**31, 2**31 - 1, shape, device=device, dtype=torch.int32, generator=g).view(torch.float32)
    return torch.randint(-2**15, 2**15 - 1, shape, device=device, dtype=torch.int16, generator=g).view(dtype)


def as_np_bits(t):
    return t.cpu().view(torch.int32 if t.dtype == torch.float32 else torch.int16).numpy()


@pytest.mark.parametrize("B,H,F,P,ctx,D,dtype", [
    (1, 12, 21, 1560, 0, 128, torch.bfloat16),      # c1: 21 frames x 30*52 patches
    (2, 4, 11, 4080, 226, 64, torch.bfloat16),      # the reference self-test shape (placement.py:189-197), 4 heads
    (1, 3, 33, 3600, 256, 128, torch.bfloat16),     # HunyuanVideo 720p layout with text tail, 3 heads
    (1, 2, 5, 7, 3, 64, torch.float32),
])
def test_permute_bit_exact(device, B, H, F, P, ctx, D, dtype):
    S = ctx + F * P
    say(f"[K1] B={B} H={H} F={F} P={P} ctx={ctx} D={D} {dtype}")
    src = [random_bits((B, H, S, D), device, dtype, seed=i) for i in range(3)]
    dst = [torch.empty_like(t) for t in src]
    placement.permute(src, dst, F, P, ctx, inverse=False)
    for s, d in zip(src, dst):
        np.testing.assert_array_equal(as_np_bits(d), O.permute(as_np_bits(s), F, P, ctx, inverse=False))
    back = torch.empty_like(src[0])
    placement.permute([dst[0]], [back], F, P, ctx, inverse=True)
    assert torch.equal(back.view(torch.int16 if dtype != torch.float32 else torch.int32),
                       src[0].view(torch.int16 if dtype != torch.float32 else torch.int32))
    inv = torch.empty_like(src[1])
    placement.permute([src[1]], [inv], F, P, ctx, inverse=True)
    np.testing.assert_array_equal(as_np_bits(inv), O.permute(as_np_bits(src[1]), F, P, ctx, inverse=True))


def test_reference_placement_api_with_head_mask(device):
    ctx, F, P, B, H, D = 226, 11, 408, 2, 6, 64
    S = ctx + F * P
    say("[K1] hunyuan_sparse_head_placement / hidden_states_placement with best_mask_idx")
    q, k, v = (random_bits((B, H, S, D), device, seed=10 + i) for i in range(3))
    mask = torch.tensor([[1, 0, 1, 1, 0, 0], [0, 1, 1, 0, 1, 0]], device=device)
    qo, ko, vo = (torch.empty_like(t) for t in (q, k, v))
    placement.hunyuan_sparse_head_placement(q, k, v, qo, ko, vo, mask, ctx, F, P)
    m = mask.cpu().numpy()
    for s, d in ((q, qo), (k, ko), (v, vo)):
        np.testing.assert_array_equal(as_np_bits(d), O.permute(as_np_bits(s), F, P, ctx, head_is_temporal=m))
    ho = torch.empty_like(qo)
    placement.hunyuan_hidden_states_placement(qo, ho, mask, ctx, F, P)
    assert torch.equal(ho.view(torch.int16), q.view(torch.int16))
    t = q.clone()
    placement.hunyuan_token_reorder_to_token_major(t, ctx, F * P, F, P)
    np.testing.assert_array_equal(as_np_bits(t), O.permute(as_np_bits(q), F, P, ctx))
    placement.hunyuan_token_reorder_to_frame_major(t, ctx, F * P, F, P)
    assert torch.equal(t.view(torch.int16), q.view(torch.int16))


# ---------------------------------------------------------------- K2 --------

STAT_CASES = [
    # (heads, grid, D, BT)
    (2, (4, 16, 16), 64, 64),        # c0 shape
    (2, (3, 10, 20), 128, 128),      # T = 600: ragged last block (88 rows)
    (3, (5, 13, 17), 64, 128),       # T = 1105, NT = 9
    (1, (21, 30, 52), 128, 128),     # c1 shape, one head: NT = 256, 8 groups
    (1, (9, 45, 80), 128, 64),       # NT = 507: 16 groups, last one partial
]


def bf16_inputs(heads, grid, D, BT, seed=0, density=0.15):
    wl = Workload("t", heads=heads, head_dim=D, grid=grid, block_size=BT, density=density,
                  prescale=D ** -0.5 / 128 ** -0.5 if D != 128 else 1.0)
    return wl, make_inputs(wl, seed=seed, dtype=torch.bfloat16)


@pytest.mark.parametrize("heads,grid,D,BT", STAT_CASES)
def test_block_stats(device, heads, grid, D, BT):
    wl, (q, k, v) = bf16_inputs(heads, grid, D, BT)
    say(f"[K2] heads={heads} T={wl.seq_len} D={D} BT={BT}")
    st = ops.block_stats(q.to(device), k.to(device), v.to(device), BT, 32)
    T = wl.seq_len
    ref = O.block_stats(*(t.reshape(heads, T, D) for t in (q, k, v)), BT, dtype=torch.float64)
    hg = O.group_moment(ref.hc, 32)
    def close(got, exp, name, rtol=2e-5):
        got = got.cpu().double().reshape(exp.shape)
        tol = rtol * float(exp.abs().max()) + 1e-6
        err = float((got - exp).abs().max())
        say(f"[K2]   {name}: max err {err:.3e} (tol {tol:.3e})")
        assert err <= tol, name
    close(st.qc, ref.qc, "qc")
    close(st.kc, ref.kc, "kc")
    close(st.vc, ref.vc, "vc")
    close(st.hnorm, ref.hnorm, "hnorm", 1e-4)
    close(st.hgroup, hg, "hgroup", 1e-4)


@pytest.mark.parametrize("heads,T,BT", [(12, 32760, 128), (2, 5000, 128), (3, 9000, 64), (1, 1100, 128)])
def test_block_stats_split_matches_unsplit(device, heads, T, BT):
    """Small grids split each group over several workgroups: the per-block statistics
    are the same computation (bit-identical), the group moment differs only in the order
    of its sum.  (2, 5000, 128) ends in a partial group of 8 blocks."""
    from pasa_amd import _lib
    need = _lib.load().pasa_block_stats_workspace_bytes(heads, T, 0, 128, BT, 32)
    assert need > 0, "shape chosen to split"
    g = torch.Generator().manual_seed(T)
    q, k, v = (torch.randn(1, heads, T, 128, generator=g).to(device, torch.bfloat16) for _ in range(3))
    say(f"[K2 split] heads={heads} T={T} BT={BT} workspace={need >> 20} MiB")
    a = ops.block_stats(q, k, v, BT, 32, split=True)
    b = ops.block_stats(q, k, v, BT, 32, split=False)
    for name in ("qc", "kc", "vc", "hnorm"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name
    d = float((a.hgroup - b.hgroup).abs().max())
    scale = float(b.hgroup.abs().max())
    say(f"[K2 split]   hgroup max |split - unsplit| {d:.3e} of max {scale:.3e}")
    assert d <= 1e-5 * scale
    assert torch.equal(a.hgroup, ops.block_stats(q, k, v, BT, 32, split=True).hgroup)   # deterministic


# ---------------------------------------------------------------- K3 --------

@pytest.mark.parametrize("NT,ns", [(16, 4), (100, 15), (591, 59), (929, 92), (1024, 1), (4096, 409), (3, 3)])
def test_select_from_scores_bit_exact(device, NT, ns):
    say(f"[K3] select_from_scores NT={NT} ns={ns}")
    g = torch.Generator().manual_seed(NT)
    BH = 3
    s = torch.randn(1, BH, NT, NT, generator=g)
    s[0, 0] = torch.round(s[0, 0] * 2) / 2            # heavy ties
    s[0, 1, :, ::3] = 0.0
    s[0, 1, :, 1::3] = -0.0                           # -0.0 ties with +0.0
    s[0, 2, 0] = 1.0                                  # an all-equal row
    sel = ops.select_from_scores(s.to(device), ns)
    want = O.topk_indices(s, ns)
    np.testing.assert_array_equal(sel.idx.cpu().numpy(), want.numpy())
    np.testing.assert_array_equal(sel.selmask.cpu().numpy().view(np.uint32), O.selection_mask(want, NT))


@pytest.mark.parametrize("NT,ns,BH", [(4097, 410, 2), (5000, 1, 1), (6000, 6000, 1), (9000, 8192, 1)])
def test_select_from_scores_long_rows_bit_exact(device, NT, ns, BH):
    """Rows of more than 4096 blocks take the radix select over the row in memory: the same
    rule (score desc, index asc; -0.0 == +0.0) on constructed ties, bit-exact."""
    say(f"[K3] select_from_scores (long rows) NT={NT} ns={ns} BH={BH}")
    g = torch.Generator().manual_seed(NT + ns)
    s = torch.randn(1, BH, NT, NT, generator=g)
    s[0, 0] = torch.round(s[0, 0] * 4) / 4            # heavy ties at every rank
    s[0, 0, 1, ::2] = 0.0
    s[0, 0, 1, 1::2] = -0.0                           # -0.0 ties with +0.0
    s[0, 0, 2] = 1.0                                  # an all-equal row
    sel = ops.select_from_scores(s.to(device), ns)
    rows = list(range(0, NT, max(1, NT // 300))) + [1, 2, NT - 1]   # the oracle on a sample of rows
    sub = s[:, :, rows]
    want = O.topk_indices(sub, ns)
    np.testing.assert_array_equal(sel.idx.cpu()[:, :, rows].numpy(), want.numpy())
    np.testing.assert_array_equal(sel.selmask.cpu()[:, :, rows].numpy().view(np.uint32), O.selection_mask(want, NT))
    # the bitmask alone (the attention call's form) equals the one written with the indices
    m2 = torch.empty_like(sel.selmask)
    _lib.call("pasa_select_from_scores", s.to(device).data_ptr(), ns, None, m2.data_ptr(), BH, NT,
              torch.cuda.current_stream().cuda_stream)
    assert torch.equal(m2, sel.selmask)


@pytest.mark.parametrize("heads,grid,D,BT,density,use_noise", [
    (2, (4, 16, 16), 64, 64, 0.25, False),
    (2, (21, 30, 52), 128, 128, 0.15, True),
    (1, (21, 45, 80), 128, 128, 0.10, False),
])
def test_select(device, heads, grid, D, BT, density, use_noise):
    wl, (q, k, v) = bf16_inputs(heads, grid, D, BT)
    say(f"[K3] select heads={heads} T={wl.seq_len} density={density} noise={use_noise}")
    st = ops.block_stats(q.to(device), k.to(device), v.to(device), BT, 32)
    NT = st.qc.shape[2]
    noise = torch.randn(1, heads, NT, generator=torch.Generator().manual_seed(3)) if use_noise else None
    scale = D ** -0.5
    sel = ops.select_blocks(st, density, scale, True, None if noise is None else noise.to(device),
                            return_scores=True)
    ref = O.select_scores(st.qc.cpu().double(), st.kc.cpu().double(), st.hnorm.cpu().double(), scale,
                          True, None if noise is None else noise.double())
    got = sel.scores.cpu().double()
    err = float((got - ref).abs().max())
    say(f"[K3]   score max err {err:.3e}")
    assert err <= 1e-5 * float(ref.abs().max()) + 1e-5
    want = O.topk_indices(sel.scores.cpu(), sel.ns)
    np.testing.assert_array_equal(sel.idx.cpu().numpy(), want.numpy())


@pytest.mark.parametrize("heads,grid,BT,density", [
    (2, (4, 16, 16), 64, 0.25),       # NS 4: one register of keys
    (1, (21, 45, 80), 64, 0.10),      # c2 at block 64: NT 1182, NS 118
    (1, (33, 45, 80), 128, 0.10),     # c3 video rows: NT 929, NS 92
])
def test_select_without_indices(device, heads, grid, BT, density):
    """idx = NULL skips the index list: the bitmask is the one the full call writes, and
    K4 computes the same output bit for bit from it."""
    D = 128
    wl, (q, k, v) = bf16_inputs(heads, grid, D, BT)
    say(f"[K3] select without indices heads={heads} T={wl.seq_len} BT={BT}")
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    st = ops.block_stats(qd, kd, vd, BT, 32)
    scale = D ** -0.5
    full = ops.select_blocks(st, density, scale)
    bare = ops.select_blocks(st, density, scale, indices=False)
    assert bare.idx is None
    assert torch.equal(bare.selmask, full.selmask)
    o_full = ops.sparse_attn(qd, kd, vd, st, full, scale, BT)
    o_bare = ops.sparse_attn(qd, kd, vd, st, bare, scale, BT)
    assert torch.equal(o_full.view(torch.int16), o_bare.view(torch.int16))


# ---------------------------------------------------------------- K4 --------

ATTN_CASES = [
    # heads, grid, D, BT, density, gamma
    (2, (4, 16, 16), 64, 64, 0.25, "literal"),      # c0 shape in bf16
    (2, (3, 10, 20), 128, 128, 0.4, "literal"),     # ragged last block
    (2, (3, 10, 20), 128, 128, 0.4, "consistent"),
    (2, (5, 13, 17), 64, 128, 0.3, "literal"),
    (1, (9, 45, 80), 128, 64, 0.1, "literal"),      # BT 64, NT 507: query-block pairs, the last one a repeat
    (2, (3, 10, 20), 128, 64, 0.4, "consistent"),   # BT 64 pairs, NT 10, ragged last block
    (1, (1, 5, 11), 128, 64, 0.5, "literal"),       # BT 64, NT 1: one pair, its second block a repeat
    (2, (21, 30, 52), 128, 128, 0.15, "literal"),   # c1 shape, 2 heads
]


@pytest.mark.parametrize("heads,grid,D,BT,density,gamma", ATTN_CASES)
def test_sparse_attn_shared_selection(device, heads, grid, D, BT, density, gamma):
    wl, (q, k, v) = bf16_inputs(heads, grid, D, BT, seed=1)
    say(f"[K4] heads={heads} T={wl.seq_len} D={D} BT={BT} density={density} gamma={gamma}")
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    scale = D ** -0.5
    st = ops.block_stats(qd, kd, vd, BT, 32)
    sel = ops.select_blocks(st, density, scale)
    o = ops.sparse_attn(qd, kd, vd, st, sel, scale, BT, gamma)
    idx = sel.idx.cpu()
    ref = O.pisa_pg_attention(q, k, v, density, BT, 32, scale, gamma=gamma, indices=idx)
    rp = O.pisa_pg_attention(q, k, v, density, BT, 32, scale, gamma=gamma, indices=idx, ref_precision=True)
    floor = O.parity_metrics(rp, ref)
    check_parity(o.cpu(), ref, f"K4 {wl.seq_len}x{D} BT{BT} {gamma}", floor)


def test_pair_rows_with_unequal_tile_counts(device):
    """BT 64 runs two query blocks per workgroup in lock step.  Rows of a pair with
    different numbers of selected blocks (never written by pasa_select, whose rows all
    hold NS bits) still give each block its own result: odd blocks here drop their
    lowest-scoring selection."""
    heads, grid, D, BT, density = 2, (3, 10, 20), 128, 64, 0.4
    wl, (q, k, v) = bf16_inputs(heads, grid, D, BT, seed=3)
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    scale = D ** -0.5
    st = ops.block_stats(qd, kd, vd, BT, 32)
    sel = ops.select_blocks(st, density, scale)
    NT, NS = st.qc.shape[2], sel.ns
    assert NS >= 2
    idx = sel.idx.cpu()
    short = idx[..., :NS - 1].contiguous()
    m_full = O.selection_mask(idx, NT)
    m_short = O.selection_mask(short, NT)
    mask = m_full.copy()
    mask[..., 1::2, :] = m_short[..., 1::2, :]
    say(f"[K4] unequal pair rows: heads={heads} NT={NT} NS={NS} (odd blocks NS-1)")
    sel2 = ops.Selection(idx=sel.idx, selmask=torch.from_numpy(mask.view(np.int32)).to(device), scores=None,
                         ns=NS)
    o = ops.sparse_attn(qd, kd, vd, st, sel2, scale, BT, "literal").cpu()
    ref_full = O.pisa_pg_attention(q, k, v, density, BT, 32, scale, indices=idx)
    ref_short = O.pisa_pg_attention(q, k, v, density, BT, 32, scale, indices=short)
    T = wl.seq_len
    odd_rows = ((torch.arange(T) // BT) % 2 == 1)[None, None, :, None]
    ref = torch.where(odd_rows, ref_short, ref_full)
    check_parity(o, ref, "K4 BT64 pairs with unequal rows")


def test_full_density_equals_dense_attention(device):
    wl, (q, k, v) = bf16_inputs(2, (3, 10, 20), 128, 128, seed=2)
    say("[K4] density 1.0 vs softmax attention")
    o = ops.pisa_pg_attention(q.to(device), k.to(device), v.to(device), density=1.0, block_size=128)
    ref = O.dense_attention(q.double(), k.double(), v.double(), O.effective_scale(128 ** -0.5))
    check_parity(o.cpu(), ref, "density=1")


def fp32_gamma(n):
    """Higham's gamma_n for fp32: any order of n rounded fp32 operations (products and
    sums) on a dot product is within gamma_n * sum|a_i b_i| of the exact value."""
    u = 2.0 ** -24
    return n * u / (1 - n * u)


def score_error_bound(qc, kc, hnorm, scale, noise=None):
    """Exact selection scores and a bound on how far any fp32 evaluation of them can be.

    qc, kc: fp32 [NT, D] and hnorm fp32 [NT] as K2 wrote them (K3 reads exactly these).
    K3 forms fl(scale * kc) first (as the reference does), then the fp32 dot product
    with qc in some order (error <= gamma_{D+1} * sum_d |qc_d * skc_d|, products
    included), then fl(logf(fl(h + 1e-6))) (the add's relative rounding 2^-24 moves
    the log by at most 2^-24 after division by h + 1e-6; logf itself is within 2 ulp of
    its result; 4 ulp are allowed), then the bias add(s) (half an ulp of |score| each).  The exact score
    is computed in fp64 from the same fp32 inputs.  Returns (exact [NT, NT], bound
    [NT, NT])."""
    D = qc.shape[-1]
    skc = (kc.float() * float(scale)).double()           # fl(scale * kc), exactly as K3 rounds it
    q64 = qc.double()
    dot = q64 @ skc.T
    dot_abs = q64.abs() @ skc.abs().T
    hp = (hnorm.float() + 1e-6).double()                  # fl(h + 1e-6)
    lb = torch.log(hp)
    exact = dot + lb[None, :]
    n_adds = 1
    if noise is not None:
        exact = exact + noise.double()[None, :]
        n_adds = 2

    def ulp32(x):
        return torch.exp2(torch.floor(torch.log2(x.abs().clamp_min(2.0 ** -126))) - 23)

    log_err = 2.0 ** -22 + 4 * ulp32(lb)
    bound = fp32_gamma(D + 1) * dot_abs + log_err[None, :] + n_adds * 0.5 * ulp32(exact.abs() + dot_abs)
    return exact, bound


def check_selection_near_ties(st_gpu, gpu_idx, scale, ns, heads, noise=None, what=""):
    """The GPU selection of each tested head equals the top-ns of the exact scores of
    the GPU's own block statistics, except at near ties.  If the GPU keeps block j and
    drops block i that the exact ranking keeps, its fp32 scores put j at or above i, so
    exact_i - exact_j <= bound_i + bound_j must hold for every such pair."""
    n_differ, n_rows = 0, 0
    for i, h in enumerate(heads):
        qc, kc, hn = (t[0, h].cpu() for t in (st_gpu.qc, st_gpu.kc, st_gpu.hnorm))
        nz = None if noise is None else noise[0, h].cpu()
        exact, bound = score_error_bound(qc, kc, hn, scale, nz)
        order = torch.sort(exact, dim=-1, descending=True, stable=True)
        gi = gpu_idx[0, i].long()
        for I in range(exact.shape[0]):
            mine = set(gi[I].tolist())
            ref = set(order.indices[I, :ns].tolist())
            n_rows += 1
            if mine == ref:
                continue
            n_differ += 1
            for j in mine - ref:
                for r in ref - mine:
                    gap = float(exact[I, r] - exact[I, j])
                    lim = float(bound[I, r] + bound[I, j])
                    assert gap <= lim, (what, h, I, j, r, gap, lim)
    say(f"[sel] {what}: {n_differ} of {n_rows} query blocks differ from the exact-score top-{ns}, "
        f"all within the fp32 rounding bound of a tie")


def check_end_to_end(o, q, k, v, wl, st_gpu, gpu_idx, heads, noise=None, what="", text_valid=None,
                     gamma="literal"):
    """Whole-op parity on the slices ``heads`` of the GPU run (q, k, v, o and gpu_idx
    hold those slices only; st_gpu the full GPU statistics):
      1. the GPU selection is the exact top-k of its statistics up to rounding near ties;
      2. with the GPU's selection, the output meets the north_star bound against the
         fp32 oracle on every row, and stays within 1.5x (+ one ulp) of the error the
         reference's own bf16 roundings give (the ref_precision oracle);
      3. against the oracle's own pipeline (its statistics and selection): cosine over all
         rows, and the excess bound on every row whose selection is the same."""
    kw = dict(text_tokens=wl.text_tokens, text_valid=text_valid, gamma=gamma)
    H, NT, ns = q.shape[1], wl.num_blocks(), gpu_idx.shape[-1]
    nz = None if noise is None else noise[:, list(heads)]
    check_selection_near_ties(st_gpu, gpu_idx, wl.op_scale, ns, heads, noise, what)
    ref_sel = O.pisa_pg_attention(q, k, v, wl.density, wl.block_size, 32, wl.op_scale, indices=gpu_idx, **kw)
    rp = O.pisa_pg_attention(q, k, v, wl.density, wl.block_size, 32, wl.op_scale, indices=gpu_idx,
                             ref_precision=True, **kw)
    floor = O.parity_metrics(rp, ref_sel)
    m_sel = check_parity(o.cpu(), ref_sel, what + " (GPU selection)", floor)
    ref, aux = O.pisa_pg_attention(q, k, v, wl.density, wl.block_size, 32, wl.op_scale, noise=nz,
                                   return_aux=True, **kw)
    oidx = aux["idx"].reshape(1, H, NT, -1)
    differ = (torch.sort(oidx, -1).values != torch.sort(gpu_idx, -1).values).any(-1)   # [1, H, NT]
    m = O.parity_metrics(o.cpu(), ref)
    say(f"[E2E] {what} vs the oracle's own pipeline: {int(differ.sum())} of {H * NT} query blocks select "
        f"differently; cos={m['cos']:.7f} max_abs/rms={m['max_abs_over_rms']:.3e}")
    assert m["cos"] >= COS_MIN
    keep = (~differ).repeat_interleave(wl.block_size, -1)[..., : wl.video_tokens]   # [1, H, Tv]
    keep = torch.cat([keep, keep.new_ones(*keep.shape[:-1], wl.text_tokens)], -1)  # text rows: dense
    rms = float(ref.double().pow(2).mean().sqrt())
    e = (o.cpu().double() - ref.double()).abs()
    excess = float(((e - O.bf16_ulp(ref.double())).clamp_min(0)).amax(-1)[keep].max())
    say(f"[E2E] {what} rows with identical selection: excess/rms={excess / rms:.3e}")
    assert excess <= max(EXCESS_OVER_RMS, 1.5 * floor["excess_over_rms"]) * rms
    return dict(m_sel, floor_max_abs_over_rms=floor["max_abs_over_rms"],
                kernel_over_floor=m_sel["max_abs"] / floor["max_abs"])


def test_end_to_end_c1_two_heads_with_noise(device):
    wl = small_workload(WORKLOADS["c1"], heads=2, grid=WORKLOADS["c1"].grid)
    q, k, v = make_inputs(wl, seed=0)
    say(f"[E2E] c1 shape, 2 heads, T={wl.seq_len}, use_random noise")
    NT = wl.num_blocks()
    noise = torch.randn(1, 2, NT, generator=torch.Generator().manual_seed(5))
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    st = ops.block_stats(qd, kd, vd, wl.block_size, 32)
    sel = ops.select_blocks(st, wl.density, wl.op_scale, True, noise.to(device))
    o = ops.pisa_pg_attention(qd, kd, vd, density=wl.density, block_size=wl.block_size,
                              scale=wl.op_scale, use_random=True, noise=noise.to(device))
    check_end_to_end(o, q, k, v, wl, st, sel.idx.cpu(), (0, 1), noise, "c1 end-to-end")


def test_end_to_end_c2_full_shape(device):
    wl = WORKLOADS["c2"]
    say(f"[E2E] c2 full shape: {wl.heads} heads x {wl.seq_len} tokens (oracle on heads 0 and 39)")
    q, k, v = make_inputs(wl, seed=0)
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    o = ops.pisa_pg_attention(qd, kd, vd, density=wl.density, block_size=wl.block_size, scale=wl.op_scale)
    o2 = ops.pisa_pg_attention(qd, kd, vd, density=wl.density, block_size=wl.block_size, scale=wl.op_scale)
    assert torch.equal(o.view(torch.int16), o2.view(torch.int16)), "run-to-run bitwise determinism"
    st = ops.block_stats(qd, kd, vd, wl.block_size, 32)
    idx = ops.select_blocks(st, wl.density, wl.op_scale).idx.cpu()
    oc = o.cpu()
    for h in (0, wl.heads - 1):
        sl = slice(h, h + 1)
        r = check_end_to_end(oc[:, sl], q[:, sl], k[:, sl], v[:, sl], wl, st, idx[:, sl], (h,), None,
                             f"c2 head {h}")
        say(f"[E2E] c2 head {h}: kernel/floor max-abs ratio {r['kernel_over_floor']:.3f}")
        assert r["kernel_over_floor"] <= 1.5


def run_heads(wl, heads, device, text_valid=None):
    """The GPU op on the given heads of a workload (heads are independent slices, so this
    equals running every head and keeping these), with its statistics and selection."""
    q, k, v = make_inputs(wl, seed=0, heads=heads)
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    o = ops.pisa_pg_attention(qd, kd, vd, density=wl.density, block_size=wl.block_size, scale=wl.op_scale,
                              text_tokens=wl.text_tokens, text_valid=text_valid)
    st = ops.block_stats(qd, kd, vd, wl.block_size, 32, text_tokens=wl.text_tokens)
    idx = ops.select_blocks(st, wl.density, wl.op_scale).idx.cpu()
    return q, k, v, o, st, idx


def test_end_to_end_c3_full_shape_two_heads(device):
    wl = WORKLOADS["c3"]
    heads = range(0, wl.heads, wl.heads - 1)        # the first and the last head
    say(f"[E2E] c3 full shape: heads {list(heads)} of {wl.heads}, {wl.video_tokens} video + {wl.text_tokens} text "
        f"tokens, NT {wl.num_blocks()}")
    q, k, v, o, st, idx = run_heads(wl, heads, device)
    r = check_end_to_end(o, q, k, v, wl, st, idx, (0, 1), None, "c3 full shape")
    say(f"[E2E] c3: kernel/floor max-abs ratio {r['kernel_over_floor']:.3f}")
    assert r["kernel_over_floor"] <= 1.5


@pytest.mark.parametrize("name,text_valid", [("c2", None), ("c3", None), ("c3", 141)])
def test_end_to_end_block64_first_and_last_head(device, name, text_valid):
    """Block size 64, the processors' default (query blocks run in pairs), at the full c2 and
    c3 shapes as bench.py times them (``c2_block64``, ``c3_block64``): the first and the last
    head.  With text_valid 141 of the 256 text rows are the prompt (three prompt tiles, an
    odd count, so one pair holds the last prompt tile and the first padding tile)."""
    wl = dataclasses.replace(WORKLOADS[name], block_size=64)
    heads = (0, wl.heads - 1)
    say(f"[E2E] {name} shape at block 64, heads {heads}: {wl.video_tokens} video + {wl.text_tokens} text tokens "
        f"(valid {text_valid}), NT {wl.num_blocks()}")
    q, k, v, o, st, idx = run_heads(wl, heads, device, text_valid)
    r = check_end_to_end(o, q, k, v, wl, st, idx, (0, 1), None, f"{name} block 64", text_valid=text_valid)
    say(f"[E2E] {name} block 64: kernel/floor max-abs ratio {r['kernel_over_floor']:.3f}")
    assert r["kernel_over_floor"] <= 1.5


def test_end_to_end_more_than_4096_blocks(device):
    """A sequence of 4200 key blocks (268,800 tokens at block size 64, one head, density 0.02):
    the radix-select top-k feeds the tuned attention kernel; checked end to end like c2."""
    base = WORKLOADS["c2"]
    wl = dataclasses.replace(base, heads=1, grid=(4, 140, 480), block_size=64, density=0.02)
    assert wl.num_blocks() == 4200
    say(f"[E2E] long sequence: T={wl.seq_len}, NT {wl.num_blocks()}, NS {ops.num_selected(wl.density, 4200)}")
    q, k, v, o, st, idx = run_heads(wl, range(0, 1), device)
    r = check_end_to_end(o, q, k, v, wl, st, idx, (0,), None, "4200 blocks")
    assert r["kernel_over_floor"] <= 1.5


def test_end_to_end_c2_fp16_one_head(device):
    """fp16 q, k, v end to end at the c2 shape (bench.py's ``c2_fp16``), head 0: the GPU
    selection is the exact top-k up to near ties, and the output meets the bound against
    the fp32 oracle on that selection, within 1.5x (+ one fp16 ulp) of the oracle run at
    the reference's roundings in fp16."""
    wl = dataclasses.replace(WORKLOADS["c2"], dtype=torch.float16)
    say(f"[E2E] c2 fp16, head 0: T={wl.seq_len}, NT {wl.num_blocks()}")
    q, k, v = make_inputs(wl, seed=0, heads=range(0, 1))
    assert q.dtype == torch.float16
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    o = ops.pisa_pg_attention(qd, kd, vd, density=wl.density, block_size=wl.block_size, scale=wl.op_scale)
    assert o.dtype == torch.float16
    st = ops.block_stats(qd, kd, vd, wl.block_size, 32)
    sel = ops.select_blocks(st, wl.density, wl.op_scale)
    idx = sel.idx.cpu()
    check_selection_near_ties(st, idx, wl.op_scale, sel.ns, (0,), None, "c2 fp16")
    ref = O.pisa_pg_attention(q, k, v, wl.density, wl.block_size, 32, wl.op_scale, indices=idx)
    rp = O.pisa_pg_attention(q, k, v, wl.density, wl.block_size, 32, wl.op_scale, indices=idx,
                             ref_precision=torch.float16)
    floor = O.parity_metrics(rp, ref, torch.float16)
    m = check_parity(o.cpu(), ref, "c2 fp16 head 0 (GPU selection)", floor, torch.float16)
    ratio = m["max_abs"] / floor["max_abs"]
    say(f"[E2E] c2 fp16 head 0: kernel/floor max-abs ratio {ratio:.3f}")
    assert ratio <= 1.5


@pytest.mark.parametrize("name,heads", [("c1", None), ("c2", (0, 39))])
def test_placed_route_at_bench_shapes(device, name, heads):
    """The placed call (placement folded into K2/K4) is bit-identical to K1 -> call -> K1
    inverse at the shapes bench.py times both routes: all 12 heads of c1 (F 21, P 1560,
    ``other_configs.c1.with_permutations``) and the first and last head of c2 (F 21,
    P 3600, ``placement_folded``)."""
    wl = WORKLOADS[name]
    hs = range(wl.heads) if heads is None else heads
    F, Hh, W = wl.grid
    P, X = Hh * W, wl.text_tokens
    say(f"[placed] {name}: heads {list(hs)}, F={F} P={P}")
    q, k, v = make_inputs(wl, seed=0, heads=hs, device=device)
    o = ops.pisa_pg_attention(q, k, v, wl.density, block_size=wl.block_size, scale=wl.op_scale, text_tokens=X,
                              placement=ops.Placement(F, P, None))
    bufs = [torch.empty_like(t) for t in (q, k, v)]
    placement.permute([q, k, v], bufs, F, P, X)
    ot = ops.pisa_pg_attention(bufs[0], bufs[1], bufs[2], wl.density, block_size=wl.block_size,
                               scale=wl.op_scale, text_tokens=X)
    ref = torch.empty_like(ot)
    placement.permute([ot], [ref], F, P, X, inverse=True)
    torch.cuda.synchronize()
    assert torch.equal(o.view(torch.int16), ref.view(torch.int16))


# ------------------------------------------------------------ text segment --

TEXT_CASES = [
    # heads, grid, text, BT, density, gamma, prompt rows (None: no padding)
    (2, (3, 10, 20), 40, 128, 0.4, "literal", None),      # last video block 88 rows; one partial text tile
    (1, (5, 13, 17), 256, 64, 0.2, "literal", None),      # BT 64 kernel; four text tiles
    (2, (3, 10, 20), 300, 128, 0.3, "consistent", None),  # three text tiles, the last partial
    (2, (3, 10, 20), 300, 128, 0.3, "literal", 77),       # prompt 1 partial tile, padding 2 tiles
    (2, (3, 10, 20), 256, 128, 0.4, "literal", 128),      # segment edge on a tile edge
    (1, (5, 13, 17), 256, 64, 0.2, "consistent", 200),    # BT 64: 4 prompt tiles, 1 padding tile
    (1, (5, 13, 17), 256, 64, 0.2, "literal", 0),         # all padding: video rows see no text
    (2, (3, 10, 20), 40, 128, 0.4, "literal", 39),        # one padding row
]


def text_inputs(heads, grid, text, BT, density, seed):
    wl = small_workload(WORKLOADS["c3"], heads=heads, grid=grid, block_size=BT, density=density,
                        text_tokens=text, prescale=1.0, scale=None)
    return wl, make_inputs(wl, seed=seed, dtype=torch.bfloat16)


@pytest.mark.parametrize("heads,grid,text,BT,density,gamma,valid", TEXT_CASES)
def test_text_segment_shared_selection(device, heads, grid, text, BT, density, gamma, valid):
    wl, (q, k, v) = text_inputs(heads, grid, text, BT, density, seed=4)
    T, Tv = wl.seq_len, wl.video_tokens
    say(f"[text] heads={heads} Tv={Tv} text={text} valid={valid} BT={BT} density={density} gamma={gamma}")
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    scale = 128 ** -0.5
    st = ops.block_stats(qd, kd, vd, BT, 32, text_tokens=text)
    ref_st = O.block_stats(*(t[0, :, :Tv].double() for t in (q, k, v)), BT, dtype=torch.float64)
    assert st.qc.shape[2] == wl.num_blocks()
    torch.testing.assert_close(st.kc[0].cpu().double(), ref_st.kc, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(st.vc[0].cpu().double(), ref_st.vc, rtol=1e-5, atol=1e-4)
    sel = ops.select_blocks(st, density, scale)
    o = ops.sparse_attn(qd, kd, vd, st, sel, scale, BT, gamma, text_tokens=text, text_valid=valid)
    idx = sel.idx.cpu()
    kw = dict(gamma=gamma, indices=idx, text_tokens=text, text_valid=valid)
    ref = O.pisa_pg_attention(q, k, v, density, BT, 32, scale, **kw)
    rp = O.pisa_pg_attention(q, k, v, density, BT, 32, scale, ref_precision=True, **kw)
    floor = O.parity_metrics(rp, ref)
    check_parity(o.cpu(), ref, f"text {Tv}+{text} valid {valid} BT{BT} {gamma}", floor)
    seg = Tv + (text if valid is None else valid)
    if seg > Tv:
        check_parity(o.cpu()[..., Tv:seg, :], ref[..., Tv:seg, :], "prompt rows (dense)")
    if seg < T:
        check_parity(o.cpu()[..., seg:, :], ref[..., seg:, :], "padding rows (dense)")


def test_text_segment_full_density_equals_dense_attention(device):
    wl, (q, k, v) = text_inputs(2, (3, 10, 20), 100, 128, 1.0, seed=5)
    say("[text] density 1.0 with a text segment vs softmax attention")
    o = ops.pisa_pg_attention(q.to(device), k.to(device), v.to(device), density=1.0, block_size=128,
                              text_tokens=100)
    ref = O.dense_attention(q.double(), k.double(), v.double(), O.effective_scale(128 ** -0.5))
    check_parity(o.cpu(), ref, "text density=1")


def test_text_padding_full_density_is_block_diagonal(device):
    # cu_seqlens [0, seg, T] semantics: two independent dense attentions
    wl, (q, k, v) = text_inputs(2, (3, 10, 20), 100, 128, 1.0, seed=6)
    seg = wl.video_tokens + 37
    say(f"[text] density 1.0, 37 of 100 text rows valid vs two dense attentions (split at {seg})")
    o = ops.pisa_pg_attention(q.to(device), k.to(device), v.to(device), density=1.0, block_size=128,
                              text_tokens=100, text_valid=37).cpu()
    es = O.effective_scale(128 ** -0.5)
    qd, kd, vd = q.double(), k.double(), v.double()
    check_parity(o[..., :seg, :], O.dense_attention(qd[..., :seg, :], kd[..., :seg, :], vd[..., :seg, :], es),
                 "segment [0, seg)")
    check_parity(o[..., seg:, :], O.dense_attention(qd[..., seg:, :], kd[..., seg:, :], vd[..., seg:, :], es),
                 "padding segment")


def test_end_to_end_c3_one_head_text_segment(device):
    wl = small_workload(WORKLOADS["c3"], heads=1, grid=(9, 45, 80))
    say(f"[E2E] c3 layout, 1 head, {wl.video_tokens} video + {wl.text_tokens} text tokens")
    q, k, v, o, st, idx = run_heads(wl, range(0, 1), device)
    check_end_to_end(o, q, k, v, wl, st, idx, (0,), None, "c3 one head")


# ------------------------------------------------------------ dense warm-up --

@pytest.mark.parametrize("heads,T,text,valid", [(2, 600, 0, None), (1, 129, 0, None), (2, 1000, 100, 37),
                                                 (1, 700, 300, 0), (2, 384, 128, 128)])
def test_dense_attention(device, heads, T, text, valid):
    """K4's exact-tile path without selection: softmax attention, block-diagonal with a
    text segment; at the floor set by rounding P to bf16 (the oracle at density 1 with
    the reference's roundings)."""
    say(f"[dense] heads={heads} T={T} text={text} valid={valid}")
    g = torch.Generator().manual_seed(T + text)
    q, k, v = (torch.randn(1, heads, T, 128, generator=g).to(torch.bfloat16) for _ in range(3))
    o = ops.dense_attention(q.to(device), k.to(device), v.to(device), text_tokens=text, text_valid=valid).cpu()
    es = O.effective_scale(128 ** -0.5)
    seg = T - text + (text if valid is None else valid)
    qd, kd, vd = q.double(), k.double(), v.double()
    ref = torch.empty(1, heads, T, 128, dtype=torch.float64)
    ref[..., :seg, :] = O.dense_attention(qd[..., :seg, :], kd[..., :seg, :], vd[..., :seg, :], es)
    if seg < T:
        ref[..., seg:, :] = O.dense_attention(qd[..., seg:, :], kd[..., seg:, :], vd[..., seg:, :], es)
    rp = O.pisa_pg_attention(q.float(), k.float(), v.float(), 1.0, 128, 32, 128 ** -0.5, ref_precision=True,
                             text_tokens=text, text_valid=valid)
    floor = O.parity_metrics(rp, ref)
    check_parity(o, ref, f"dense T={T} text={text} valid={valid}", floor)


def test_processor_dense_split_matches_two_sdpa_calls(device):
    """processors.dense.attention with a cu_seqlens split equals two dense attentions."""
    from pasa_amd.processors import dense as DN
    g = torch.Generator().manual_seed(11)
    q, k, v = (torch.randn(1, 2, 500, 128, generator=g).to(torch.bfloat16).to(device) for _ in range(3))
    o = DN.attention(q, k, v, 421).float().cpu()
    ref = torch.cat([torch.nn.functional.scaled_dot_product_attention(q[:, :, :421].float(), k[:, :, :421].float(),
                                                                       v[:, :, :421].float()),
                     torch.nn.functional.scaled_dot_product_attention(q[:, :, 421:].float(), k[:, :, 421:].float(),
                                                                       v[:, :, 421:].float())], dim=2).cpu()
    check_parity(o, ref.double(), "processor dense split")


# ------------------------------------------------------------------ fp16 ------
# The D = 128 path takes fp16 q, k, v as well: the statistics stay fp32, P, the phase-2
# pack and the output are fp16 (the reference casts P to v's dtype and stores its
# statistics and output in it).  The floor is the oracle at fp16 precision.

def f16_inputs(heads, grid, BT, seed=0, density=0.15, text=0):
    base = WORKLOADS["c3"] if text else WORKLOADS["c1"]
    wl = small_workload(base, heads=heads, grid=grid, block_size=BT, density=density, text_tokens=text,
                        prescale=1.0, scale=None)
    return wl, make_inputs(wl, seed=seed, dtype=torch.float16)


@pytest.mark.parametrize("heads,grid,BT", [(2, (3, 10, 20), 128), (1, (9, 45, 80), 64), (1, (21, 30, 52), 128)])
def test_block_stats_f16(device, heads, grid, BT):
    wl, (q, k, v) = f16_inputs(heads, grid, BT)
    T = wl.seq_len
    say(f"[K2 fp16] heads={heads} T={T} BT={BT}")
    st = ops.block_stats(q.to(device), k.to(device), v.to(device), BT, 32)
    ref = O.block_stats(*(t.reshape(heads, T, 128) for t in (q, k, v)), BT, dtype=torch.float64)
    hg = O.group_moment(ref.hc, 32)
    for name, got, exp, rtol in (("qc", st.qc, ref.qc, 2e-5), ("kc", st.kc, ref.kc, 2e-5), ("vc", st.vc, ref.vc, 2e-5),
                                 ("hnorm", st.hnorm, ref.hnorm, 1e-4), ("hgroup", st.hgroup, hg, 1e-4)):
        got = got.cpu().double().reshape(exp.shape)
        tol = rtol * float(exp.abs().max()) + 1e-6
        err = float((got - exp).abs().max())
        say(f"[K2 fp16]   {name}: max err {err:.3e} (tol {tol:.3e})")
        assert err <= tol, name


@pytest.mark.parametrize("heads,grid,BT,density,gamma,text,valid", [
    (2, (3, 10, 20), 128, 0.4, "literal", 0, None),        # ragged last block
    (1, (9, 45, 80), 64, 0.1, "literal", 0, None),         # block 64: query-block pairs, the last a repeat
    (2, (21, 30, 52), 128, 0.15, "consistent", 0, None),   # c1 shape
    (1, (3, 10, 20), 128, 0.4, "literal", 256, 77),        # text segment with padding
    (1, (3, 10, 20), 64, 0.4, "literal", 40, None),        # text segment at block 64
])
def test_sparse_attn_f16(device, heads, grid, BT, density, gamma, text, valid):
    wl, (q, k, v) = f16_inputs(heads, grid, BT, seed=5, density=density, text=text)
    say(f"[K4 fp16] heads={heads} T={wl.seq_len} text={text} valid={valid} BT={BT} density={density} {gamma}")
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    scale = 128 ** -0.5
    st = ops.block_stats(qd, kd, vd, BT, 32, text_tokens=text)
    sel = ops.select_blocks(st, density, scale)
    o = ops.sparse_attn(qd, kd, vd, st, sel, scale, BT, gamma, text_tokens=text, text_valid=valid)
    assert o.dtype == torch.float16
    kw = dict(gamma=gamma, indices=sel.idx.cpu(), text_tokens=text, text_valid=valid)
    ref = O.pisa_pg_attention(q, k, v, density, BT, 32, scale, **kw)
    rp = O.pisa_pg_attention(q, k, v, density, BT, 32, scale, ref_precision=torch.float16, **kw)
    floor = O.parity_metrics(rp, ref, torch.float16)
    check_parity(o.cpu(), ref, f"K4 fp16 {wl.seq_len}x128 BT{BT} text {text} {gamma}", floor, torch.float16)
    # fp16 carries three more significand bits than bf16: the same selection run on the
    # bf16 roundings of the inputs is further off
    qb, kb, vb = qd.bfloat16(), kd.bfloat16(), vd.bfloat16()
    stb = ops.block_stats(qb, kb, vb, BT, 32, text_tokens=text)
    ob = ops.sparse_attn(qb, kb, vb, stb, sel, scale, BT, gamma, text_tokens=text, text_valid=valid)
    e16 = (o.cpu().double() - ref.double()).abs().max().item()
    e_bf = (ob.cpu().double() - ref.double()).abs().max().item()
    say(f"[K4 fp16]   max err fp16 {e16:.3e}, bf16 {e_bf:.3e}")
    assert e16 < e_bf


def test_dense_attention_f16(device):
    heads, T, text, valid = 2, 1000, 100, 37
    g = torch.Generator().manual_seed(17)
    q, k, v = (torch.randn(1, heads, T, 128, generator=g).to(torch.float16) for _ in range(3))
    o = ops.dense_attention(q.to(device), k.to(device), v.to(device), text_tokens=text, text_valid=valid).cpu()
    assert o.dtype == torch.float16
    es = O.effective_scale(128 ** -0.5)
    seg = T - text + valid
    qd, kd, vd = q.double(), k.double(), v.double()
    ref = torch.empty(1, heads, T, 128, dtype=torch.float64)
    ref[..., :seg, :] = O.dense_attention(qd[..., :seg, :], kd[..., :seg, :], vd[..., :seg, :], es)
    ref[..., seg:, :] = O.dense_attention(qd[..., seg:, :], kd[..., seg:, :], vd[..., seg:, :], es)
    rp = O.pisa_pg_attention(q.float(), k.float(), v.float(), 1.0, 128, 32, 128 ** -0.5,
                             ref_precision=torch.float16, text_tokens=text, text_valid=valid)
    floor = O.parity_metrics(rp, ref, torch.float16)
    check_parity(o, ref, f"dense fp16 T={T} text={text} valid={valid}", floor, torch.float16)


def test_placed_attention_f16_equals_permute_attend_unpermute(device):
    from pasa_amd import placement as PL
    F, P, text, H, D, density = 5, 200, 40, 2, 128, 0.3
    T = F * P + text
    g = torch.Generator().manual_seed(21)
    q, k, v = (torch.randn(1, H, T, D, generator=g).to(torch.float16).to(device) for _ in range(3))
    fl = torch.tensor([[1, 0]], dtype=torch.int32, device=device)
    o = ops.pisa_pg_attention(q, k, v, density, block_size=128, text_tokens=text, placement=ops.Placement(F, P, fl))
    qs, ks, vs = (torch.empty_like(t) for t in (q, k, v))
    PL.hunyuan_sparse_head_placement(q, k, v, qs, ks, vs, fl, text, F, P)
    ot = ops.pisa_pg_attention(qs, ks, vs, density, block_size=128, text_tokens=text)
    ref = torch.empty_like(ot)
    PL.hunyuan_hidden_states_placement(ot, ref, fl, text, F, P)
    torch.cuda.synchronize()
    assert o.dtype == torch.float16 and torch.equal(o, ref)


# ---------------------------------------------------- placement folded in --

@pytest.mark.parametrize("F,P,text,flags,density", [(5, 200, 0, None, 0.3), (7, 131, 40, [1, 0], 0.25),
                                                    (3, 300, 256, [0, 1], 0.4), (4, 257, 13, [1, 1], 0.5)])
def test_placed_attention_equals_permute_attend_unpermute(device, F, P, text, flags, density):
    """The token-major view of frame-major tensors (placement folded into K2 and K4) is
    bit-identical to permuting with K1, attending and permuting back."""
    from pasa_amd import placement as PL
    H, D = 2, 128
    T = F * P + text
    say(f"[placed] F={F} P={P} text={text} flags={flags} density={density}")
    g = torch.Generator().manual_seed(F * 1000 + P)
    q, k, v = (torch.randn(1, H, T, D, generator=g).to(torch.bfloat16).to(device) for _ in range(3))
    fl = None if flags is None else torch.tensor([flags], dtype=torch.int32, device=device)
    o = ops.pisa_pg_attention(q, k, v, density, block_size=128, text_tokens=text,
                              placement=ops.Placement(F, P, fl))
    qs, ks, vs = (torch.empty_like(t) for t in (q, k, v))
    mask = torch.ones(1, H, dtype=torch.int32, device=device) if fl is None else fl
    PL.hunyuan_sparse_head_placement(q, k, v, qs, ks, vs, mask, text, F, P)
    ot = ops.pisa_pg_attention(qs, ks, vs, density, block_size=128, text_tokens=text)
    ref = torch.empty_like(ot)
    PL.hunyuan_hidden_states_placement(ot, ref, mask, text, F, P)
    torch.cuda.synchronize()
    assert torch.equal(o, ref)


HEAD_DIM_CASES = [  # (head dim, dtype, text tokens, block size)
    (96, torch.bfloat16, 0, 64),
    (32, torch.bfloat16, 0, 64),
    (80, torch.bfloat16, 0, 128),
    (64, torch.float16, 0, 64),
    (64, torch.bfloat16, 128, 64),
    (48, torch.float16, 64, 128),
]


@pytest.mark.parametrize("D,dtype,text,BT", HEAD_DIM_CASES)
def test_operator_pads_other_head_dims(device, D, dtype, text, BT):
    """pisa_pg_attention at a head dim the kernels do not take directly (or 64 where the
    call needs the D = 128 kernels: fp16, a text segment) runs zero-padded and returns
    the unpadded math: compared with the oracle at the true head dim, on the selection
    the kernels make for the padded inputs, to the reference-precision floor."""
    wl = Workload("hd", heads=2, head_dim=D, grid=(4, 16, 24), block_size=BT, density=0.2, text_tokens=text,
                  prescale=D ** -0.5 / 128 ** -0.5, dtype=dtype)
    q, k, v = make_inputs(wl, seed=11, dtype=dtype)
    say(f"[head dim] D={D} {dtype} text={text} BT={BT} T={wl.seq_len}")
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    scale = D ** -0.5
    o = ops.pisa_pg_attention(qd, kd, vd, wl.density, block_size=BT, scale=scale, text_tokens=text)
    assert o.shape == q.shape and o.dtype == dtype
    Dk = ops.kernel_head_dim(D, dtype, text)
    assert Dk != D or D == 64
    pad = lambda t: torch.nn.functional.pad(t, (0, Dk - D)).contiguous()
    st = ops.block_stats(pad(qd), pad(kd), pad(vd), BT, 32, text_tokens=text)
    sel = ops.select_blocks(st, wl.density, scale)
    kw = dict(indices=sel.idx.cpu(), text_tokens=text)
    ref = O.pisa_pg_attention(q, k, v, wl.density, BT, 32, scale, **kw)
    rp = O.pisa_pg_attention(q, k, v, wl.density, BT, 32, scale, ref_precision=dtype, **kw)
    check_parity(o.cpu(), ref, f"head dim {D} {dtype} text {text} BT{BT}", O.parity_metrics(rp, ref, dtype), dtype)

