"""CPU oracle for the PISA-PG hot path — TEST INFRASTRUCTURE ONLY.

This module restates the reference's algorithm on the CPU (torch, fp32 or fp64)
so that the gfx950 kernels can be checked against it.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it, and only as the checker or the timed CPU baseline: the product path
(``pasa_amd``) never imports or calls anything here.

Each function cites the reference file:line it restates.  Paths are relative to
the reference tree (ZHANGWENTAI/PASA):
  group_pisa_attention.py = svg/kernels/triton/group_pisa_attention.py
  placement.py            = svg/models/hyvideo/placement.py

How each part is pinned (tests/test_oracle_*.py):
  permutation  - the reference's reshape/transpose closed form, bijectivity,
                 round trip, fixed context tail;
  block stats  - brute-force per-token loops on tiny inputs (ragged last block);
  group moment - explicit loop with zero padding and division by G;
  top-k        - brute-force stable sort on (-score, index), constructed ties,
                 -0.0 == +0.0, NS from Python's int();
  attention    - the sequential reference loop (``pisa_pg_attention_loop``)
                 against the closed form (``pisa_pg_attention``), density = 1
                 == softmax attention, constant blocks == softmax attention,
                 key-shift invariance, value-shift equivariance (consistent
                 Gamma), G = 1 == brute-force first-order Taylor, O(eps^2)
                 convergence of the first-order term;
  rounding     - bf16_ulp / f16_ulp against the spacing of adjacent representable
                 values, and the reference-precision emulation: outputs
                 representable in the requested type, equal to the unrounded
                 oracle to within that type's rounding.
Every function above has at least one such check: none is "parity unpinned".
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

LOG2E = 1.44269504  # the constant the reference multiplies by (group_pisa_attention.py:162)


# ----------------------------------------------------------------------------
# K1: layout permutation (placement.py:6-31, kernel branches :73-100, :320-343)
# ----------------------------------------------------------------------------

def permute_index(seq_len: int, num_frame: int, frame_size: int, context_length: int,
                  inverse: bool) -> np.ndarray:
    """src_row[dst_row] of the permutation, as an int64 array of length seq_len.

    Forward (frame -> token major): source t = f*P + p goes to p*F + f
    (placement.py:74-78); inverse: source t = p*F + f goes to f*P + p (:321-325);
    rows t >= seq_len - context_length stay in place."""
    F, P = num_frame, frame_size
    assert seq_len == context_length + F * P
    r = np.arange(seq_len, dtype=np.int64)
    src = r.copy()
    body = r < seq_len - context_length
    rb = r[body]
    if not inverse:
        p, f = rb // F, rb % F
        src[body] = f * P + p
    else:
        f, p = rb // P, rb % P
        src[body] = p * F + f
    return src


def permute(x: np.ndarray, num_frame: int, frame_size: int, context_length: int = 0,
            inverse: bool = False, head_is_temporal: Optional[np.ndarray] = None) -> np.ndarray:
    """Apply the permutation along axis 2 of a [B, H, S, D] array (any dtype)."""
    B, H, S, D = x.shape
    src = permute_index(S, num_frame, frame_size, context_length, inverse)
    out = x[:, :, src, :].copy()
    if head_is_temporal is not None:
        keep = np.asarray(head_is_temporal).reshape(B, H) == 0
        out[keep] = x[keep]
    return out


# ----------------------------------------------------------------------------
# K2: block statistics (group_pisa_attention.py:86-129, 268-288) and the group
# moment (:291-301)
# ----------------------------------------------------------------------------

@dataclass
class Stats:
    qc: torch.Tensor      # [BH, NT, D]  block mean of q
    kc: torch.Tensor      # [BH, NT, D]  block mean of k
    vc: torch.Tensor      # [BH, NT, D]  block SUM of v
    hc: torch.Tensor      # [BH, NT, D, D]  H_j = sum_t (k_t - kc_j) v_t^T
    hnorm: torch.Tensor   # [BH, NT]  ||H_j||_F
    n: torch.Tensor       # [NT]  block lengths


def _pad_blocks(x: torch.Tensor, bt: int) -> torch.Tensor:
    BH, T, D = x.shape
    nt = math.ceil(T / bt)
    pad = nt * bt - T
    if pad:
        x = torch.cat([x, x.new_zeros(BH, pad, D)], dim=1)
    return x.reshape(BH, nt, bt, D)


def block_lengths(seq_len: int, block_size: int) -> torch.Tensor:
    """n_j = block_size except the last block: T - (NT-1)*BT (:91, :191, :219-220)."""
    nt = math.ceil(seq_len / block_size)
    n = torch.full((nt,), float(block_size), dtype=torch.float64)
    n[-1] = seq_len - (nt - 1) * block_size
    return n


def block_stats(q, k, v, block_size: int, dtype=torch.float32) -> Stats:
    """q, k, v: [BH, T, D] (any float dtype; computed in ``dtype``)."""
    q, k, v = (t.to(dtype) for t in (q, k, v))
    BH, T, D = q.shape
    n = block_lengths(T, block_size).to(dtype)
    qb, kb, vb = (_pad_blocks(t, block_size) for t in (q, k, v))
    qc = qb.sum(2) / n[None, :, None]          # :101
    kc = kb.sum(2) / n[None, :, None]          # :102
    vc = vb.sum(2)                             # :103
    hc = torch.einsum("bjtd,bjte->bjde", kb, vb) - kc[..., :, None] * vc[..., None, :]  # :106-107
    hnorm = (hc * hc).sum((-1, -2)).sqrt()     # :110, sqrt at :287
    return Stats(qc, kc, vc, hc, hnorm, n)


def group_moment(hc: torch.Tensor, group_size: int) -> torch.Tensor:
    """hbar_g = (1/G) sum_{j in g} H_j, last group zero-padded (:291-301). -> [BH, NG, D, D]"""
    BH, NT, D, E = hc.shape
    ng = math.ceil(NT / group_size)
    pad = ng * group_size - NT
    if pad:
        hc = torch.cat([hc, hc.new_zeros(BH, pad, D, E)], dim=1)
    return hc.reshape(BH, ng, group_size, D, E).mean(2)


# ----------------------------------------------------------------------------
# K3: selection (group_pisa_attention.py:365-375)
# ----------------------------------------------------------------------------

def num_selected(density: float, num_blocks: int) -> int:
    """top_k = min(max(1, int(density * NT)), NT) in Python double (:373)."""
    return min(max(1, int(density * num_blocks)), num_blocks)


def select_scores(qc, kc, hnorm, scale: float, use_cov_bias: bool = True,
                  noise: Optional[torch.Tensor] = None) -> torch.Tensor:
    """score[I, j] = qc_I . (scale * kc_j) + log(hnorm_j + 1e-6) [+ noise_j] (:365-371)."""
    score = torch.matmul(qc, (kc * scale).transpose(-1, -2))
    if use_cov_bias:
        log_bias = torch.log(hnorm + 1e-6)
        if noise is not None:
            log_bias = log_bias + noise.to(log_bias.dtype)
        score = score + log_bias.unsqueeze(-2)
    return score


def topk_indices(scores: torch.Tensor, ns: int) -> torch.Tensor:
    """Indices of the ns largest scores per row, ordered (score desc, index asc).

    torch.topk (:374) leaves tie order unspecified; the rule fixed here (lowest
    index first; -0.0 == +0.0) is the one the gfx950 kernel implements."""
    s = scores.to(torch.float64) + 0.0   # -0.0 + 0.0 == +0.0
    order = torch.sort(s, dim=-1, descending=True, stable=True).indices
    return order[..., :ns].to(torch.int32).contiguous()


def selection_mask(idx: torch.Tensor, num_blocks: int) -> np.ndarray:
    """uint32 words [.., ceil(NT/32)]: bit b of word w set iff block 32w+b selected."""
    nw = (num_blocks + 31) // 32
    flat = idx.reshape(-1, idx.shape[-1]).numpy()
    out = np.zeros((flat.shape[0], nw), dtype=np.uint32)
    for r in range(flat.shape[0]):
        for j in flat[r]:
            out[r, j >> 5] |= np.uint32(1) << np.uint32(j & 31)
    return out.reshape(*idx.shape[:-1], nw)


# ----------------------------------------------------------------------------
# K4: attention, closed form (group_pisa_attention.py:154-262)
# ----------------------------------------------------------------------------

def _rounding(ref_precision):
    """The storage rounding ``ref_precision`` asks for: False -> none, True -> bf16, a
    torch dtype (bfloat16 or float16) -> that type (the reference rounds to its input
    dtype: `p.to(v.dtype)`, stats stored like q)."""
    if ref_precision is False or ref_precision is None:
        return lambda x: x
    dt = torch.bfloat16 if ref_precision is True else ref_precision
    assert dt in (torch.bfloat16, torch.float16), dt
    return lambda x: x.to(dt).to(x.dtype)


def _attention_one(q, k, v, kc, vc, hgroup, idx, n, block_size, group_size, scale, gamma,
                   chunk, ref_precision=False, xk=None, xv=None):
    """One slice.  q,k,v [T,D]; kc,vc [NT,D]; hgroup [NG,D,D]; idx [NT,NS].

    xk, xv: optional [X, D] extra keys/values attended exactly by every query
    block, after its selected blocks (the text segment of ``text_tokens``).

    ref_precision: round where the reference's kernels round (its bf16 storage of
    kc/vc (group_pisa_attention.py:275-277) and of h_group at its use (:251), P and
    P-bar cast to bf16 before their dot products (:185, :240), the bf16 output
    store (:262)), giving the error floor of the reference's own precision."""
    T, D = q.shape
    NT, NS = idx.shape
    NG = hgroup.shape[0]
    bt = block_size
    c = scale * LOG2E
    dt = q.dtype
    qb = _pad_blocks(q[None], bt)[0]                     # [NT, BT, D]
    kb = _pad_blocks(k[None], bt)[0]
    vb = _pad_blocks(v[None], bt)[0]
    keyvalid = (torch.arange(NT * bt) < T).reshape(NT, bt)
    out = torch.empty(NT, bt, D, dtype=dt)
    # zero-order block index -> group, padded to NG*G
    npad = NG * group_size - NT
    nlen = n.to(dt)
    rnd = _rounding(ref_precision)
    kc, vc, hgroup = rnd(kc), rnd(vc), rnd(hgroup)
    for i0 in range(0, NT, chunk):
        i1 = min(NT, i0 + chunk)
        Q = qb[i0:i1]                                    # [m, BT, D]
        sel = idx[i0:i1].long()                          # [m, NS]
        m = i1 - i0
        Ks = kb[sel].reshape(m, NS * bt, D)
        Vs = vb[sel].reshape(m, NS * bt, D)
        kv = keyvalid[sel].reshape(m, 1, NS * bt)
        if xk is not None:
            Ks = torch.cat([Ks, xk[None].expand(m, -1, -1)], dim=1)
            Vs = torch.cat([Vs, xv[None].expand(m, -1, -1)], dim=1)
            kv = torch.cat([kv, kv.new_ones(m, 1, xk.shape[0])], dim=2)
        x = c * torch.matmul(Q, Ks.transpose(1, 2))      # :177
        x = x.masked_fill(~kv, float("-inf"))            # :178
        m1 = x.amax(-1)                                  # [m, BT]
        # phase 2 scores on block means
        xb = c * torch.matmul(Q, kc.T)                   # [m, BT, NT]  :216-217
        selmask = torch.zeros(m, NT, dtype=torch.bool)
        selmask.scatter_(1, sel, True)
        xb = xb.masked_fill(selmask[:, None, :], float("-inf"))     # :223-229
        if npad:
            xb = torch.cat([xb, xb.new_full((m, bt, npad), float("-inf"))], dim=-1)
        xg = xb.reshape(m, bt, NG, group_size)
        gmax = xg.amax(-1)                               # [m, BT, NG]
        run = torch.cummax(torch.maximum(gmax, m1[..., None]), dim=-1).values   # running max m_g
        mf = run[..., -1]                                # final max
        pe = torch.exp2(x - mf[..., None])
        L = pe.sum(-1)
        A = torch.matmul(rnd(pe), Vs)                    # exact part :184-185
        pb = torch.exp2(xg - mf[..., None, None])        # relative to the final max
        pbf = pb.reshape(m, bt, NG * group_size)[..., :NT]
        A = A + torch.matmul(rnd(pbf), vc)               # zero order :239-240
        wsum = pb.sum(-1)                                # [m, BT, NG]  :252
        r = torch.einsum("mtd,gde->mtge", Q, hgroup)     # Q . hbar_g :251
        A = A + scale * torch.einsum("mtg,mtge->mte", wsum, r)   # first order :253
        nl = nlen
        if npad:
            nl = torch.cat([nl, nl.new_zeros(npad)])
        nl = nl.reshape(NG, group_size)
        if gamma == "literal":                           # :201, :242-243, never rescaled
            pg = torch.exp2(xg - run[..., None])
        else:
            pg = pb
        Gam = (pg * nl[None, None]).sum((-1, -2))
        out[i0:i1] = rnd(A / (L + Gam)[..., None])       # :258-259, store :262
    return out.reshape(NT * bt, D)[:T]


def pisa_pg_attention(q, k, v, density: float = 0.15, block_size: int = 64, group_size: int = 32,
                      scale: Optional[float] = None, use_cov_bias: bool = True,
                      noise: Optional[torch.Tensor] = None, gamma: str = "literal",
                      indices: Optional[torch.Tensor] = None, dtype=torch.float32,
                      chunk: int = 32, return_aux: bool = False, ref_precision: bool = False,
                      text_tokens: int = 0, text_valid: Optional[int] = None):
    """Reference PISA-PG output (:307-398) on the CPU.

    q, k, v: [B, H, T, D] (any float dtype, computed in ``dtype``).
    noise: [B, H, NT] per-key-block selection noise (the reference's use_random).
    indices: optional [B, H, NT, NS] selection to use instead of computing it
    (isolates the attention stage from score rounding).
    gamma: 'literal' (reference: Gamma never rescaled) or 'consistent'.
    ref_precision: emulate the reference's roundings in the attention stage (the
    selection stays fp32); see _attention_one.  True rounds to bf16; a dtype
    (torch.bfloat16 or torch.float16) rounds to that type, the reference's rounding
    for inputs of that dtype.
    text_tokens: the last ``text_tokens`` rows form a text segment (HunyuanVideo puts
    its text tokens last, svg/models/hyvideo/attention.py:308-310; the reference
    documents the intent at group_pisa_attention.py:317, 330-333 but runs PISA over
    text as ordinary tokens, which is text_tokens=0).  Blocks, statistics, selection
    and the correction cover the video rows only; every video query block also
    attends to all text keys exactly, and text query rows attend densely to all keys.
    text_valid: the first text_valid text tokens are real, the rest padding (HunyuanVideo
    pads its prompt; its dense path attends block-diagonally over cu_seqlens
    [0, Tv + text_valid, T], svg/models/hyvideo/attention.py:315-323).  Video rows then
    take exact keys only from the valid text rows, valid text rows attend densely to
    [0, Tv + text_valid) and padding rows to the padding segment [Tv + text_valid, T)."""
    B, H, T, D = q.shape
    scale = D ** -0.5 if scale is None else scale
    BH = B * H
    Tv = T - text_tokens
    assert 0 <= text_tokens < T
    tval = text_tokens if text_valid is None else text_valid
    assert 0 <= tval <= text_tokens
    seg = Tv + tval
    q3, k3, v3 = (t.reshape(BH, T, D).to(dtype) for t in (q, k, v))
    if text_tokens:
        full = (q3, k3, v3)
        q3, k3, v3 = (t[:, :Tv] for t in full)
    st = block_stats(q3, k3, v3, block_size, dtype)
    hgroup = group_moment(st.hc, group_size)
    NT = st.qc.shape[1]
    scores = None
    if indices is None:
        ns = num_selected(density, NT)
        nz = None if noise is None else noise.reshape(BH, NT).to(dtype)
        scores = select_scores(st.qc, st.kc, st.hnorm, scale, use_cov_bias, nz)
        idx = topk_indices(scores, ns)
    else:
        idx = indices.reshape(BH, NT, -1).to(torch.int32)
    out = torch.empty(BH, T, D, dtype=dtype)
    for b in range(BH):
        xk = xv = None
        if tval:
            xk, xv = full[1][b, Tv:seg], full[2][b, Tv:seg]
        out[b, :Tv] = _attention_one(q3[b], k3[b], v3[b], st.kc[b], st.vc[b], hgroup[b], idx[b], st.n,
                                     block_size, group_size, scale, gamma, chunk, ref_precision, xk, xv)
        # dense text rows, in the same base-2 arithmetic: each segment attends to itself
        for r0, r1, k0, k1 in ((Tv, seg, 0, seg), (seg, T, seg, T)):
            if r1 <= r0:
                continue
            x = (scale * LOG2E) * torch.matmul(full[0][b, r0:r1], full[1][b, k0:k1].T)
            p = torch.exp2(x - x.amax(-1, keepdim=True))
            # ref_precision: P cast to bf16 before the P.V product, as the exact phase
            # does (:185) and as flash attention does on the reference's dense path; the
            # row sum stays fp32 (:184)
            rnd = _rounding(ref_precision)
            o = torch.matmul(rnd(p), full[2][b, k0:k1]) / p.sum(-1, keepdim=True)
            out[b, r0:r1] = rnd(o)
    out = out.reshape(B, H, T, D)
    if return_aux:
        return out, dict(stats=st, hgroup=hgroup, scores=scores, idx=idx)
    return out


# ----------------------------------------------------------------------------
# K4: the sequential reference loop, for small inputs (group_pisa_attention.py:154-262)
# ----------------------------------------------------------------------------

def pisa_pg_attention_loop(q, k, v, idx, block_size: int, group_size: int, scale: float,
                           gamma: str = "literal", dtype=torch.float64, text_tokens: int = 0,
                           text_valid: Optional[int] = None):
    """Literal restatement of pisa_pg_fwd_kernel's loops for one slice.

    q, k, v [T, D]; idx [NT, NS].  Phase 1 walks idx in order (:170-186); phase 2
    walks groups in order with the O(NS) selection re-test (:212-253); Gamma is
    rescaled only when gamma == 'consistent'.  Intended for tiny inputs.
    text_tokens: the last rows are text: phase 1 of each video row then walks the
    (valid) text keys one by one; text rows run one online-softmax pass over every key
    of their segment (see pisa_pg_attention's text_valid)."""
    q, k, v = (t.to(dtype) for t in (q, k, v))
    T_all = q.shape[0]
    tval = text_tokens if text_valid is None else text_valid
    if text_tokens:
        qt, kt, vt = q[-text_tokens:], k[-text_tokens:], v[-text_tokens:]
        kall, vall = k, v
        q, k, v = q[:-text_tokens], k[:-text_tokens], v[:-text_tokens]
    T, D = q.shape
    bt = block_size
    NT = math.ceil(T / bt)
    st = block_stats(q[None], k[None], v[None], bt, dtype)
    kc, vc = st.kc[0], st.vc[0]
    hg = group_moment(st.hc, group_size)[0]
    c = scale * LOG2E
    last_len = T - (NT - 1) * bt
    out = torch.zeros(T, D, dtype=dtype)
    for I in range(NT):
        rows = range(I * bt, min(T, (I + 1) * bt))
        for i in rows:
            qi = q[i]
            acc = torch.zeros(D, dtype=dtype)
            l = torch.tensor(0.0, dtype=dtype)
            m = torch.tensor(float("-inf"), dtype=dtype)
            for j in idx[I].tolist():                      # Phase 1
                ks = range(j * bt, min(T, (j + 1) * bt))
                s = torch.stack([c * (qi @ k[t]) for t in ks])
                new_m = torch.maximum(m, s.max())
                alpha = torch.exp2(m - new_m)
                p = torch.exp2(s - new_m)
                l = l * alpha + p.sum()
                acc = acc * alpha + sum(p[u] * v[t] for u, t in enumerate(ks))
                m = new_m
            for t in range(tval):                          # valid text keys, exact
                s_t = c * (qi @ kt[t])
                new_m = torch.maximum(m, s_t)
                alpha = torch.exp2(m - new_m)
                p_t = torch.exp2(s_t - new_m)
                l = l * alpha + p_t
                acc = acc * alpha + p_t * vt[t]
                m = new_m
            g_l = torch.tensor(0.0, dtype=dtype)
            sel = set(idx[I].tolist())
            for start in range(0, NT, group_size):         # Phase 2
                g = start // group_size
                members = [j for j in range(start, start + group_size) if j < NT and j not in sel]
                if not members:
                    s_max = torch.tensor(float("-inf"), dtype=dtype)
                else:
                    xs = torch.stack([c * (qi @ kc[j]) for j in members])
                    s_max = xs.max()
                new_m = torch.maximum(m, s_max)
                alpha = torch.exp2(m - new_m)
                acc = acc * alpha
                l = l * alpha
                if gamma != "literal":
                    g_l = g_l * alpha
                m = new_m
                if not members:
                    continue
                p = torch.exp2(xs - m)
                for u, j in enumerate(members):
                    acc = acc + p[u] * vc[j]
                    g_l = g_l + p[u] * (last_len if j == NT - 1 else bt)
                acc = acc + (qi @ hg[g]) * (p.sum() * scale)
            out[i] = acc / (l + g_l)
    if text_tokens:
        out = torch.cat([out, torch.zeros(text_tokens, D, dtype=dtype)])
        for i in range(text_tokens):
            acc = torch.zeros(D, dtype=dtype)
            l = torch.tensor(0.0, dtype=dtype)
            m = torch.tensor(float("-inf"), dtype=dtype)
            keys = range(0, T + tval) if i < tval else range(T + tval, T_all)
            for t in keys:
                s_t = c * (qt[i] @ kall[t])
                new_m = torch.maximum(m, s_t)
                alpha = torch.exp2(m - new_m)
                p_t = torch.exp2(s_t - new_m)
                l = l * alpha + p_t
                acc = acc * alpha + p_t * vall[t]
                m = new_m
            out[T + i] = acc / l
    return out


def effective_scale(scale: float) -> float:
    """Natural-log temperature of the reference's base-2 softmax: exp2(scale*1.44269504*x)
    = exp(scale*1.44269504*ln2*x); the truncated log2(e) differs from 1/ln2 by ~6e-10."""
    return scale * LOG2E * math.log(2.0)


def dense_attention(q, k, v, scale: float, dtype=torch.float64) -> torch.Tensor:
    """softmax(scale * q k^T) v — the closed form several invariants reduce to."""
    q, k, v = (t.to(dtype) for t in (q, k, v))
    w = torch.softmax(scale * torch.matmul(q, k.transpose(-1, -2)), dim=-1)
    return torch.matmul(w, v)


# ----------------------------------------------------------------------------
# Parity metrics (north_star tolerance)
# ----------------------------------------------------------------------------

def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |x| (8 significant bits): 2^(floor(log2|x|) - 7)."""
    ax = x.abs().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(ax)) - 7)


def f16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of fp16 numbers at |x| (11 significant bits, subnormal spacing 2^-24 below
    2^-14): 2^(max(floor(log2|x|), -14) - 10)."""
    ax = x.abs().clamp_min(2.0 ** -14)
    return torch.exp2(torch.floor(torch.log2(ax)) - 10)


def ulp(x: torch.Tensor, dtype=torch.bfloat16) -> torch.Tensor:
    """Spacing of ``dtype`` (bfloat16 or float16) numbers at |x|."""
    return f16_ulp(x) if dtype == torch.float16 else bf16_ulp(x)


def parity_metrics(out: torch.Tensor, ref: torch.Tensor, dtype=torch.bfloat16) -> dict:
    """Agreement of ``out`` with the fp32 reference ``ref``.

    cos, max_abs and max_abs_over_rms are the north_star figures.  ``excess_over_rms``
    is max(|err| - ulp(|ref|)) / RMS(ref): the error left after allowing one ulp of
    the output type ``dtype`` (bf16 or fp16) at each reference element, the quantum of
    any result stored in it (the reference stores P and its output in the input
    dtype).  ``bound_ok`` is cos >= 0.999 and excess_over_rms <= 2e-2."""
    a = out.detach().to(torch.float64).reshape(-1).cpu()
    b = ref.detach().to(torch.float64).reshape(-1).cpu()
    cos = float(torch.dot(a, b) / (a.norm() * b.norm()).clamp_min(1e-300))
    e = (a - b).abs()
    err = float(e.max())
    rms = float(b.pow(2).mean().sqrt())
    excess = float((e - ulp(b, dtype)).clamp_min(0).max())
    return dict(cos=cos, max_abs=err, rms=rms, max_abs_over_rms=err / max(rms, 1e-300),
                excess_over_rms=excess / max(rms, 1e-300),
                bound_ok=bool(cos >= 0.999 and excess <= 2e-2 * rms))
