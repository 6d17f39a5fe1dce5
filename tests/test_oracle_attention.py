"""Pins the oracle's PISA-PG attention (reference group_pisa_attention.py:154-262).

Two independent restatements are cross-checked (the vectorised closed form and
the literal sequential loop), and the closed form is tied to mathematics that
fixes it: softmax attention when nothing is approximated, invariances, the
first-order Taylor expansion for G = 1, and O(eps^2) convergence."""
import math

import numpy as np
import pytest
import torch

from oracle import pisa_oracle as O

f64 = torch.float64


def rand_qkv(B, H, T, D, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return tuple(torch.randn(B, H, T, D, generator=g, dtype=f64) * scale for _ in range(3))


@pytest.mark.parametrize("T,bt,G,density,gamma", [
    (96, 16, 2, 0.34, "literal"), (96, 16, 2, 0.34, "consistent"),
    (100, 16, 3, 0.25, "literal"), (70, 8, 4, 0.2, "literal"), (64, 16, 32, 0.25, "literal"),
    (45, 16, 1, 0.5, "literal")])
def test_closed_form_matches_sequential_loop(T, bt, G, density, gamma):
    q, k, v = rand_qkv(1, 2, T, 6, seed=T + bt + G, scale=1.5)
    s = 6 ** -0.5
    out, aux = O.pisa_pg_attention(q, k, v, density, bt, G, s, gamma=gamma, dtype=f64, return_aux=True)
    for b in range(2):
        ref = O.pisa_pg_attention_loop(q[0, b], k[0, b], v[0, b], aux["idx"][b], bt, G, s, gamma)
        torch.testing.assert_close(out[0, b], ref, rtol=1e-10, atol=1e-10)


def test_literal_and_consistent_differ_only_when_phase2_raises_max():
    # A constant key block has H = 0, so its selection score carries log(1e-6) and it
    # stays unselected, while its mean score is large: phase 2 raises the running max.
    q, k, v = rand_qkv(1, 1, 128, 8, seed=1, scale=1.0)
    k = k.clone()
    k[..., 32:48, :] = 4.0 * q[0, 0, :, :].mean(0) / q[0, 0, :, :].mean(0).norm()
    k[..., 80:96, :] = 6.0
    lit = O.pisa_pg_attention(q, k, v, 0.125, 16, 2, 8 ** -0.5, gamma="literal", dtype=f64)
    con = O.pisa_pg_attention(q, k, v, 0.125, 16, 2, 8 ** -0.5, gamma="consistent", dtype=f64)
    assert not torch.allclose(lit, con)
    # with queries/keys constant per block the selection holds the per-row maximum,
    # phase 2 never raises it and the two forms coincide
    qc, kc = const_blocks(q, 16), const_blocks(k, 16)
    lit = O.pisa_pg_attention(qc, kc, v, 0.125, 16, 2, 8 ** -0.5, gamma="literal", dtype=f64)
    con = O.pisa_pg_attention(qc, kc, v, 0.125, 16, 2, 8 ** -0.5, gamma="consistent", dtype=f64)
    torch.testing.assert_close(lit, con, rtol=1e-12, atol=1e-12)


def const_blocks(x, bt):
    B, H, T, D = x.shape
    nt = math.ceil(T / bt)
    xb = torch.cat([x, x.new_zeros(B, H, nt * bt - T, D)], 2).reshape(B, H, nt, bt, D)
    return xb[:, :, :, :1, :].expand(B, H, nt, bt, D).reshape(B, H, nt * bt, D)[:, :, :T].contiguous()


@pytest.mark.parametrize("T,bt", [(128, 16), (100, 16), (64, 64)])
def test_full_density_is_softmax_attention(T, bt):
    q, k, v = rand_qkv(1, 2, T, 8, seed=T, scale=1.2)
    s = 0.4
    out = O.pisa_pg_attention(q, k, v, 1.0, bt, 4, s, dtype=f64)
    torch.testing.assert_close(out, O.dense_attention(q, k, v, O.effective_scale(s)), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("density", [0.1, 0.25, 0.5])
def test_constant_blocks_is_softmax_attention(density):
    # q, k constant per block => H = 0, the selection takes each row's largest
    # block scores, and the zero-order terms are exact.
    q, k, v = rand_qkv(1, 2, 160, 8, seed=7, scale=1.0)
    q, k = const_blocks(q, 16), const_blocks(k, 16)
    s = 8 ** -0.5
    out = O.pisa_pg_attention(q, k, v, density, 16, 4, s, dtype=f64)
    torch.testing.assert_close(out, O.dense_attention(q, k, v, O.effective_scale(s)), rtol=1e-10, atol=1e-10)


def test_key_shift_invariance():
    q, k, v = rand_qkv(1, 2, 112, 8, seed=9)
    delta = torch.randn(8, dtype=f64) * 0.7
    a = O.pisa_pg_attention(q, k, v, 0.3, 16, 2, 0.5, dtype=f64)
    b = O.pisa_pg_attention(q, k + delta, v, 0.3, 16, 2, 0.5, dtype=f64)
    torch.testing.assert_close(a, b, rtol=1e-9, atol=1e-9)


def test_value_shift_equivariance_consistent():
    q, k, v = rand_qkv(1, 2, 112, 8, seed=10)
    delta = torch.randn(8, dtype=f64)
    a = O.pisa_pg_attention(q, k, v, 0.3, 16, 2, 0.5, gamma="consistent", dtype=f64)
    b = O.pisa_pg_attention(q, k, v + delta, 0.3, 16, 2, 0.5, gamma="consistent", dtype=f64)
    torch.testing.assert_close(b, a + delta, rtol=1e-9, atol=1e-9)


def brute_first_order(q, k, v, idx, bt, s):
    """G = 1: exact on selected blocks, e^{s q.kbar}(Vhat + s H^T q) on the others."""
    T, D = q.shape
    nt = math.ceil(T / bt)
    se = O.effective_scale(s)   # exponent temperature; the first-order term keeps s
    out = torch.zeros(T, D, dtype=f64)
    for I in range(nt):
        sel = set(idx[I].tolist())
        for i in range(I * bt, min(T, (I + 1) * bt)):
            num = torch.zeros(D, dtype=f64)
            den = torch.tensor(0.0, dtype=f64)
            for j in range(nt):
                rows = list(range(j * bt, min(T, (j + 1) * bt)))
                if j in sel:
                    for t in rows:
                        w = torch.exp(se * (q[i] @ k[t]))
                        num += w * v[t]
                        den += w
                else:
                    kb = k[rows].mean(0)
                    vh = v[rows].sum(0)
                    Hj = sum(torch.outer(k[t] - kb, v[t]) for t in rows)
                    w = torch.exp(se * (q[i] @ kb))
                    num += w * (vh + s * (Hj.T @ q[i]))
                    den += w * len(rows)
            out[i] = num / den
    return out


def test_group_size_one_is_first_order_taylor():
    q, k, v = rand_qkv(1, 1, 72, 5, seed=12)
    s = 0.45
    out, aux = O.pisa_pg_attention(q, k, v, 0.2, 16, 1, s, gamma="consistent", dtype=f64, return_aux=True)
    ref = brute_first_order(q[0, 0], k[0, 0], v[0, 0], aux["idx"][0], 16, s)
    torch.testing.assert_close(out[0, 0], ref, rtol=1e-10, atol=1e-10)


def test_first_order_error_is_quadratic():
    # keys = block mean + eps * zero-mean perturbation; fixed selection; G = 1.
    g = torch.Generator().manual_seed(13)
    T, D, bt = 96, 6, 16
    nt = T // bt
    q = torch.randn(1, 1, T, D, generator=g, dtype=f64)
    v = torch.randn(1, 1, T, D, generator=g, dtype=f64)
    centres = torch.randn(nt, D, generator=g, dtype=f64).repeat_interleave(bt, 0)
    pert = torch.randn(T, D, generator=g, dtype=f64).reshape(nt, bt, D)
    pert = (pert - pert.mean(1, keepdim=True)).reshape(T, D)
    idx = torch.tensor([[i] for i in range(nt)], dtype=torch.int32)[None, None]
    errs = []
    for eps in (0.2, 0.1, 0.05):
        k = (centres + eps * pert)[None, None]
        approx = O.pisa_pg_attention(q, k, v, block_size=bt, group_size=1, scale=0.5,
                                     gamma="consistent", indices=idx, dtype=f64)
        errs.append(float((approx - O.dense_attention(q, k, v, O.effective_scale(0.5))).abs().max()))
    r1, r2 = errs[0] / errs[1], errs[1] / errs[2]
    assert 3.0 < r1 < 5.0 and 3.3 < r2 < 4.7, errs


def test_explicit_indices_and_noise():
    q, k, v = rand_qkv(1, 1, 96, 8, seed=14)
    out, aux = O.pisa_pg_attention(q, k, v, 0.25, 16, 2, 0.5, dtype=f64, return_aux=True)
    again = O.pisa_pg_attention(q, k, v, block_size=16, group_size=2, scale=0.5,
                                indices=aux["idx"].reshape(1, 1, 6, -1), dtype=f64)
    torch.testing.assert_close(out, again, rtol=0, atol=0)
    noise = torch.randn(1, 1, 6, dtype=f64) * 50  # dominates the score
    _, aux2 = O.pisa_pg_attention(q, k, v, 0.25, 16, 2, 0.5, noise=noise, dtype=f64, return_aux=True)
    top = torch.argsort(noise.reshape(-1), descending=True)[:1]
    assert all(int(row[0]) == int(top[0]) for row in aux2["idx"][0])


def test_parity_metrics():
    a = torch.tensor([1.0, 2.0, 3.0])
    m = O.parity_metrics(a, a)
    assert m["cos"] == pytest.approx(1.0) and m["max_abs"] == 0.0
    m = O.parity_metrics(a + torch.tensor([0.0, 0.0, 0.1]), a)
    assert m["max_abs"] == pytest.approx(0.1, abs=1e-6)


# ------------------------------------------------------------ text segment --

@pytest.mark.parametrize("T,text,bt,G,density,gamma", [
    (100, 12, 16, 2, 0.34, "literal"), (100, 12, 16, 2, 0.34, "consistent"),
    (90, 17, 8, 3, 0.25, "literal"), (64, 40, 16, 1, 0.5, "literal")])
def test_text_segment_closed_form_matches_sequential_loop(T, text, bt, G, density, gamma):
    q, k, v = rand_qkv(1, 2, T, 6, seed=T + text, scale=1.5)
    s = 6 ** -0.5
    out, aux = O.pisa_pg_attention(q, k, v, density, bt, G, s, gamma=gamma, dtype=f64, return_aux=True,
                                   text_tokens=text)
    assert aux["idx"].shape[1] == -(-(T - text) // bt)      # blocks cover the video rows only
    for b in range(2):
        ref = O.pisa_pg_attention_loop(q[0, b], k[0, b], v[0, b], aux["idx"][b], bt, G, s, gamma,
                                       text_tokens=text)
        torch.testing.assert_close(out[0, b], ref, rtol=1e-10, atol=1e-10)


def test_text_segment_full_density_is_softmax_attention():
    q, k, v = rand_qkv(1, 2, 77, 8, seed=5)
    out = O.pisa_pg_attention(q, k, v, 1.0, 16, 2, 8 ** -0.5, dtype=f64, text_tokens=13)
    ref = O.dense_attention(q, k, v, O.effective_scale(8 ** -0.5))
    torch.testing.assert_close(out, ref, rtol=1e-10, atol=1e-10)


def test_text_rows_are_dense_and_video_rows_ignore_text_queries():
    q, k, v = rand_qkv(1, 1, 80, 8, seed=6)
    s = 8 ** -0.5
    out = O.pisa_pg_attention(q, k, v, 0.25, 16, 2, s, dtype=f64, text_tokens=16)
    ref = O.dense_attention(q, k, v, O.effective_scale(s))
    torch.testing.assert_close(out[..., 64:, :], ref[..., 64:, :], rtol=1e-10, atol=1e-10)
    q2 = q.clone()
    q2[..., 64:, :] = torch.randn(16, 8, dtype=f64)           # text queries do not touch video rows
    out2 = O.pisa_pg_attention(q2, k, v, 0.25, 16, 2, s, dtype=f64, text_tokens=16)
    torch.testing.assert_close(out2[..., :64, :], out[..., :64, :], rtol=0, atol=0)


def test_text_segment_with_negligible_text_keys_is_video_only_pisa():
    # Text keys far below every score (exp2 underflows to 0) change nothing for video rows.
    q, k, v = rand_qkv(1, 1, 96, 8, seed=7)
    k = k.clone()
    q = q.clone()
    q[..., :, 0] = q[..., :, 0].abs() + 1.0            # every query has a positive first coordinate
    k[..., 80:, :] = 0.0
    k[..., 80:, 0] = -1e4                              # text keys: q.k <= -1e4
    s = 8 ** -0.5
    out = O.pisa_pg_attention(q, k, v, 0.25, 16, 2, s, dtype=f64, text_tokens=16)
    ref = O.pisa_pg_attention(q[..., :80, :], k[..., :80, :], v[..., :80, :], 0.25, 16, 2, s, dtype=f64)
    torch.testing.assert_close(out[..., :80, :], ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("text,valid", [(12, 5), (17, 0), (20, 20), (33, 30)])
def test_text_padding_closed_form_matches_sequential_loop(text, valid):
    T = 96 + text
    q, k, v = rand_qkv(1, 2, T, 6, seed=text + valid, scale=1.5)
    s = 6 ** -0.5
    out, aux = O.pisa_pg_attention(q, k, v, 0.3, 16, 2, s, dtype=f64, return_aux=True, text_tokens=text,
                                   text_valid=valid)
    for b in range(2):
        ref = O.pisa_pg_attention_loop(q[0, b], k[0, b], v[0, b], aux["idx"][b], 16, 2, s, text_tokens=text,
                                       text_valid=valid)
        torch.testing.assert_close(out[0, b], ref, rtol=1e-10, atol=1e-10)


def test_text_padding_is_block_diagonal_for_text_rows():
    # Text rows reduce to dense attention within their segment; video rows ignore padding keys.
    q, k, v = rand_qkv(1, 1, 110, 8, seed=9)
    s = 8 ** -0.5
    Tv, seg = 80, 92
    out = O.pisa_pg_attention(q, k, v, 0.25, 16, 2, s, dtype=f64, text_tokens=30, text_valid=12)
    es = O.effective_scale(s)
    torch.testing.assert_close(out[..., Tv:seg, :], O.dense_attention(q[..., Tv:seg, :], k[..., :seg, :],
                                                                     v[..., :seg, :], es), rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(out[..., seg:, :], O.dense_attention(q[..., seg:, :], k[..., seg:, :],
                                                                   v[..., seg:, :], es), rtol=1e-10, atol=1e-10)
    k2, v2 = k.clone(), v.clone()
    k2[..., seg:, :] = torch.randn(18, 8, dtype=f64)   # padding keys/values do not reach video rows
    v2[..., seg:, :] = torch.randn(18, 8, dtype=f64)
    out2 = O.pisa_pg_attention(q, k2, v2, 0.25, 16, 2, s, dtype=f64, text_tokens=30, text_valid=12)
    torch.testing.assert_close(out2[..., :seg, :], out[..., :seg, :], rtol=0, atol=0)
    full = O.pisa_pg_attention(q, k, v, 0.25, 16, 2, s, dtype=f64, text_tokens=30)
    assert not torch.allclose(full[..., :Tv, :], out[..., :Tv, :])   # padding keys matter when unmasked


def test_literal_gamma_known_answer():
    """A hand-worked case of the literal (never rescaled) Gamma, group_pisa_attention.py
    :201 (g_l starts at 0), :231-235 (the running max rescales acc and l_i only),
    :242-243 (g_l += sum p-bar * n), :258-259 (o = acc / (l_i + g_l)).

    One channel, blocks of one token, groups of one block; scale = 1 / LOG2E so that the
    base-2 score is c * q * k = q * k.  q = 1 everywhere, keys 0, 1, 2 with values 1, 2, 4,
    and every query block selects block 0.  Then for every row:
      phase 1: m = 0, l = 1, acc = 1;
      group 1 (mean score 1 > m): acc, l *= 2^-1 -> 0.5, 0.5; acc += 1 * 2 -> 2.5; g_l = 1 * 1 = 1;
      group 2 (mean score 2 > m): acc, l *= 2^-1 -> 1.25, 0.25; g_l stays 1; acc += 4 -> 5.25; g_l = 2;
      o = 5.25 / (0.25 + 2) = 7/3.
    With Gamma rescaled like acc and l (the 'consistent' form) g_l = 0.5 + 1 = 1.5 and
    o = 5.25 / 1.75 = 3, which is also exact softmax attention, (1 + 2*2 + 4*4) / (1 + 2 + 4):
    single-token blocks make the zero-order term exact and H_j = 0."""
    q = torch.ones(1, 1, 3, 1, dtype=f64)
    k = torch.tensor([0.0, 1.0, 2.0], dtype=f64).reshape(1, 1, 3, 1)
    v = torch.tensor([1.0, 2.0, 4.0], dtype=f64).reshape(1, 1, 3, 1)
    idx = torch.zeros(1, 1, 3, 1, dtype=torch.int32)
    scale = 1.0 / O.LOG2E
    lit = O.pisa_pg_attention(q, k, v, 1 / 3, 1, 1, scale, gamma="literal", indices=idx, dtype=f64)
    con = O.pisa_pg_attention(q, k, v, 1 / 3, 1, 1, scale, gamma="consistent", indices=idx, dtype=f64)
    torch.testing.assert_close(lit[0, 0, :, 0], torch.full((3,), 7 / 3, dtype=f64), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(con[0, 0, :, 0], torch.full((3,), 3.0, dtype=f64), rtol=1e-12, atol=1e-12)
    loop = O.pisa_pg_attention_loop(q[0, 0], k[0, 0], v[0, 0], idx[0, 0], 1, 1, scale, "literal")
    torch.testing.assert_close(loop[:, 0], torch.full((3,), 7 / 3, dtype=f64), rtol=1e-12, atol=1e-12)


def test_reference_precision_rounds_only_where_the_reference_does():
    """The ref_precision mode (the reference's own bf16 roundings: stored kc/vc/h_group,
    P and P-bar before their products, the output) on the hand-worked case above:
    every intermediate there is a power of two or a small integer, exact in bf16, so
    only the output rounds and the result is bf16(7/3) for the literal Gamma."""
    q = torch.ones(1, 1, 3, 1, dtype=f64)
    k = torch.tensor([0.0, 1.0, 2.0], dtype=f64).reshape(1, 1, 3, 1)
    v = torch.tensor([1.0, 2.0, 4.0], dtype=f64).reshape(1, 1, 3, 1)
    idx = torch.zeros(1, 1, 3, 1, dtype=torch.int32)
    rp = O.pisa_pg_attention(q, k, v, 1 / 3, 1, 1, 1.0 / O.LOG2E, indices=idx, dtype=f64, ref_precision=True)
    want = torch.tensor(7 / 3, dtype=f64).to(torch.bfloat16).to(f64)
    assert float(want) != 7 / 3
    torch.testing.assert_close(rp[0, 0, :, 0], want.expand(3), rtol=0, atol=0)


def test_reference_precision_text_rows_round_p():
    """Dense text rows at the reference's precision: P is rounded to bf16 before P.V and
    the row sum stays fp32, so the result equals that computation spelled out."""
    g = torch.Generator().manual_seed(3)
    T, X, D = 40, 9, 4
    q, k, v = (torch.randn(1, 1, T, D, generator=g, dtype=f64) for _ in range(3))
    out = O.pisa_pg_attention(q, k, v, 0.5, 8, 2, 0.5, dtype=f64, text_tokens=X, ref_precision=True)
    x = (0.5 * O.LOG2E) * (q[0, 0, T - X:] @ k[0, 0].T)
    p = torch.exp2(x - x.amax(-1, keepdim=True))
    pb = p.to(torch.bfloat16).to(f64)
    want = ((pb @ v[0, 0]) / p.sum(-1, keepdim=True)).to(torch.bfloat16).to(f64)
    torch.testing.assert_close(out[0, 0, T - X:], want, rtol=0, atol=0)
    assert not torch.equal(pb, p)


@pytest.mark.parametrize("dtype,fn", [(torch.bfloat16, O.bf16_ulp), (torch.float16, O.f16_ulp)])
def test_ulp_is_the_spacing_of_adjacent_values(dtype, fn):
    """ulp(x) = next representable value above |x| minus |x|, over normal and (fp16)
    subnormal magnitudes, from the bit patterns themselves."""
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(4000, generator=g, dtype=f64) * torch.exp2(torch.randint(-30, 12, (4000,), generator=g))).to(dtype)
    x = x[torch.isfinite(x) & (x != 0)].abs()
    nxt = (x.view(torch.int16) + 1).view(dtype)
    ok = torch.isfinite(nxt)
    spacing = nxt[ok].double() - x[ok].double()
    torch.testing.assert_close(fn(x[ok].double()), spacing, rtol=0, atol=0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_reference_precision_rounds_to_the_requested_type(dtype):
    """ref_precision=dtype: every output is representable in dtype, and it differs from
    the unrounded oracle by no more than the roundings of P, the statistics and the
    output can account for (a few ulps of dtype relative to the output scale)."""
    q, k, v = rand_qkv(1, 2, 200, 16, seed=9, scale=1.0)
    s = 16 ** -0.5
    exact, aux = O.pisa_pg_attention(q, k, v, 0.3, 16, 4, s, dtype=f64, return_aux=True)
    idx = aux["idx"].reshape(1, 2, -1, aux["idx"].shape[-1])
    rp = O.pisa_pg_attention(q, k, v, 0.3, 16, 4, s, dtype=f64, indices=idx, ref_precision=dtype)
    assert torch.equal(rp, rp.to(dtype).to(f64))
    err = (rp - exact).abs().max().item()
    scale = exact.abs().max().item()
    eps = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    assert 0 < err <= 16 * eps * scale
    # fp16 keeps more bits than bf16, so its emulation lands closer to the exact oracle
    if dtype == torch.float16:
        rb = O.pisa_pg_attention(q, k, v, 0.3, 16, 4, s, dtype=f64, indices=idx, ref_precision=True)
        assert err < (rb - exact).abs().max().item()
