"""Pins the oracle's block statistics, group moment and selection.

Block statistics (reference group_pisa_attention.py:86-129, :287) and the group
moment (:291-301) are checked against per-token / per-block Python loops in
float64; the selection (:365-375) against explicit dot products and a
brute-force stable sort on (-score, index)."""
import math

import numpy as np
import pytest
import torch

from oracle import pisa_oracle as O


def brute_stats(q, k, v, bt):
    T, D = q.shape
    nt = math.ceil(T / bt)
    qc = np.zeros((nt, D)); kc = np.zeros((nt, D)); vc = np.zeros((nt, D))
    hc = np.zeros((nt, D, D)); hn = np.zeros(nt)
    for j in range(nt):
        rows = range(j * bt, min(T, (j + 1) * bt))
        n = len(rows)
        qc[j] = sum(q[t] for t in rows) / n
        kc[j] = sum(k[t] for t in rows) / n
        vc[j] = sum(v[t] for t in rows)
        for t in rows:
            hc[j] += np.outer(k[t] - kc[j], v[t])
        hn[j] = math.sqrt(float((hc[j] ** 2).sum()))
    return qc, kc, vc, hc, hn


@pytest.mark.parametrize("T,bt,D", [(64, 16, 4), (70, 16, 5), (33, 8, 3), (5, 8, 2), (129, 32, 6)])
def test_block_stats_brute_force(T, bt, D):
    rng = np.random.default_rng(T + bt + D)
    q, k, v = (rng.standard_normal((T, D)) for _ in range(3))
    st = O.block_stats(*(torch.from_numpy(a)[None] for a in (q, k, v)), bt, dtype=torch.float64)
    qc, kc, vc, hc, hn = brute_stats(q, k, v, bt)
    np.testing.assert_allclose(st.qc[0].numpy(), qc, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(st.kc[0].numpy(), kc, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(st.vc[0].numpy(), vc, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(st.hc[0].numpy(), hc, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(st.hnorm[0].numpy(), hn, rtol=1e-10)
    assert st.n.tolist() == [min(bt, T - j * bt) for j in range(math.ceil(T / bt))]


def test_h_is_centred_moment():
    # H_j = sum k v^T - kc vc^T equals sum (k - kc) v^T and also sum k (v - vbar)^T.
    rng = np.random.default_rng(3)
    T, D, bt = 48, 4, 16
    k, v = rng.standard_normal((T, D)), rng.standard_normal((T, D))
    st = O.block_stats(*(torch.from_numpy(a)[None] for a in (k, k, v)), bt, dtype=torch.float64)
    for j in range(3):
        kb, vb = k[j * bt:(j + 1) * bt], v[j * bt:(j + 1) * bt]
        alt = (kb.T @ (vb - vb.mean(0)))
        np.testing.assert_allclose(st.hc[0, j].numpy(), alt, atol=1e-12)


@pytest.mark.parametrize("nt,G", [(16, 32), (64, 32), (70, 32), (7, 3), (9, 1)])
def test_group_moment_zero_padded_mean(nt, G):
    rng = np.random.default_rng(nt * 7 + G)
    hc = rng.standard_normal((2, nt, 3, 3))
    got = O.group_moment(torch.from_numpy(hc), G).numpy()
    ng = math.ceil(nt / G)
    assert got.shape == (2, ng, 3, 3)
    for b in range(2):
        for g in range(ng):
            acc = np.zeros((3, 3))
            for j in range(g * G, min(nt, (g + 1) * G)):
                acc += hc[b, j]
            np.testing.assert_allclose(got[b, g], acc / G, atol=1e-12)   # divides by G, not by #blocks


@pytest.mark.parametrize("density,nt,expect", [
    (0.1, 591, 59), (0.15, 256, 38), (0.25, 16, 4), (0.10, 929, 92), (1.0, 10, 10),
    (0.0, 10, 1), (2.0, 10, 10), (0.29, 100, 28), (-0.5, 8, 1), (0.999999, 3, 2)])
def test_num_selected(density, nt, expect):
    assert O.num_selected(density, nt) == expect
    assert expect == min(max(1, int(density * nt)), nt)


def test_select_scores_explicit():
    rng = np.random.default_rng(5)
    nt, D = 7, 5
    qc, kc = rng.standard_normal((nt, D)), rng.standard_normal((nt, D))
    hn = np.abs(rng.standard_normal(nt))
    noise = rng.standard_normal(nt)
    s = 0.37
    got = O.select_scores(*(torch.from_numpy(a) for a in (qc, kc, hn)), s, True, torch.from_numpy(noise)).numpy()
    for i in range(nt):
        for j in range(nt):
            ref = sum(qc[i, d] * (s * kc[j, d]) for d in range(D)) + (math.log(hn[j] + 1e-6) + noise[j])
            assert abs(got[i, j] - ref) < 1e-12
    got2 = O.select_scores(*(torch.from_numpy(a) for a in (qc, kc, hn)), s, False, torch.from_numpy(noise)).numpy()
    np.testing.assert_allclose(got2, (qc @ (s * kc).T), atol=1e-12)   # no bias, and noise ignored


def brute_topk(row, ns):
    return [j for j, _ in sorted(enumerate(row), key=lambda p: (-p[1], p[0]))][:ns]


def test_topk_brute_force_with_ties():
    rng = np.random.default_rng(11)
    rows = rng.integers(-3, 4, size=(40, 37)).astype(np.float32)   # many ties
    rows[0, :] = 0.0
    rows[1, ::2] = -0.0                                               # -0.0 ties with +0.0
    rows[2] = rng.standard_normal(37).astype(np.float32)
    for ns in (1, 5, 36, 37):
        got = O.topk_indices(torch.from_numpy(rows), ns).numpy()
        for r in range(rows.shape[0]):
            assert got[r].tolist() == brute_topk(rows[r].tolist(), ns)


def test_topk_negative_zero_equals_zero():
    row = torch.tensor([[0.0, -0.0, 0.0, -0.0, -1.0]])
    assert O.topk_indices(row, 4)[0].tolist() == [0, 1, 2, 3]
    row = torch.tensor([[-0.0, 0.0]])
    assert O.topk_indices(row, 1)[0].tolist() == [0]


def test_selection_mask():
    idx = torch.tensor([[[0, 33, 31, 64]]], dtype=torch.int32)
    m = O.selection_mask(idx, 70)
    assert m.shape == (1, 1, 3)
    assert m[0, 0, 0] == (1 | (1 << 31))
    assert m[0, 0, 1] == (1 << 1)
    assert m[0, 0, 2] == 1
