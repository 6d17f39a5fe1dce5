"""Pins oracle.permute against the reference's reshape/transpose closed forms.

Reference: svg/models/hyvideo/placement.py:6-31 (the torch closed forms, which
put the fixed context tail at the END of the sequence) and the kernel branches
:73-100 / :320-343 (index maps).  The closed forms below are the reference's
formulation (reshape -> transpose -> reshape), a different computation from the
oracle's index arithmetic."""
import numpy as np
import pytest

from oracle import pisa_oracle as O


def closed_to_token_major(x, ctx, F, P):
    B, H, S, D = x.shape
    out = x.copy()
    body = x[:, :, : S - ctx]
    out[:, :, : S - ctx] = body.reshape(B, H, F, P, D).transpose(0, 1, 3, 2, 4).reshape(B, H, F * P, D)
    return out


def closed_to_frame_major(x, ctx, F, P):
    B, H, S, D = x.shape
    out = x.copy()
    body = x[:, :, : S - ctx]
    out[:, :, : S - ctx] = body.reshape(B, H, P, F, D).transpose(0, 1, 3, 2, 4).reshape(B, H, F * P, D)
    return out


@pytest.mark.parametrize("F,P,ctx", [(4, 16, 0), (3, 7, 5), (21, 30, 0), (11, 40, 26), (1, 9, 3), (5, 1, 2)])
def test_forward_inverse_match_closed_forms(F, P, ctx):
    rng = np.random.default_rng(F * 100 + P + ctx)
    S = ctx + F * P
    x = rng.standard_normal((2, 3, S, 4)).astype(np.float32)
    np.testing.assert_array_equal(O.permute(x, F, P, ctx, inverse=False), closed_to_token_major(x, ctx, F, P))
    np.testing.assert_array_equal(O.permute(x, F, P, ctx, inverse=True), closed_to_frame_major(x, ctx, F, P))


@pytest.mark.parametrize("F,P,ctx", [(4, 16, 0), (21, 30, 7), (33, 13, 256)])
def test_bijective_and_round_trip(F, P, ctx):
    S = ctx + F * P
    for inv in (False, True):
        src = O.permute_index(S, F, P, ctx, inv)
        assert np.array_equal(np.sort(src), np.arange(S))
        assert np.array_equal(src[S - ctx:], np.arange(S - ctx, S))
    x = np.arange(2 * S * 2).reshape(1, 2, S, 2)
    y = O.permute(x, F, P, ctx, inverse=False)
    np.testing.assert_array_equal(O.permute(y, F, P, ctx, inverse=True), x)
    np.testing.assert_array_equal(O.permute(O.permute(x, F, P, ctx, True), F, P, ctx, False), x)


def test_single_token_moves():
    # frame f, patch p (frame-major index f*P + p) lands at p*F + f in token-major order.
    F, P = 3, 5
    x = np.zeros((1, 1, F * P, 1), dtype=np.int64)
    x[0, 0, :, 0] = np.arange(F * P)
    y = O.permute(x, F, P, 0)
    for f in range(F):
        for p in range(P):
            assert y[0, 0, p * F + f, 0] == f * P + p


def test_head_mask_keeps_spatial_heads():
    F, P, ctx = 4, 6, 3
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 3, ctx + F * P, 8))
    mask = np.array([[1, 0, 1], [0, 0, 1]])
    y = O.permute(x, F, P, ctx, head_is_temporal=mask)
    full = O.permute(x, F, P, ctx)
    for b in range(2):
        for h in range(3):
            np.testing.assert_array_equal(y[b, h], full[b, h] if mask[b, h] else x[b, h])
