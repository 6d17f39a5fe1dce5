"""Pins of the prologue oracle (oracle/prologue_oracle.py) on the CPU: library
routines, closed forms and invariants, each chosen so that a plausible mistake (a
dropped weight, a rounding in the wrong place, a swapped sign or pair order) fails."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import prologue_oracle as P


def bf16(x):
    return x.to(torch.bfloat16)


def rand_bf16(*shape, seed=0, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    return bf16(torch.randn(*shape, generator=g) * scale)


def test_rms_norm_once_equals_torch_rms_norm():
    # torch's rms_norm on bf16 CPU tensors computes in fp32 and rounds once
    x = rand_bf16(512, 128, seed=1, scale=3.0)
    w = bf16(torch.rand(128, generator=torch.Generator().manual_seed(2)) + 0.5)
    for eps in (1e-6, 1e-3):
        assert torch.equal(P.rms_norm_once(x, w, eps), F.rms_norm(x, (128,), w, eps))
    x2 = rand_bf16(64, 5120, seed=3)
    w2 = bf16(torch.rand(5120) + 0.5)
    assert torch.equal(P.rms_norm_once(x2, w2, 1e-6), F.rms_norm(x2, (5120,), w2, 1e-6))


def test_rms_norm_closed_forms():
    # rows of +-a: mean(x^2) = a^2, so x*rstd = +-1/sqrt(1 + eps/a^2)
    a = 3.0
    x = bf16(torch.tensor([[a, -a] * 32]))
    w = bf16(torch.linspace(0.5, 2.0, 64))
    eps = 1e-6
    r = 1.0 / math.sqrt(1.0 + eps / a ** 2)
    sign = torch.tensor([1.0, -1.0] * 32)
    want_once = bf16(sign * r * w.float())
    assert torch.equal(P.rms_norm_once(x, w, eps)[0], want_once)
    want_twice = bf16(bf16(sign * r).float() * w.float())
    assert torch.equal(P.rms_norm_twice(x, w, eps)[0], want_twice)


def test_rms_norm_scale_invariant_and_weight_used():
    x = rand_bf16(32, 64, seed=4)
    w = bf16(torch.rand(64) + 0.5)
    for fn in (P.rms_norm_once, P.rms_norm_twice):
        # a power-of-two scale is exact in fp, so with eps = 0 the output is unchanged
        assert torch.equal(fn(x, w, 0.0), fn(bf16(x.float() * 8.0), w, 0.0))
        assert not torch.equal(fn(x, w, 1e-6), fn(x, None, 1e-6))
        y = fn(x, None, 0.0).float()
        torch.testing.assert_close((y * y).mean(-1), torch.ones(32), rtol=2e-2, atol=0)


def test_rms_norm_roundings_differ_only_by_the_intermediate_cast():
    x = rand_bf16(256, 128, seed=5, scale=4.0)
    w = bf16(torch.rand(128) * 3 + 0.1)
    once, twice = P.rms_norm_once(x, w, 1e-6), P.rms_norm_twice(x, w, 1e-6)
    frac = (once != twice).float().mean().item()
    assert 0.01 < frac < 0.6                        # the forms are distinguishable
    ulp = (once.float() - twice.float()).abs() / torch.clamp(once.float().abs(), min=1e-30)
    assert float(ulp.max()) <= 2 ** -7              # ... by about one bf16 ulp
    one = bf16(torch.ones(128))                     # with w = 1 the extra cast is a no-op
    agree = (P.rms_norm_once(x, one, 1e-6) == P.rms_norm_twice(x, one, 1e-6)).float().mean()
    assert float(agree) > 0.999


def angles_tables(S, D, seed=0, fixed=None):
    g = torch.Generator().manual_seed(seed)
    ang = torch.rand(S, D // 2, generator=g, dtype=torch.float64) * 6.0 if fixed is None else \
        torch.full((S, D // 2), fixed, dtype=torch.float64)
    cos = torch.cos(ang).repeat_interleave(2, -1).float()
    sin = torch.sin(ang).repeat_interleave(2, -1).float()
    return ang, cos, sin


def test_rope_closed_forms():
    x = rand_bf16(2, 3, 6, 16, seed=6)
    ang0, c0, s0 = angles_tables(6, 16, fixed=0.0)
    assert torch.equal(P.rope_cossin(x, c0, s0), x)
    assert torch.equal(P.rope_complex(x, torch.cos(ang0), torch.sin(ang0)), x)
    # quarter turn: (a, b) -> (-b, a) exactly when cos is 0 and sin is 1
    c = torch.zeros(6, 16)
    s = torch.ones(6, 16)
    want = torch.stack([-x[..., 1::2], x[..., 0::2]], -1).flatten(-2)
    assert torch.equal(P.rope_cossin(x, c, s), want)
    assert torch.equal(P.rope_complex(x, torch.zeros(6, 8, dtype=torch.float64),
                                      torch.ones(6, 8, dtype=torch.float64)), want)


def test_rope_forms_agree_preserve_norm_and_compose():
    x = rand_bf16(1, 2, 40, 128, seed=7)
    ang, cos, sin = angles_tables(40, 128, seed=8)
    a = P.rope_cossin(x, cos, sin).float()
    b = P.rope_complex(x, torch.cos(ang), torch.sin(ang)).float()
    assert float((a - b).abs().max()) <= 2 ** -7 * float(x.float().abs().max())
    assert float((a != b).float().mean()) < 0.05
    n_in = x.float()[..., 0::2] ** 2 + x.float()[..., 1::2] ** 2
    n_out = a[..., 0::2] ** 2 + a[..., 1::2] ** 2
    torch.testing.assert_close(n_out, n_in, rtol=2e-2, atol=1e-2)
    ang2 = torch.rand(40, 64, dtype=torch.float64, generator=torch.Generator().manual_seed(9))
    twice = P.rope_complex(P.rope_complex(x, torch.cos(ang), torch.sin(ang)), torch.cos(ang2), torch.sin(ang2))
    once = P.rope_complex(x, torch.cos(ang + ang2), torch.sin(ang + ang2))
    torch.testing.assert_close(twice.float(), once.float(), rtol=0, atol=2 ** -6 * float(x.float().abs().max()))
    # pair order: swapping the channels of a pair is the inverse rotation's job, not this one's
    xs = torch.stack([x[..., 1::2], x[..., 0::2]], -1).flatten(-2)
    assert not torch.equal(P.rope_cossin(xs, cos, sin), P.rope_cossin(x, cos, sin))


def test_qkv_prologue_composition_layout():
    # no norm and no rope: a pure head split; rope rows past rope_rows untouched
    B, S, H, D = 2, 10, 3, 64
    xq, xk, xv = (rand_bf16(B, S, H * D, seed=s) for s in (10, 11, 12))
    q, k, v = P.qkv_prologue(xq, xk, xv, H)
    assert torch.equal(q, xq.reshape(B, S, H, D).permute(0, 2, 1, 3))
    assert torch.equal(v, xv.reshape(B, S, H, D).permute(0, 2, 1, 3))
    _, cos, sin = angles_tables(7, D, seed=13)
    q2, k2, v2 = P.qkv_prologue(xq, xk, xv, H, rope=("cossin", cos, sin), rope_rows=7)
    assert torch.equal(q2[:, :, 7:], q[:, :, 7:]) and torch.equal(v2, v)
    assert not torch.equal(q2[:, :, :7], q[:, :, :7])
    # per-head norm of head h equals the row norm of that head's slice alone
    w = bf16(torch.rand(D) + 0.5)
    qh, _, _ = P.qkv_prologue(xq, None, None, H, wq=w, norm="head", rounding="twice")
    for h in range(H):
        assert torch.equal(qh[:, h], P.rms_norm_twice(xq[..., h * D:(h + 1) * D], w, 1e-6))
