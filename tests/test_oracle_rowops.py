"""Pins of the row-ops oracle (oracle/rowops_oracle.py) on the CPU: LayerNorm against
torch.nn.functional.layer_norm, closed forms, and the modulation / residual identities."""
import math

import numpy as np
import torch
import torch.nn.functional as F

from oracle import rowops_oracle as R


def test_layer_norm_matches_torch():
    g = torch.Generator().manual_seed(0)
    for N in (8, 520, 1536, 5120):
        x = torch.randn(6, N, generator=g) * 3 + 1.5
        ours = R.layer_norm_rows(x, 1e-6)
        ref = F.layer_norm(x, (N,), eps=1e-6)
        assert (ours - ref).abs().max() < 2e-5, N


def test_layer_norm_affine_and_modulation_match_torch_steps():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(2, 5, 64, generator=g).to(torch.bfloat16)
    w, b = torch.randn(64, generator=g), torch.randn(64, generator=g)
    sc, sh = torch.randn(2, 1, 64, generator=g), torch.randn(2, 1, 64, generator=g)
    _, y = R.row_ops(x, layernorm=True, weight=w, bias=b, scale=sc, shift=sh, y_dtype=torch.float32)
    ref = F.layer_norm(x.float(), (64,), w, b, eps=1e-6) * (1 + sc) + sh
    assert (y - ref).abs().max() < 1e-4


def test_closed_forms():
    # constant rows normalise to exactly 0; alternating +-a rows to +-1/sqrt(1 + eps/a^2)
    c = torch.full((3, 1536), 7.25)
    assert torch.equal(R.layer_norm_rows(c, 1e-6), torch.zeros(3, 1536))
    a = 0.5
    alt = torch.tensor([a, -a] * 768).reshape(1, 1536)
    out = R.layer_norm_rows(alt, 1e-6)
    expect = 1.0 / math.sqrt(1.0 + 1e-6 / (a * a))
    assert torch.allclose(out.abs(), torch.full_like(out, expect), rtol=1e-6)
    assert torch.equal(torch.sign(out), torch.sign(alt))


def test_identities():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(4, 256, generator=g).to(torch.bfloat16)
    r = torch.randn(4, 256, generator=g).to(torch.bfloat16)
    # gate 0: h = r exactly
    h, _ = R.row_ops(x, residual=r, gate=torch.zeros(256), y_dtype=None)
    assert torch.equal(h, r)
    # scale = shift = 0: modulation is the identity on the normalised row
    _, y0 = R.row_ops(x, layernorm=True, y_dtype=torch.float32)
    _, y1 = R.row_ops(x, layernorm=True, scale=torch.zeros(256), shift=torch.zeros(256), y_dtype=torch.float32)
    assert torch.equal(y0, y1)
    # plain residual in bf16 equals torch's bf16 add
    h, _ = R.row_ops(x, residual=r, y_dtype=None)
    assert torch.equal(h, r + x)
    # gated residual equals the reference's fallback expression
    gate = torch.randn(1, 1, 256, generator=g)
    h, _ = R.row_ops(x.reshape(1, 4, 256), residual=r.reshape(1, 4, 256), gate=gate, y_dtype=None)
    assert torch.equal(h, (r.reshape(1, 4, 256).float() + x.reshape(1, 4, 256) * gate).to(torch.bfloat16))


def test_wave_sum_order_is_a_permutation_sum():
    g = torch.Generator().manual_seed(3)
    v = torch.randn(5, 64, generator=g, dtype=torch.float32)
    s = R._wave_sum(v)
    assert torch.allclose(s.double(), v.double().sum(-1), atol=1e-5)


def test_sqrt_is_correctly_rounded():
    """sqrt_rn equals the float64 root rounded to float32 (double rounding is exact for
    square roots from binary64 to binary32), including near-tie inputs."""
    g = torch.Generator().manual_seed(4)
    x = torch.cat([torch.rand(200000, generator=g) * 50, torch.rand(1000, generator=g) * 1e-30,
                   (torch.arange(1, 4097, dtype=torch.float32) ** 2) * (1 + 2.0 ** -23)])
    exact = torch.from_numpy(np.sqrt(x.double().numpy()).astype(np.float32))
    assert torch.equal(R.sqrt_rn(x), exact)
