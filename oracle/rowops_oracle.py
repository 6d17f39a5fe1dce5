"""CPU oracle for the DiT block row operations (K6): gated residual, LayerNorm and
shift/scale modulation.

TEST INFRASTRUCTURE ONLY.  Only tests/ may import this module, as the checker; no
product code path calls it.

The steps restate the Wan block's elementwise work (svg/models/wan/custom_models.py:32-112)
in fp32 torch on the CPU, one rounded operation per step as in the reference's PyTorch
fallback there:

* gated residual: h = r + x * gate (custom_models.py:64, :111; Triton form
  svg/kernels/triton/modulate.py:85-122), plain residual h = r + x (:81), rounded to
  h's storage type.
* LayerNorm: the two-pass form of svg/kernels/triton/layernorm.py:38-61 / :127-150:
  mean = sum(x)/N, var = sum((x-mean)^2)/N, rstd = 1/sqrt(var + eps),
  y = (x - mean) * rstd [* w + b].
* modulation: y = x * (1 + scale) + shift (custom_models.py:54, :101;
  modulate.py:36-41).

The two row sums are taken in the kernel's fixed order (per lane l the chunks
l, l+64, ... of 8 elements in sequence, then a butterfly over the 64 lanes) and every
operation is a correctly rounded fp32 one (``sqrt_rn``), so the GPU result is
reproduced bit for bit on any host.  Pinned: equal to
torch.nn.functional.layer_norm up to the order of the sums, closed forms (constant rows,
alternating rows), and the identities scale = shift = 0 and gate = 0.
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch

LANES = 64


def sqrt_rn(t: torch.Tensor) -> torch.Tensor:
    """Correctly rounded fp32 square root.  torch's CPU float32 sqrt is not: on the
    hosts measured it differs from the IEEE result for 0.7% to 17% of random inputs,
    depending on the CPU, so the oracle takes numpy's (the hardware instruction)."""
    return torch.from_numpy(np.sqrt(t.detach().cpu().numpy().astype(np.float32)))


def _lane_sums(v: torch.Tensor, skip_padding: bool) -> torch.Tensor:
    """Per-lane sequential fp32 sums over the lane's chunks: [M, N] -> [M, 64]."""
    M, N = v.shape
    nc = N // 8
    cpt = (nc + LANES - 1) // LANES
    ch = torch.zeros(M, cpt * LANES, 8, dtype=torch.float32)
    ch[:, :nc] = v.reshape(M, nc, 8)
    ch = ch.reshape(M, cpt, LANES, 8)
    valid = (torch.arange(cpt)[:, None] * LANES + torch.arange(LANES)[None, :]) < nc  # [cpt, 64]
    acc = torch.zeros(M, LANES, dtype=torch.float32)
    for i in range(cpt):
        for e in range(8):
            nxt = acc + ch[:, i, :, e]
            acc = torch.where(valid[i][None, :], nxt, acc) if skip_padding else nxt
    return acc


def _wave_sum(part: torch.Tensor) -> torch.Tensor:
    """Butterfly over 64 lanes (x += x[lane ^ m], m = 32 .. 1); [M, 64] -> [M]."""
    idx = torch.arange(LANES)
    x = part
    for m in (32, 16, 8, 4, 2, 1):
        x = x + x[:, idx ^ m]
    return x[:, 0]


def layer_norm_rows(v: torch.Tensor, eps: float) -> torch.Tensor:
    """(v - mean) * rstd over the last dim, fp32, in the kernel's summation order."""
    shape = v.shape
    v = v.reshape(-1, shape[-1]).float()
    N = v.shape[1]
    n = torch.tensor(float(N), dtype=torch.float32)
    mean = _wave_sum(_lane_sums(v, skip_padding=False)) / n
    d = v - mean[:, None]
    var = _wave_sum(_lane_sums(d * d, skip_padding=True)) / n
    rstd = torch.tensor(1.0, dtype=torch.float32) / sqrt_rn(var + torch.tensor(eps, dtype=torch.float32))
    return (d * rstd[:, None]).reshape(shape)


def _rows_param(t: Optional[torch.Tensor], shape) -> Optional[torch.Tensor]:
    """fp32 modulation rows broadcast over [B, S, N] (t: [N], [1, N], [B, N] or [B, 1, N])."""
    if t is None:
        return None
    t = t.float()
    if len(shape) == 3:
        return t.reshape(-1, 1, shape[-1])
    return t.reshape(-1, shape[-1])


def row_ops(x: torch.Tensor, *, residual: Optional[torch.Tensor] = None, gate: Optional[torch.Tensor] = None,
            h_dtype: torch.dtype = torch.bfloat16, layernorm: bool = False, weight: Optional[torch.Tensor] = None,
            bias: Optional[torch.Tensor] = None, scale: Optional[torch.Tensor] = None,
            shift: Optional[torch.Tensor] = None, y_dtype: Optional[torch.dtype] = torch.bfloat16,
            eps: float = 1e-6):
    """(h, y) of one row-ops call; h is None without a residual, y None when y_dtype is None."""
    v = x.float()
    h = None
    if residual is not None:
        r = residual.float()
        v = r + v * _rows_param(gate, x.shape) if gate is not None else r + v
        h = v.to(h_dtype)
        v = h.float()
    if y_dtype is None:
        return h, None
    if layernorm:
        v = layer_norm_rows(v, eps)
    if weight is not None:
        v = v * weight.float()
    if bias is not None:
        v = v + bias.float()
    if scale is not None:
        v = v * (1.0 + _rows_param(scale, x.shape)) + _rows_param(shift, x.shape)
    return h, v.to(y_dtype)
