"""DiT block row operations (K6) on the GPU: gated residual, LayerNorm and shift/scale
modulation of token rows, fused into one pass (``pasa_row_ops``).

Drop-in names for the reference's Triton kernels, same arguments and results:

* ``triton_layernorm_forward(x, w, b, eps, elementwise_affine=True)`` -> fp32
  (svg/kernels/triton/layernorm.py:200-206)
* ``triton_modulate_shift_forward(x, scale, shift, output_dtype=torch.float32)``
  -> x * (1 + scale) + shift (svg/kernels/triton/modulate.py:45-78)
* ``triton_modulate_gate_residual_forward(residual, x, gate, output_dtype=torch.float32)``
  -> residual + x * gate (modulate.py:125-164)

and the fused calls the Wan block makes with them (svg/models/wan/custom_models.py:23-115):
``ln_modulate`` (norm1 / norm3 + modulation), ``gate_residual_ln`` (gated residual
update in place + norm2), ``residual_ln_modulate`` (cross-attention residual in place +
norm3 + modulation) and ``gate_residual`` (the feed-forward's gated residual in place).

Modulation vectors are fp32 [B, 1, N] or [B, N] (one row per batch of ``x``'s [B, S, N]);
the reference's Triton kernels read only their first row, which is the same for B = 1.
There is no CPU path: every call needs ROCm device tensors.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib

_DT = {torch.bfloat16: 0, torch.float32: 2}
MAX_COLS = 8192


def _rows(x: torch.Tensor) -> Tuple[int, int, int]:
    """(rows, cols, rows_per_batch) of a [B, S, N] or [M, N] tensor."""
    if x.dim() == 3:
        return x.shape[0] * x.shape[1], x.shape[2], x.shape[1]
    if x.dim() == 2:
        return x.shape[0], x.shape[1], x.shape[0]
    raise ValueError(f"row ops take [B, S, N] or [M, N] tensors, got {tuple(x.shape)}")


def _param(t: Optional[torch.Tensor], n: int, batches: int) -> Tuple[Optional[torch.Tensor], int]:
    """fp32 contiguous modulation rows and their stride (0 = one row for all batches)."""
    if t is None:
        return None, 0
    t = t.to(torch.float32).reshape(-1, n).contiguous()
    if t.shape[0] == 1:
        return t, 0
    if t.shape[0] != batches:
        raise ValueError(f"modulation has {t.shape[0]} rows for {batches} batches")
    return t, n


def _widen(t: torch.Tensor) -> torch.Tensor:
    """Types the kernel does not read (fp16) widen to fp32, exactly."""
    return t if t.dtype in _DT else t.to(torch.float32)


def _check(t: torch.Tensor, name: str):
    if not t.is_cuda:
        raise ValueError(f"{name}: the row-ops kernel needs ROCm device tensors (there is no CPU path)")
    if t.dtype not in _DT:
        raise ValueError(f"{name}: dtype {t.dtype} not in (bfloat16, float32)")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def row_ops(x: torch.Tensor, *, residual: Optional[torch.Tensor] = None, gate: Optional[torch.Tensor] = None,
            h_out: Optional[torch.Tensor] = None, layernorm: bool = False, weight: Optional[torch.Tensor] = None,
            bias: Optional[torch.Tensor] = None, scale: Optional[torch.Tensor] = None,
            shift: Optional[torch.Tensor] = None, y: Optional[torch.Tensor] = None, eps: float = 1e-6) -> None:
    """One ``pasa_row_ops`` call on the current stream (see include/pasa.h)."""
    _check(x, "x")
    M, N, S = _rows(x)
    B = M // S
    for name, t in (("residual", residual), ("h_out", h_out), ("y", y)):
        if t is not None:
            _check(t, name)
            if t.shape != x.shape:
                raise ValueError(f"{name} shape {tuple(t.shape)} != x shape {tuple(x.shape)}")
    gate, gs = _param(gate, N, B)
    scale, ss = _param(scale, N, B)
    shift, hs = _param(shift, N, B)
    # one stride serves gate, scale and shift: rows given per batch make every one per batch
    stride = max(gs, ss, hs)
    if stride:
        gate = gate if gate is None or gs else gate.expand(B, N).contiguous()
        scale = scale if scale is None or ss else scale.expand(B, N).contiguous()
        shift = shift if shift is None or hs else shift.expand(B, N).contiguous()
    wb_dt = torch.float32
    if weight is not None or bias is not None:
        ref = weight if weight is not None else bias
        wb_dt = ref.dtype if ref.dtype in _DT else torch.float32
        weight = None if weight is None else weight.to(wb_dt).contiguous()
        bias = None if bias is None else bias.to(wb_dt).contiguous()
    lib = _lib.load()
    p = lambda t: None if t is None else t.data_ptr()
    _lib.check("pasa_row_ops", lib.pasa_row_ops(
        p(x), _DT[x.dtype], p(residual), _DT[residual.dtype] if residual is not None else 0, p(gate), p(h_out),
        _DT[h_out.dtype] if h_out is not None else 0,
        int(layernorm), p(weight), p(bias), _DT[wb_dt], p(scale), p(shift), p(y),
        _DT[y.dtype] if y is not None else 0, M, N, S, stride, float(eps),
        torch.cuda.current_stream(x.device).cuda_stream))


# ---- the reference's three kernels ---------------------------------------------------

def triton_layernorm_forward(x, w, b, eps, elementwise_affine=True):
    """LayerNorm of the last dimension in fp32, returned as fp32."""
    if elementwise_affine:
        assert w is not None and b is not None
    else:
        assert w is None and b is None
    x = _widen(x).contiguous()
    y = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    row_ops(x, layernorm=True, weight=w, bias=b, y=y, eps=eps)
    return y


def triton_modulate_shift_forward(x, scale, shift, output_dtype=torch.float32):
    """y = x * (1 + scale) + shift."""
    x = _widen(x).contiguous()
    y = torch.empty(x.shape, dtype=output_dtype, device=x.device)
    row_ops(x, scale=scale, shift=shift, y=y)
    return y


def triton_modulate_gate_residual_forward(residual, x, gate, output_dtype=torch.float32):
    """y = residual + x * gate."""
    x = _widen(x).contiguous()
    y = torch.empty(x.shape, dtype=output_dtype, device=x.device)
    row_ops(x, residual=_widen(residual).contiguous(), gate=gate, h_out=y)
    return y


# ---- fused calls of the Wan block ------------------------------------------------------

def ln_modulate(x, scale, shift, eps, weight=None, bias=None, out_dtype=torch.bfloat16):
    """LayerNorm(x) [* weight + bias] * (1 + scale) + shift, one pass (norm1 / norm3)."""
    y = torch.empty(x.shape, dtype=out_dtype, device=x.device)
    row_ops(x.contiguous(), layernorm=True, weight=weight, bias=bias, scale=scale, shift=shift, y=y, eps=eps)
    return y


def gate_residual_ln(h, x, gate, eps, weight=None, bias=None, out_dtype=torch.bfloat16):
    """h <- bf16(h + x * gate) in place; returns LayerNorm(h) * weight + bias (norm2)."""
    y = torch.empty(h.shape, dtype=out_dtype, device=h.device)
    row_ops(x.contiguous(), residual=h, gate=gate, h_out=h, layernorm=True, weight=weight, bias=bias, y=y,
            eps=eps)
    return y


def residual_ln_modulate(h, x, scale, shift, eps, out_dtype=torch.bfloat16):
    """h <- bf16(h + x) in place; returns LayerNorm(h) * (1 + scale) + shift (norm3)."""
    y = torch.empty(h.shape, dtype=out_dtype, device=h.device)
    row_ops(x.contiguous(), residual=h, h_out=h, layernorm=True, scale=scale, shift=shift, y=y, eps=eps)
    return y


def gate_residual(h, x, gate):
    """h <- bf16(h + x * gate) in place."""
    row_ops(x.contiguous(), residual=h, gate=gate, h_out=h)
    return h
