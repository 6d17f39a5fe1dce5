"""The attention processors' prologue on MI355X: Q/K RMSNorm and rotary embedding,
fused with the head split (K5, ``pasa_qkv_prologue`` in the C ABI).

Drop-in names for the prologue ops the reference calls:

* ``triton_rmsnorm_forward(x, w, eps)``: svg/kernels/triton/rmsnorm.py:51-101
  (row RMSNorm, one rounding).
* ``rms_norm_forward(x, weight, eps)``: in place on [..., D]; the absent
  ``_kernels.rms_norm_forward`` (svg/models/hyvideo/attention.py:167-173), with the
  rounding of its PyTorch fallback (diffusers RMSNorm, :196-200).
* ``apply_qk_rope_inplace_cossin_txtlast(query, key, cos, sin, txt_len)``: the absent
  ``_kernels`` op (hyvideo/attention.py:175-190); fallback semantics :211-230.
* ``apply_qk_rope_inplace_cossin_complex(query, key, freqs_real, freqs_imag, n)``: the
  absent ``_kernels`` op (svg/models/wan/attention.py:36-39); fallback semantics :49-57.

``qkv_prologue`` is the fused form the processors use: projections [B, S, H*D] in,
head-major [B, H, S, D] out, in one pass.  Like the attention ops, everything here
runs through libpasa_amd.so on a ROCm device; there is no CPU path.
"""
from __future__ import annotations

from typing import Optional, Sequence, Tuple

import torch

from . import _lib

LAYOUT_BHSD, LAYOUT_BSHD = 0, 1
NORMS = {None: 0, "head": 1, "row": 2}
ROUNDINGS = {"once": 0, "twice": 1}
ROPE_COSSIN_F32, ROPE_COMPLEX_F64 = 1, 2
MAX_ROW_CHANNELS = 8192  # heads * head_dim limit of the kernel


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _dev_bf16(*ts: Optional[torch.Tensor]) -> None:
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("the prologue kernel needs ROCm device tensors (there is no CPU path)")
        if t.dtype != torch.bfloat16:
            raise ValueError(f"the prologue kernel takes bf16 tensors, got {t.dtype}")
        if not t.is_contiguous():
            raise ValueError("the prologue kernel needs contiguous tensors")


def rope_tables_cossin(cos: torch.Tensor, sin: torch.Tensor, device) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp32 contiguous [rows, D] cos / sin on ``device`` (diffusers' real form)."""
    return (cos.to(device=device, dtype=torch.float32).contiguous(),
            sin.to(device=device, dtype=torch.float32).contiguous())


def rope_tables_complex(freqs, device, rows: int, half_dim: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp64 contiguous [rows, D/2] real / imaginary parts of the rotation coefficients.

    ``freqs`` is a complex tensor broadcastable to [rows, D/2] (the Wan processor's
    ``rotary_emb``) or a (real, imag) pair.  Complex64 widens to fp64 exactly, as the
    reference's complex128 product does."""
    if isinstance(freqs, (tuple, list)):
        re, im = freqs
    else:
        re, im = freqs.real, freqs.imag
    re = re.to(device=device, dtype=torch.float64).reshape(-1, half_dim)
    im = im.to(device=device, dtype=torch.float64).reshape(-1, half_dim)
    if re.shape[0] != rows or im.shape[0] != rows:
        raise ValueError(f"rotary table has {re.shape[0]} rows, expected {rows}")
    return re.contiguous(), im.contiguous()


def qkv_prologue(xq: Optional[torch.Tensor], xk: Optional[torch.Tensor], xv: Optional[torch.Tensor],
                 heads: int, *, wq: Optional[torch.Tensor] = None, wk: Optional[torch.Tensor] = None,
                 norm: Optional[str] = None, rounding: str = "once", eps: float = 1e-6,
                 rope: Optional[Tuple[str, torch.Tensor, torch.Tensor]] = None,
                 rope_rows: Optional[int] = None, in_layout: str = "bshd", out_layout: str = "bhsd",
                 out: Optional[Sequence[Optional[torch.Tensor]]] = None, out_seq_len: Optional[int] = None,
                 out_row0: int = 0) -> Tuple[Optional[torch.Tensor], ...]:
    """RMSNorm (``norm`` 'row' over H*D or 'head' over D, weights wq / wk) and rotary
    embedding of Q and K, plus the layout change of Q, K and V, in one launch.

    Inputs share one shape: [B, S, H*D] ('bshd') or [B, H, S, D] ('bhsd').
    ``rope`` = ('cossin', cos, sin) with fp32 [rope_rows, D] tables, or
    ('complex', re, im) with fp64 [rope_rows, D/2] tables; rows past ``rope_rows``
    (default: all) are not rotated.  ``out`` (optional) gives the three outputs;
    ``out_seq_len`` / ``out_row0`` place the S input rows inside longer outputs.
    Returns the outputs (None where the input was None)."""
    xs = (xq, xk, xv)
    ref = next((x for x in xs if x is not None), None)
    if ref is None:
        raise ValueError("no tensor given")
    _dev_bf16(*xs, wq, wk)
    if in_layout == "bshd":
        B, S, C = ref.shape
        H = int(heads)
        if C % H:
            raise ValueError(f"hidden {C} is not a multiple of heads {H}")
        D = C // H
    elif in_layout == "bhsd":
        B, H, S, D = ref.shape
    else:
        raise ValueError(f"unknown layout {in_layout!r}")
    for x in xs:
        if x is not None and x.shape != ref.shape:
            raise ValueError("q, k and v inputs must have one shape")
    OS = S if out_seq_len is None else int(out_seq_len)
    shape = (B, H, OS, D) if out_layout == "bhsd" else (B, OS, H * D)
    if out is None:
        outs = [None if x is None else torch.empty(shape, device=x.device, dtype=x.dtype) for x in xs]
    else:
        outs = list(out)
        for x, o in zip(xs, outs):
            if (x is None) != (o is None):
                raise ValueError("out must hold a tensor exactly where an input is given")
            if o is not None:
                _dev_bf16(o)
                if tuple(o.shape) != shape:
                    raise ValueError(f"output shape {tuple(o.shape)} != {shape}")
    cos = sin = None
    rope_mode = 0
    if rope is not None:
        kind, cos, sin = rope
        rope_mode = {"cossin": ROPE_COSSIN_F32, "complex": ROPE_COMPLEX_F64}[kind]
        want = torch.float32 if rope_mode == ROPE_COSSIN_F32 else torch.float64
        for t in (cos, sin):
            if not t.is_cuda or t.dtype != want or not t.is_contiguous():
                raise ValueError(f"{kind} rotary tables must be contiguous {want} device tensors")
    rows = S if rope_rows is None else int(rope_rows)
    lay = {"bhsd": LAYOUT_BHSD, "bshd": LAYOUT_BSHD}
    p = lambda t: None if t is None else t.data_ptr()
    _lib.call("pasa_qkv_prologue", p(xq), p(xk), p(xv), p(outs[0]), p(outs[1]), p(outs[2]), p(wq), p(wk),
              B, S, H, D, lay[in_layout], lay[out_layout], OS, int(out_row0), NORMS[norm], ROUNDINGS[rounding],
              float(eps), p(cos), p(sin), rope_mode, rows, _lib.DTYPE_BF16, _stream(ref))
    return tuple(outs)


# ---------------------------------------------------------------- drop-in names --

def triton_rmsnorm_forward(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """Row RMSNorm over the last dim N, one rounding (reference rmsnorm.py:51-101).
    x: [M, N] or [B, S, N] bf16; N a multiple of 64, at most 8192."""
    N = x.shape[-1]
    hd = 128 if N % 128 == 0 else 64
    if N % 64:
        raise ValueError(f"row length {N} is not a multiple of 64")
    x3 = x.reshape(1, -1, N)
    (y, _, _) = qkv_prologue(x3, None, None, N // hd, wq=w, norm="row", rounding="once", eps=eps,
                             out_layout="bshd")
    return y.reshape(x.shape)


def rms_norm_forward(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """In-place RMSNorm over the last dim D (64 or 128) of every row of x, with the
    rounding of diffusers' RMSNorm (the reference's fallback).  Returns x."""
    D = x.shape[-1]
    x4 = x.view(1, 1, -1, D)
    qkv_prologue(x4, None, None, 1, wq=weight, norm="head", rounding="twice", eps=eps, in_layout="bhsd",
                 out=(x4, None, None))
    return x


def apply_qk_rope_inplace_cossin_txtlast(query: torch.Tensor, key: torch.Tensor, cos: torch.Tensor,
                                         sin: torch.Tensor, txt_len: int):
    """In-place rotary embedding of query and key [B, H, L, D] on rows [0, L - txt_len);
    cos / sin: [L - txt_len, D] (diffusers' real form).  Returns (query, key)."""
    L = query.shape[2]
    c, s = rope_tables_cossin(cos, sin, query.device)
    qkv_prologue(query, key, None, query.shape[1], rope=("cossin", c, s), rope_rows=L - int(txt_len),
                 in_layout="bhsd", out=(query, key, None))
    return query, key


def apply_qk_rope_inplace_cossin_complex(query: torch.Tensor, key: torch.Tensor, freqs_real: torch.Tensor,
                                         freqs_imag: torch.Tensor, len_text_prompt: int = 0):
    """In-place complex-form rotary embedding (pairs as complex numbers, fp64) of query
    and key [B, H, L, D] on rows [0, L - len_text_prompt); freqs: [L - len, D/2].
    The reference only calls it with len_text_prompt = 0."""
    L, D = query.shape[2], query.shape[3]
    rows = L - int(len_text_prompt)
    re, im = rope_tables_complex((freqs_real, freqs_imag), query.device, rows, D // 2)
    qkv_prologue(query, key, None, query.shape[1], rope=("complex", re, im), rope_rows=rows,
                 in_layout="bhsd", out=(query, key, None))
    return query, key
