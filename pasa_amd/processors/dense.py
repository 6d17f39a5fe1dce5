"""Dense attention of the processors' warm-up layers (``first_layers_fp`` /
``first_times_fp``): the reference's flash_attention / varlen attention
(svg/models/wan/attention.py:299-301, :378-379; svg/models/hyvideo/attention.py:450-476,
:509-510, :632-633, :671-672).

bf16 or fp16 device tensors with head_dim 128 run on K4's exact-tile path
(``pasa_amd.ops.dense_attention``, 1.6x PyTorch SDPA at the Wan-14B 720p shape).
Other inputs (fp32 models, other head dims, the CPU tensors of the processor unit
tests) take PyTorch SDPA, as the reference does.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from .. import ops


def kernel_ok(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> bool:
    return (query.is_cuda and query.dtype in (torch.bfloat16, torch.float16) and query.shape[-1] == 128
            and query.shape == key.shape == value.shape and key.dtype == value.dtype == query.dtype)


def attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
              valid: Optional[int] = None) -> torch.Tensor:
    """softmax attention of [B, H, N, D] tensors; with ``valid`` < N, block-diagonal over
    [0, valid) and [valid, N) (cu_seqlens [0, valid, N])."""
    N = query.shape[2]
    valid = N if valid is None else int(valid)
    if kernel_ok(query, key, value) and 1 <= valid <= N:
        return ops.dense_attention(query.contiguous(), key.contiguous(), value.contiguous(),
                                   text_tokens=N - valid, text_valid=0)
    if valid >= N:
        return F.scaled_dot_product_attention(query, key, value, dropout_p=0.0, is_causal=False)
    out = torch.empty_like(query)
    for a, b in ((0, valid), (valid, N)):
        if b > a:
            out[:, :, a:b] = F.scaled_dot_product_attention(query[:, :, a:b], key[:, :, a:b], value[:, :, a:b],
                                                            dropout_p=0.0, is_causal=False)
    return out
