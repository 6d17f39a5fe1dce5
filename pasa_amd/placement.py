"""Frame-major <-> token-major layout permutation (K1) with the reference's API.

Mirrors svg/models/hyvideo/placement.py: the closed forms
``hunyuan_token_reorder_to_token_major`` / ``..._to_frame_major`` (:6-31) and the
kernel launchers ``hunyuan_sparse_head_placement`` (:124-153, Q/K/V forward, per-
head temporal/spatial flag) and ``hunyuan_hidden_states_placement`` (:360-387,
inverse).  The last ``context_length`` tokens stay in place.  All work runs in
the gfx950 kernel behind ``pasa_permute``; there is no CPU path.
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch

from . import _lib
from .ops import _DTYPES, _check_device, _stream


def permute(srcs: Sequence[torch.Tensor], dsts: Sequence[torch.Tensor], num_frame: int,
            frame_size: int, context_length: int = 0, inverse: bool = False,
            head_is_temporal: Optional[torch.Tensor] = None) -> None:
    """Permute up to three [B,H,S,D] tensors into ``dsts`` (S = ctx + F*P).

    forward: dst[p*F + f] = src[f*P + p];  inverse: dst[f*P + p] = src[p*F + f].
    ``head_is_temporal``: optional [B,H] flags; slices flagged 0 are copied as-is."""
    if not 1 <= len(srcs) <= 3 or len(srcs) != len(dsts):
        raise ValueError("permute takes 1 to 3 (src, dst) pairs")
    _check_device(*srcs, *dsts)
    ref = srcs[0]
    for t in (*srcs, *dsts):
        if t.shape != ref.shape or t.dtype != ref.dtype:
            raise ValueError("all tensors must share shape and dtype")
    B, H, S, D = ref.shape
    if S != context_length + num_frame * frame_size:
        raise ValueError(f"seq_len {S} != {context_length} + {num_frame} * {frame_size}")
    flags = None
    if head_is_temporal is not None:
        flags = head_is_temporal.to(device=ref.device, dtype=torch.int32).reshape(B * H).contiguous()
    p = [t.data_ptr() for t in srcs] + [None] * (3 - len(srcs))
    d = [t.data_ptr() for t in dsts] + [None] * (3 - len(dsts))
    _lib.call("pasa_permute", p[0], p[1], p[2], d[0], d[1], d[2], len(srcs), B * H, num_frame,
              frame_size, context_length, D, _DTYPES.get(ref.dtype, -1),
              None if flags is None else flags.data_ptr(), int(bool(inverse)), _stream(ref))


def hunyuan_token_reorder_to_token_major(tensor, fix_len, reorder_len, reorder_num_frame, frame_size):
    """Reorder from frame major to token major, in place (reference :6-17)."""
    assert reorder_len == reorder_num_frame * frame_size
    assert tensor.shape[2] == fix_len + reorder_len
    out = torch.empty_like(tensor)
    permute([tensor], [out], reorder_num_frame, frame_size, fix_len, inverse=False)
    tensor.copy_(out)
    return tensor


def hunyuan_token_reorder_to_frame_major(tensor, fix_len, reorder_len, reorder_num_frame, frame_size):
    """Reorder from token major to frame major, in place (reference :20-31)."""
    assert reorder_len == reorder_num_frame * frame_size
    assert tensor.shape[2] == fix_len + reorder_len
    out = torch.empty_like(tensor)
    permute([tensor], [out], reorder_num_frame, frame_size, fix_len, inverse=True)
    tensor.copy_(out)
    return tensor


def hunyuan_sparse_head_placement(query, key, value, query_out, key_out, value_out, best_mask_idx,
                                  context_length, num_frame, frame_size):
    """Q/K/V to token-major for heads with best_mask_idx == 1 (reference :124-153)."""
    permute([query, key, value], [query_out, key_out, value_out], num_frame, frame_size,
            context_length, inverse=False, head_is_temporal=best_mask_idx)


def hunyuan_hidden_states_placement(hidden_states, hidden_states_out, best_mask_idx, context_length,
                                    num_frame, frame_size):
    """O back to frame-major for heads with best_mask_idx == 1 (reference :360-387)."""
    permute([hidden_states], [hidden_states_out], num_frame, frame_size, context_length,
            inverse=True, head_is_temporal=best_mask_idx)
    return hidden_states_out
