"""Sparse decode step: one token per stream through the recurrent attention
with RoPE fused (the T = 1 call that the reference's decode drivers make per
generated token: dragon.rs:1749-1808, generation.rs:458 ->
sequence_dispatch.rs:83-136 -> linear.rs:43-57).

Only the active rows of rho are read and written; the active set is
returned bit-exactly on request.
"""
from __future__ import annotations

import ctypes
from typing import NamedTuple, Optional

import torch

from . import _lib
from .recurrent import DEFAULT_ROPE_THETA, _ptr, _stream_ptr, supports_backend


class DecodeOutput(NamedTuple):
    readout: torch.Tensor                   # a [B, H, D] f32
    active_idx: Optional[torch.Tensor]      # [B, H, N] int32, ascending, -1 padded
    active_cnt: Optional[torch.Tensor]      # [B, H] int32


def decode_step(x: torch.Tensor, value: torch.Tensor, rho: torch.Tensor, *,
                position: Optional[int] = 0, theta: float = DEFAULT_ROPE_THETA,
                decay: Optional[torch.Tensor] = None, want_active: bool = False,
                out: Optional[torch.Tensor] = None) -> Optional[DecodeOutput]:
    """x [B,H,N] f32 (unrotated; ``position=None`` means already rotated),
    value [B,Hv,D] f32, rho [B,H,N,D] f32 updated IN PLACE,
    rho = (rho + rot(x)^T v) * decay.  ``decay`` [H] f32 (ALiBi, exp(-slope):
    attention.rs:201-208) scales every row, so the step streams all of rho;
    without it only the active rows are touched.  Returns None where the
    reference would (zero dims, value heads not in {1,H}, non-f32, not on a
    supported device)."""
    if not supports_backend():
        return None
    if not (x.is_cuda and value.is_cuda and rho.is_cuda):
        return None
    if x.dim() != 3 or value.dim() != 3 or rho.dim() != 4:
        return None
    B, H, N = x.shape
    Bv, Hv, D = value.shape
    if Bv != B or Hv not in (1, H) or tuple(rho.shape) != (B, H, N, D):
        return None
    if any(t.dtype != torch.float32 for t in (x, value, rho)):
        return None
    if decay is not None:
        # recurrent.rs:247-250: a wrong-shaped decay means ones
        if not decay.is_cuda or tuple(decay.shape) != (H,):
            decay = None
        else:
            decay = decay.to(torch.float32).contiguous()
    if not rho.is_contiguous():
        raise ValueError("decode_step updates rho in place: it must be contiguous")
    xc = x.contiguous()
    vc = value.contiguous()
    a = out if out is not None else torch.empty((B, H, D), device=x.device, dtype=torch.float32)
    idx = torch.empty((B, H, N), device=x.device, dtype=torch.int32) if want_active else None
    cnt = torch.empty((B, H), device=x.device, dtype=torch.int32) if want_active else None
    rope = None
    if position is not None:
        rope = _lib.BdhRope(_lib.BDH_ROPE_SEQUENTIAL, 0, int(position), float(theta))
    st = _lib.load().bdh_decode_step(
        B, H, Hv, N, D, _ptr(xc), _ptr(vc), _ptr(rho), _ptr(decay),
        ctypes.byref(rope) if rope else None,
        _ptr(a), _ptr(idx), _ptr(cnt), ctypes.c_void_p(_stream_ptr(x.device)))
    if not _lib.check(st):
        return None
    return DecodeOutput(a, idx, cnt)
