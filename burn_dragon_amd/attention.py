"""Dense causal attention (no state): the reference's
``burn_dragon_kernel::api::attention`` surface
(crates/burn_dragon_kernel/src/dense_causal_attention.rs:77-261) over
libbdh_hip:  ctx = tril(-1)(Q Q^T * decay^(r-c)) V.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from .recurrent import (CompiledRecurrentAttentionPlan, _dtype_code, _on_device, _ptr,
                        _shape_ok, _stream_ptr, supports_backend)

MAX_FUSED_TIME = 1024  # dense_causal_attention.rs:44


@dataclass(frozen=True)
class CompiledDenseCausalAttentionPlan(CompiledRecurrentAttentionPlan):
    """dense_causal_attention.rs:77-132 (value_dim == embd)."""


def supports_dense_causal_attention_backend() -> bool:
    """dense_causal_attention.rs:134-160."""
    return supports_backend()


def try_fused_dense_causal_attention_with_plan(query, value, decay, plan=None
                                               ) -> Optional[torch.Tensor]:
    """dense_causal_attention.rs:200-261."""
    if not supports_backend() or not _on_device(query, value, decay):
        return None
    dims = _shape_ok(query, value)
    if dims is None:
        return None
    B, H, Hv, T, N, D = dims
    if T > MAX_FUSED_TIME:
        return None
    if plan is None:
        plan = CompiledDenseCausalAttentionPlan(B, H, Hv, T, N, D)
    elif not plan.matches(query, value):
        return None
    if decay is None or tuple(decay.shape) != (H,):
        return None
    code = _dtype_code(query)
    if code is None or value.dtype != query.dtype:
        return None
    q = query.contiguous()
    v = value.contiguous()
    d = decay.to(torch.float32).contiguous()
    cplan = plan.c_plan()
    if cplan is None:
        return None
    ctx = torch.empty((B, H, T, D), device=q.device, dtype=torch.float32)
    st = _lib.load().bdh_dense_causal_attention_fwd(
        ctypes.byref(cplan), code, _ptr(q), _ptr(v), _ptr(d), _ptr(ctx),
        ctypes.c_void_p(_stream_ptr(q.device)))
    return ctx if _lib.check(st) else None


def try_fused_dense_causal_attention(query, value, decay) -> Optional[torch.Tensor]:
    """dense_causal_attention.rs:162-198."""
    return try_fused_dense_causal_attention_with_plan(query, value, decay, None)


try_fused_dense_causal_attention_wgpu = try_fused_dense_causal_attention
try_fused_dense_causal_attention_wgpu_with_plan = try_fused_dense_causal_attention_with_plan
