"""Backward (VJP) of the attention with respect to its context output, fp32,
over libbdh_hip: the reference's
``dense_causal_attention_vjp[_with_initial_rho]``
(crates/burn_dragon_kernel/src/dense_causal_attention/backward_runtime.rs:
1-148) and the recurrent attention's backward
(crates/burn_dragon_kernel/src/recurrent/backward_runtime.rs), which share one
closed form (Q = K = query):

  ctx       = tril(-1)(Q Q^T * d^(r-c)) V + (Q * d^t) rho0
  grad_q    = (W + W^T) Q + (G rho0^T) * d^t,  W = tril(-1)(G V^T) * d^(r-c)
  grad_v    = S^T G (summed over heads for shared values), S = tril(-1)(Q Q^T) * d^(r-c)
  grad_d    = sum(tril(-1)(G V^T) * gap * S) / d  (+ the state term)
  grad_rho0 = (Q * d^t)^T G

The reference computes these in f32; so does this path, at any T (past 1024
tokens as intervals with a reverse scan of the state gradient).  ``None`` is
returned where the reference's fused path does not apply (non-f32, not on a
supported device, mismatched shapes), as the forward ops do.
"""
from __future__ import annotations

import ctypes
from typing import NamedTuple, Optional

import torch

from . import _lib
from .recurrent import CompiledRecurrentAttentionPlan, _ptr, _stream_ptr, supports_backend


class DenseCausalAttentionVjp(NamedTuple):
    """backward_runtime.rs:5-14."""
    grad_query: torch.Tensor
    grad_value: torch.Tensor
    grad_decay: torch.Tensor
    grad_initial_rho: Optional[torch.Tensor]


class RecurrentAttentionGrads(NamedTuple):
    """Gradients of the recurrent attention's inputs (query, value, rho,
    decay) with respect to its context."""
    grad_query: torch.Tensor
    grad_value: torch.Tensor
    grad_rho: Optional[torch.Tensor]
    grad_decay: torch.Tensor


def _prep(grad_output, query, value, decay, rho):
    if not supports_backend():
        return None
    ts = [t for t in (grad_output, query, value, decay, rho) if t is not None]
    if any((not t.is_cuda) or t.dtype != torch.float32 for t in ts):
        return None
    if query.dim() != 4 or value.dim() != 4 or grad_output.dim() != 4:
        return None
    B, H, T, N = query.shape
    Bv, Hv, Tv, D = value.shape
    if min(B, H, T, N, D) == 0 or Bv != B or Tv != T or Hv not in (1, H):
        return None
    if tuple(grad_output.shape) != (B, H, T, D):
        return None
    if decay is not None and tuple(decay.shape) != (H,):
        return None
    if rho is not None and tuple(rho.shape) != (B, H, N, D):
        return None
    plan = CompiledRecurrentAttentionPlan(B, H, Hv, T, N, D).c_plan()
    if plan is None:
        return None
    c = lambda t: t.contiguous() if t is not None else None  # noqa: E731
    return plan, (B, H, Hv, T, N, D), c(grad_output), c(query), c(value), c(decay), c(rho)


def dense_causal_attention_vjp_with_initial_rho(grad_output, query, value, decay, initial_rho=None
                                                ) -> Optional[DenseCausalAttentionVjp]:
    """backward_runtime.rs:36-148."""
    prep = _prep(grad_output, query, value, decay, initial_rho)
    if prep is None:
        return None
    plan, (B, H, Hv, T, N, D), g, q, v, d, r = prep
    dev = q.device
    gq = torch.empty((B, H, T, N), device=dev, dtype=torch.float32)
    gv = torch.empty((B, Hv, T, D), device=dev, dtype=torch.float32)
    gd = torch.empty((H,), device=dev, dtype=torch.float32)
    gr = torch.empty((B, H, N, D), device=dev, dtype=torch.float32) if r is not None else None
    st = _lib.load().bdh_dense_causal_attention_vjp(
        ctypes.byref(plan), _ptr(q), _ptr(v), _ptr(d), _ptr(r), _ptr(g), _ptr(gq), _ptr(gv), _ptr(gd),
        _ptr(gr), ctypes.c_void_p(_stream_ptr(dev)))
    if not _lib.check(st):
        return None
    return DenseCausalAttentionVjp(gq, gv, gd, gr)


def dense_causal_attention_vjp(grad_output, query, value, decay) -> Optional[DenseCausalAttentionVjp]:
    """backward_runtime.rs:16-27."""
    return dense_causal_attention_vjp_with_initial_rho(grad_output, query, value, decay, None)


def recurrent_attention_vjp(grad_context, query, value, rho=None, decay=None
                            ) -> Optional[RecurrentAttentionGrads]:
    """The backward of try_fused_recurrent_attention with respect to its
    context (recurrent/backward_runtime.rs:336-502, 1155-1239): gradients of
    query, value, the incoming rho (None when rho is None: zeros) and decay
    (ones when None).  The outgoing rho is not differentiated, as in the
    reference (its rho output is not tracked)."""
    prep = _prep(grad_context, query, value, decay, rho)
    if prep is None:
        return None
    plan, (B, H, Hv, T, N, D), g, q, v, d, r = prep
    dev = q.device
    gq = torch.empty((B, H, T, N), device=dev, dtype=torch.float32)
    gv = torch.empty((B, Hv, T, D), device=dev, dtype=torch.float32)
    gd = torch.empty((H,), device=dev, dtype=torch.float32)
    gr = torch.empty((B, H, N, D), device=dev, dtype=torch.float32) if r is not None else None
    st = _lib.load().bdh_recurrent_attention_vjp(
        ctypes.byref(plan), _ptr(q), _ptr(v), _ptr(r), _ptr(d), _ptr(g), _ptr(gq), _ptr(gv), _ptr(gr),
        _ptr(gd), ctypes.c_void_p(_stream_ptr(dev)))
    if not _lib.check(st):
        return None
    return RecurrentAttentionGrads(gq, gv, gr, gd)
