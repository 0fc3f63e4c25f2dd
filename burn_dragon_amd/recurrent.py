"""Recurrent linear-attention forward: the reference's Burn custom-op surface
(crates/burn_dragon_kernel/src/recurrent.rs, re-exported as
``burn_dragon_kernel::api::recurrent``, lib.rs:50-56) over libbdh_hip.

Tensors are torch tensors on the HIP device; torch only provides device memory
and the stream.  Every op returns ``None`` where the reference returns ``None``
(unsupported backend, zero dims, value heads not in {1, H}, batch/time
mismatch, plan mismatch) so that callers fall back exactly as
``DragonModel::recurrent_attention_with_plan`` does
(crates/burn_dragon_core/src/model/dragon/sequence_dispatch.rs:109-135).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import NamedTuple, Optional

import torch

from . import _lib

DEFAULT_ROPE_THETA = 65536.0  # FusedKernelConfig::rope_theta (config.rs:79)


class RecurrentAttentionOutput(NamedTuple):
    """recurrent.rs:65-69: context [B,H,T,D], rho [B,H,N,D]."""
    context: torch.Tensor
    rho: torch.Tensor


@dataclass(frozen=True)
class CompiledRecurrentAttentionPlan:
    """recurrent.rs:95-149.  Integer shape plan; nothing is uploaded."""
    batch: int
    heads: int
    value_heads: int
    time: int
    latent: int
    embd: int

    @classmethod
    def new(cls, batch, heads, value_heads, time, latent, embd, device=None):
        return cls(int(batch), int(heads), int(value_heads), int(time), int(latent), int(embd))

    def matches(self, query: torch.Tensor, value: torch.Tensor) -> bool:
        return (tuple(query.shape) == (self.batch, self.heads, self.time, self.latent)
                and tuple(value.shape) == (self.batch, self.value_heads, self.time, self.embd))

    def c_plan(self) -> Optional[_lib.BdhRecurrentPlan]:
        p = _lib.BdhRecurrentPlan()
        st = _lib.load().bdh_recurrent_plan_new(self.batch, self.heads, self.value_heads,
                                                self.time, self.latent, self.embd,
                                                ctypes.byref(p))
        return p if _lib.check(st) else None


def default_alibi_slopes(n_head: int) -> list:
    """linear_attention::default_alibi_slopes (kernel/linear_attention.rs:149-160):
    slope_h = 1 / 2^(h / n_head), in f32."""
    import numpy as np
    return [float(np.float32(1.0) / np.power(np.float32(2.0), np.float32(h) / np.float32(n_head)))
            for h in range(n_head)]


def alibi_decay(slopes) -> "torch.Tensor":
    """Per-head decay exp(-slope) of the ALiBi variant (attention.rs:201-208), f32 on
    the CPU; pass it (on the device) as ``decay`` with ``rho`` the layer's state and
    no RoPE (the ALiBi arm's frequencies are 0, attention.rs:569)."""
    import numpy as np
    return torch.from_numpy(np.exp(-np.asarray(slopes, np.float32)).astype(np.float32))


def supports_backend() -> bool:
    """recurrent.rs:151-173 (exported as supports_recurrent_backend)."""
    if not torch.cuda.is_available():
        return False
    return bool(_lib.load().bdh_supports_backend())


supports_recurrent_backend = supports_backend


def _dtype_code(t: torch.Tensor) -> Optional[int]:
    if t.dtype == torch.float32:
        return _lib.BDH_F32
    if t.dtype == torch.bfloat16:
        return _lib.BDH_BF16
    return None


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _on_device(*ts) -> bool:
    return all(t is None or (t.is_cuda) for t in ts)


def _shape_ok(query, value):
    if query.dim() != 4 or value.dim() != 4:
        return None
    B, H, T, N = query.shape
    Bv, Hv, Tv, D = value.shape
    if min(B, H, T, N, D) == 0:
        return None
    if Bv != B or Tv != T or Hv not in (1, H):
        return None
    return B, H, Hv, T, N, D


def _prepare(query, value, rho, decay, plan):
    if not supports_backend() or not _on_device(query, value, rho, decay):
        return None
    dims = _shape_ok(query, value)
    if dims is None:
        return None
    B, H, Hv, T, N, D = dims
    if plan is None:
        plan = CompiledRecurrentAttentionPlan(B, H, Hv, T, N, D)
    elif not plan.matches(query, value):
        return None
    code = _dtype_code(query)
    if code is None or value.dtype != query.dtype:
        return None
    # recurrent.rs:243-250: wrong-shaped rho -> zeros, wrong-shaped decay -> ones.
    if rho is not None and tuple(rho.shape) != (B, H, N, D):
        rho = None
    if decay is not None and tuple(decay.shape) != (H,):
        decay = None
    q = query.contiguous()
    v = value.contiguous()
    r = rho.to(torch.float32).contiguous() if rho is not None else None
    d = decay.to(torch.float32).contiguous() if decay is not None else None
    return plan, code, q, v, r, d, (B, H, Hv, T, N, D)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def try_fused_recurrent_attention_with_plan(query, value, rho=None, decay=None, plan=None,
                                            *, inplace: bool = False, chunk: int = 0
                                            ) -> Optional[RecurrentAttentionOutput]:
    """recurrent.rs:221-359.  ``query`` is the rotated query [B,H,T,N]
    (f32 or bf16), ``value`` [B,Hv,T,D] of the same dtype.  The caller's rho
    is never written unless ``inplace`` (the reference's private copy,
    recurrent.rs:259)."""
    prep = _prepare(query, value, rho, decay, plan)
    if prep is None:
        return None
    plan, code, q, v, r, d, (B, H, Hv, T, N, D) = prep
    cplan = plan.c_plan()
    if cplan is None:
        return None
    ctx = torch.empty((B, H, T, D), device=q.device, dtype=torch.float32)
    if inplace and r is not None and r.data_ptr() == rho.data_ptr():
        rho_out = r
    else:
        rho_out = torch.empty((B, H, N, D), device=q.device, dtype=torch.float32)
    st = _lib.load().bdh_recurrent_attention_fwd(
        ctypes.byref(cplan), code, _ptr(q), _ptr(v), _ptr(r), _ptr(d), _ptr(ctx), _ptr(rho_out),
        chunk, ctypes.c_void_p(_stream_ptr(q.device)))
    if not _lib.check(st):
        return None
    return RecurrentAttentionOutput(ctx, rho_out)


def try_fused_recurrent_attention(query, value, rho=None, decay=None, **kw
                                  ) -> Optional[RecurrentAttentionOutput]:
    """recurrent.rs:175-219 (plan built per call)."""
    return try_fused_recurrent_attention_with_plan(query, value, rho, decay, None, **kw)


# The reference's exported names (the ``_wgpu`` suffix is historical there).
try_fused_recurrent_attention_wgpu = try_fused_recurrent_attention
try_fused_recurrent_attention_wgpu_with_plan = try_fused_recurrent_attention_with_plan


def try_fused_recurrent_attention_rope(x, value, rho=None, decay=None, *, position: int = 0,
                                       fixed: bool = False, theta: float = DEFAULT_ROPE_THETA,
                                       plan=None, inplace: bool = False, chunk: int = 0
                                       ) -> Optional[RecurrentAttentionOutput]:
    """RoPE-fused variant: ``x`` is the unrotated activation.  Equivalent to
    rotate_positions (fixed=False) / rotate_positions_fixed (fixed=True) at
    ``position`` followed by try_fused_recurrent_attention_with_plan
    (sequence_dispatch.rs:97-124)."""
    prep = _prepare(x, value, rho, decay, plan)
    if prep is None:
        return None
    plan, code, q, v, r, d, (B, H, Hv, T, N, D) = prep
    cplan = plan.c_plan()
    if cplan is None:
        return None
    rope = _lib.BdhRope(_lib.BDH_ROPE_FIXED if fixed else _lib.BDH_ROPE_SEQUENTIAL, 0,
                        int(position), float(theta))
    ctx = torch.empty((B, H, T, D), device=q.device, dtype=torch.float32)
    if inplace and r is not None and r.data_ptr() == rho.data_ptr():
        rho_out = r
    else:
        rho_out = torch.empty((B, H, N, D), device=q.device, dtype=torch.float32)
    st = _lib.load().bdh_recurrent_attention_rope_fwd(
        ctypes.byref(cplan), code, _ptr(q), _ptr(v), _ptr(r), _ptr(d), ctypes.byref(rope),
        _ptr(ctx), _ptr(rho_out), chunk, ctypes.c_void_p(_stream_ptr(q.device)))
    if not _lib.check(st):
        return None
    return RecurrentAttentionOutput(ctx, rho_out)


@dataclass
class KernelProfileSnapshot:
    """profiling.rs:3-16."""
    calls: int
    launches: int
    total_ns: int
    setup_ns: int
    copy_ns: int
    dispatch_ns: int
    transient_allocations: int
    metadata_upload_bytes: int
    metadata_reuse_hits: int
    metadata_reuse_bytes: int
    resident_rollout_steps: int


RecurrentProfileSnapshot = KernelProfileSnapshot


def recurrent_profile_enable(enabled: bool = True) -> None:
    _lib.load().bdh_profile_enable(1 if enabled else 0)


def recurrent_profile_reset() -> None:
    """recurrent.rs:57-59."""
    _lib.load().bdh_profile_reset()


def recurrent_profile_snapshot() -> KernelProfileSnapshot:
    """recurrent.rs:61-63."""
    s = _lib.BdhProfileSnapshot()
    _lib.load().bdh_profile_get(ctypes.byref(s))
    return KernelProfileSnapshot(*[getattr(s, f) for f, _ in s._fields_])


def release_stream_scratch(stream: "torch.cuda.Stream | None" = None) -> None:
    """Frees the scratch the library keeps for `stream` (default: the current
    stream) on the current device, after the stream's queued work.  Call it
    before a stream is dropped, and only after every graph captured on it that
    calls this library has been destroyed: the sets are GB-scale at long
    shapes.  No counterpart in the reference (Burn's allocator owns its
    buffers)."""
    s = stream if stream is not None else torch.cuda.current_stream()
    st = _lib.load().bdh_scratch_release(ctypes.c_void_p(s.cuda_stream))
    if st != _lib.BDH_OK:
        raise _lib.BdhError(f"bdh_scratch_release: {_lib.last_error()}")
