"""Low-rank BDH layer body around the recurrent attention (bf16 MFMA, fp32
accumulation): lowrank_residual_step_impl of
crates/burn_dragon_core/src/model/residual_stream.rs:323-572, dropout off,
with its ReLU threshold th and sparse latent mask (default none):

    x    = ReLU(cur E_h - th) * mask                  [B, H, T, N]
    a    = LN(recurrent_attention(rope(x), cur))      [B, H, T, D]
    y    = (ReLU(a Ev_h - th) * mask) * x
    next = LN(cur + LN(y' Dec)),  y' = [B*T, H*N]      [B, T, D]

LN is DragonNorm's LayerNorm arm (gamma 1, beta 0, eps 1e-5, biased
variance; norm.rs:302-328).  Weights are packed once per weight set
(``LowRankWeights.pack``); the model shares them across layers
(dragon.rs:3358).
"""
from __future__ import annotations

import ctypes
from typing import NamedTuple, Optional

import torch

from . import _lib
from .recurrent import DEFAULT_ROPE_THETA, _ptr, _stream_ptr, supports_backend


class LowRankWeights(NamedTuple):
    encoder: torch.Tensor      # packed [H, N, D] bf16
    encoder_v: torch.Tensor    # packed [H, N, D] bf16
    decoder: torch.Tensor      # packed chunk-major [H*N/128, D, 128] bf16
    heads: int
    latent: int
    embd: int

    @staticmethod
    def pack(encoder: torch.Tensor, encoder_v: torch.Tensor, decoder: torch.Tensor
             ) -> Optional["LowRankWeights"]:
        """encoder, encoder_v [1,H,D,N] or [H,D,N] f32, decoder [H*N, D] f32
        (the reference's parameter layouts).  None where unsupported."""
        if not supports_backend():
            return None
        enc = encoder.reshape(encoder.shape[-3:]) if encoder.dim() == 4 else encoder
        encv = encoder_v.reshape(encoder_v.shape[-3:]) if encoder_v.dim() == 4 else encoder_v
        if enc.dim() != 3 or tuple(encv.shape) != tuple(enc.shape) or decoder.dim() != 2:
            return None
        H, D, N = enc.shape
        if tuple(decoder.shape) != (H * N, D):
            return None
        if any(t.dtype != torch.float32 or not t.is_cuda for t in (enc, encv, decoder)):
            return None
        dev = enc.device
        ep = torch.empty((H, N, D), device=dev, dtype=torch.bfloat16)
        evp = torch.empty((H, N, D), device=dev, dtype=torch.bfloat16)
        if (H * N) % 128:
            return None
        dp = torch.empty((H * N // 128, D, 128), device=dev, dtype=torch.bfloat16)
        # contiguous copies stay referenced until the launch is enqueued
        enc_c, encv_c, dec_c = enc.contiguous(), encv.contiguous(), decoder.contiguous()
        st = _lib.load().bdh_lowrank_pack_weights(
            H, N, D, _ptr(enc_c), _ptr(encv_c), _ptr(dec_c), _ptr(ep), _ptr(evp), _ptr(dp),
            ctypes.c_void_p(_stream_ptr(dev)))
        if not _lib.check(st):
            return None
        return LowRankWeights(ep, evp, dp, H, N, D)


class LowRankLayerOutput(NamedTuple):
    next: torch.Tensor             # [B, T, D] f32
    rho: Optional[torch.Tensor]    # [B, H, N, D] f32 when requested


def lowrank_layer_forward(current: torch.Tensor, weights: LowRankWeights, *,
                          position: Optional[int] = 0, theta: float = DEFAULT_ROPE_THETA,
                          want_rho: bool = False, out: Optional[torch.Tensor] = None,
                          rho: Optional[torch.Tensor] = None, inplace: bool = False,
                          relu_threshold: float = 0.0, latent_mask: Optional[torch.Tensor] = None
                          ) -> Optional[LowRankLayerOutput]:
    """current [B,1,T,D] or [B,T,D] f32 on the device; ``position`` is the
    first token's RoPE position (None: no rotation).  ``rho`` [B,H,N,D] f32
    is the layer's carried state (None: zeros).  With ``inplace`` the
    successor state is written over ``rho`` (the model's per-layer state;
    a single token then takes the sparse decode step); otherwise it is
    returned in a new tensor when ``want_rho``.  ``relu_threshold`` is the
    config's relu_threshold (config.rs:64) and ``latent_mask`` the sparse
    latent mask ([N] or the reference's [1,1,1,N] f32, e.g.
    BlockPattern1d::mask), both applied in the two projections as
    relu_lowrank.rs reference_forward does.  Returns None where the library
    does not support the shape."""
    if not supports_backend() or weights is None:
        return None
    cur = current.reshape(current.shape[0], current.shape[-2], current.shape[-1])
    if cur.dtype != torch.float32 or not cur.is_cuda:
        return None
    B, T, D = cur.shape
    if D != weights.embd:
        return None
    H, N = weights.heads, weights.latent
    cur = cur.contiguous()
    if rho is not None:
        if (tuple(rho.shape) != (B, H, N, D) or rho.dtype != torch.float32 or not rho.is_cuda
                or (inplace and not rho.is_contiguous())):
            return None
        rho_in = rho.contiguous()
    elif inplace:
        return None
    else:
        rho_in = None
    nxt = out if out is not None else torch.empty((B, T, D), device=cur.device, dtype=torch.float32)
    if inplace:
        rho_out = rho_in
    elif want_rho:
        rho_out = torch.empty((B, H, N, D), device=cur.device, dtype=torch.float32)
    else:
        rho_out = None
    mask = None
    if latent_mask is not None:
        mask = latent_mask.reshape(-1)
        if mask.numel() != N or mask.dtype != torch.float32 or not mask.is_cuda:
            return None
        mask = mask.contiguous()
    plan = _lib.BdhLayerPlan(B, H, T, N, D)
    rope = None
    if position is not None:
        rope = _lib.BdhRope(_lib.BDH_ROPE_SEQUENTIAL, 0, int(position), float(theta))
    opts = _lib.BdhLayerOptions(float(relu_threshold), 0, _ptr(mask))
    st = _lib.load().bdh_lowrank_layer_fwd_ex(
        ctypes.byref(plan), _ptr(cur), _ptr(weights.encoder), _ptr(weights.encoder_v),
        _ptr(weights.decoder), ctypes.byref(rope) if rope else None, _ptr(rho_in), _ptr(nxt),
        _ptr(rho_out), ctypes.byref(opts), ctypes.c_void_p(_stream_ptr(cur.device)))
    if not _lib.check(st):
        return None
    return LowRankLayerOutput(nxt, rho_out)
