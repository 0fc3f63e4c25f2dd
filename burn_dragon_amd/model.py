"""BDH language-model forward with low-rank weights shared across layers
(the vanilla residual connector): DragonModel's sequence forward
(crates/burn_dragon_core/src/model/dragon.rs:3340-3420, weights shared at
:3358) and project_hidden_to_logits (:4033-4055):

    current = LN(embed[tokens])                          (:3352)
    current = lowrank_layer(current)   for each layer    (residual_stream.rs:323-572)
    logits  = current @ lm_head

Every step runs in libbdh_hip.so (bdh_embed_norm, bdh_lowrank_layer_fwd,
bdh_lm_logits); torch only owns the device buffers.
"""
from __future__ import annotations

import ctypes
from typing import NamedTuple, Optional

import torch

from . import _lib
from .layer import LowRankWeights, lowrank_layer_forward
from .recurrent import DEFAULT_ROPE_THETA, _ptr, _stream_ptr, supports_backend


class BdhModelWeights(NamedTuple):
    embed: torch.Tensor          # [vocab, D] f32
    layer: LowRankWeights        # packed encoder / encoder_v / decoder
    lm_head: torch.Tensor        # packed [vocab, D] bf16
    vocab: int
    n_layer: int


def pack_model(embed: torch.Tensor, encoder: torch.Tensor, encoder_v: torch.Tensor,
               decoder: torch.Tensor, lm_head: torch.Tensor, n_layer: int
               ) -> Optional[BdhModelWeights]:
    """embed [vocab, D], encoder / encoder_v [1,H,D,N], decoder [H*N, D],
    lm_head [D, vocab], all f32 on the device (the reference's layouts)."""
    if not supports_backend():
        return None
    layer = LowRankWeights.pack(encoder, encoder_v, decoder)
    if layer is None or embed.dim() != 2 or lm_head.dim() != 2:
        return None
    V, D = embed.shape
    if D != layer.embd or lm_head.shape[0] != D:
        return None
    Vh = lm_head.shape[1]
    head_c = lm_head.contiguous()
    packed = torch.empty((Vh, D), device=embed.device, dtype=torch.bfloat16)
    st = _lib.load().bdh_lm_head_pack(D, Vh, _ptr(head_c), _ptr(packed),
                                      ctypes.c_void_p(_stream_ptr(embed.device)))
    if not _lib.check(st):
        return None
    return BdhModelWeights(embed.contiguous(), layer, packed, Vh, int(n_layer))


def model_forward_logits(tokens: torch.Tensor, weights: BdhModelWeights, *,
                         position: Optional[int] = 0, theta: float = DEFAULT_ROPE_THETA
                         ) -> Optional[torch.Tensor]:
    """tokens [B, T] int32 on the device -> logits [B, T, vocab] f32."""
    if not supports_backend() or weights is None:
        return None
    if tokens.dim() != 2 or tokens.dtype != torch.int32 or not tokens.is_cuda:
        return None
    B, T = tokens.shape
    D = weights.layer.embd
    dev = tokens.device
    stream = ctypes.c_void_p(_stream_ptr(dev))
    lib = _lib.load()
    tok = tokens.contiguous()
    cur = torch.empty((B, T, D), device=dev, dtype=torch.float32)
    nxt = torch.empty_like(cur)
    st = lib.bdh_embed_norm(_ptr(tok), B * T, _ptr(weights.embed), weights.embed.shape[0], D,
                            _ptr(cur), stream)
    if not _lib.check(st):
        return None
    for _ in range(weights.n_layer):
        out = lowrank_layer_forward(cur, weights.layer, position=position, theta=theta, out=nxt)
        if out is None:
            return None
        cur, nxt = nxt, cur
    logits = torch.empty((B, T, weights.vocab), device=dev, dtype=torch.float32)
    st = lib.bdh_lm_logits(_ptr(cur), B * T, D, _ptr(weights.lm_head), weights.vocab,
                           _ptr(logits), stream)
    if not _lib.check(st):
        return None
    return logits
