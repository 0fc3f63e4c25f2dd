"""BDH language-model forward with low-rank weights shared across layers
(the vanilla residual connector): DragonModel's sequence forward
(crates/burn_dragon_core/src/model/dragon.rs:3340-3420, weights shared at
:3358) and project_hidden_to_logits (:4033-4055):

    current = LN(embed[tokens])                          (:3352)
    current = lowrank_layer(current)   for each layer    (residual_stream.rs:323-572)
    logits  = current @ lm_head

Every step runs in libbdh_hip.so (bdh_embed_norm, bdh_lowrank_layer_fwd,
bdh_lm_logits); torch only owns the device buffers.

With a ``BdhModelState`` (ModelState: one rho per layer and the next
position, state.rs:7-30, dragon.rs:3334) the forward continues a sequence:
each layer's attention starts from its own rho and writes the successor
over it, all layers at positions state.position.., and the position then
advances by T (forward_hidden_with_state..., dragon.rs:3338-3446).  A
prompt is one such call; each generated token is another with T = 1,
which takes the sparse decode step (the generation loop of
generation.rs:458 / dragon.rs:1749-1808).
"""
from __future__ import annotations

import ctypes
from typing import NamedTuple, Optional

import torch

from . import _lib
from .layer import LowRankWeights, lowrank_layer_forward
from .recurrent import DEFAULT_ROPE_THETA, _ptr, _stream_ptr, supports_backend


class BdhModelState:
    """Per-layer recurrent state rho [n_layer][B, H, N, D] f32 (zeros at the
    start of a sequence) and the position of the next token."""

    def __init__(self, n_layer: int, batch: int, heads: int, latent: int, embd: int,
                 device: torch.device, position: int = 0):
        self.rho = [torch.zeros((batch, heads, latent, embd), device=device, dtype=torch.float32)
                    for _ in range(n_layer)]
        self.position = int(position)


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


def new_model_state(weights: BdhModelWeights, batch: int, device: torch.device,
                    position: int = 0) -> BdhModelState:
    return BdhModelState(weights.n_layer, batch, weights.layer.heads, weights.layer.latent,
                         weights.layer.embd, device, position)


def model_forward_logits(tokens: torch.Tensor, weights: BdhModelWeights, *,
                         position: Optional[int] = 0, theta: float = DEFAULT_ROPE_THETA,
                         state: Optional[BdhModelState] = None) -> Optional[torch.Tensor]:
    """tokens [B, T] int32 on the device -> logits [B, T, vocab] f32.
    Without ``state`` every layer starts from rho = 0 at ``position``; with
    it the forward continues the state's sequence (its position wins) and
    updates the state in place."""
    if not supports_backend() or weights is None:
        return None
    if state is not None:
        if len(state.rho) != weights.n_layer:
            return None
        position = state.position
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
    for layer in range(weights.n_layer):
        rho = state.rho[layer] if state is not None else None
        out = lowrank_layer_forward(cur, weights.layer, position=position, theta=theta, out=nxt,
                                    rho=rho, inplace=state is not None)
        if out is None:
            return None
        cur, nxt = nxt, cur
    logits = torch.empty((B, T, weights.vocab), device=dev, dtype=torch.float32)
    st = lib.bdh_lm_logits(_ptr(cur), B * T, D, _ptr(weights.lm_head), weights.vocab,
                           _ptr(logits), stream)
    if not _lib.check(st):
        return None
    if state is not None:
        state.position += T
    return logits
