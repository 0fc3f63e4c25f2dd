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
                         state: Optional[BdhModelState] = None, relu_threshold: float = 0.0,
                         latent_mask: Optional[torch.Tensor] = None) -> Optional[torch.Tensor]:
    """tokens [B, T] int32 on the device -> logits [B, T, vocab] f32.
    Without ``state`` every layer starts from rho = 0 at ``position``; with
    it the forward continues the state's sequence (its position wins) and
    updates the state in place.  ``relu_threshold`` and ``latent_mask`` are
    every layer's projection options (lowrank_layer_forward)."""
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
                                    rho=rho, inplace=state is not None,
                                    relu_threshold=relu_threshold, latent_mask=latent_mask)
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


def save_model_state(path: str, state: BdhModelState, persist_sequence_state: bool = True,
                     retain_terminal_sequence_state: bool = True) -> None:
    """Writes the state's position and every layer's rho (a layer whose rho is
    None has no rho) to a state record (bdh_state_record_save; the
    StreamingRuntimeStateRecord of runtime_checkpoint.rs:16-112 for this
    path's state).  Raises on failure."""
    n = len(state.rho)
    descs = (_lib.BdhLayerStateDesc * max(n, 1))()
    ptrs = (ctypes.c_void_p * max(n, 1))()
    dev = None
    for i, r in enumerate(state.rho):
        if r is not None:
            if r.dtype != torch.float32 or not r.is_cuda or r.dim() != 4 or not r.is_contiguous():
                raise ValueError("rho must be a contiguous f32 [B,H,N,D] device tensor")
            descs[i].batch, descs[i].heads, descs[i].latent, descs[i].embd = r.shape
            ptrs[i] = r.data_ptr()
            dev = r.device
        descs[i].persist_sequence_state = int(persist_sequence_state)
        descs[i].retain_terminal_sequence_state = int(retain_terminal_sequence_state)
    stream = ctypes.c_void_p(_stream_ptr(dev)) if dev is not None else None
    st = _lib.load().bdh_state_record_save(str(path).encode(), int(state.position), n, descs, ptrs,
                                           stream)
    if st != _lib.BDH_OK:
        raise _lib.BdhError(f"bdh_state_record_save: {_lib.last_error()}")


def load_model_state(path: str, device: torch.device) -> BdhModelState:
    """Reads a state record into a new BdhModelState on `device` (rho None for
    layers recorded without one).  Raises on a corrupt or unreadable record."""
    lib = _lib.load()
    pos, n = ctypes.c_int64(), ctypes.c_int32()
    st = lib.bdh_state_record_info(str(path).encode(), ctypes.byref(pos), ctypes.byref(n), None, 0)
    if st != _lib.BDH_OK:
        raise _lib.BdhError(f"bdh_state_record_info: {_lib.last_error()}")
    descs = (_lib.BdhLayerStateDesc * max(n.value, 1))()
    st = lib.bdh_state_record_info(str(path).encode(), ctypes.byref(pos), ctypes.byref(n), descs,
                                   n.value)
    if st != _lib.BDH_OK:
        raise _lib.BdhError(f"bdh_state_record_info: {_lib.last_error()}")
    state = BdhModelState.__new__(BdhModelState)
    state.position = int(pos.value)
    state.rho = []
    ptrs = (ctypes.c_void_p * max(n.value, 1))()
    for i in range(n.value):
        d = descs[i]
        if d.batch == 0:
            state.rho.append(None)
            continue
        r = torch.empty((d.batch, d.heads, d.latent, d.embd), device=device, dtype=torch.float32)
        ptrs[i] = r.data_ptr()
        state.rho.append(r)
    st = lib.bdh_state_record_load(str(path).encode(), n.value, descs, ptrs,
                                   ctypes.c_void_p(_stream_ptr(device)))
    if st != _lib.BDH_OK:
        raise _lib.BdhError(f"bdh_state_record_load: {_lib.last_error()}")
    return state
