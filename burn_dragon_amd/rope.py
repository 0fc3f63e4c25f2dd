"""RoPE helpers on the host side of the boundary.

``rope_freqs`` returns the exact f32 table the kernels use
(Attention::build_freqs, attention.rs:552-576).  ``active_rows_mask`` is the
structural active set of the sparse decode step, evaluated with torch on the
device in the reference's f32 op order (attention.rs:544-546):
    i active  <=>  x_i != 0  or  (x_{i^1} != 0 and frac(p * f_i) != 0)
It is used to count the exact rows a decode step moves (byte accounting).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

DEFAULT_ROPE_THETA = 65536.0


def rope_freqs(latent: int, theta: float = DEFAULT_ROPE_THETA) -> np.ndarray:
    out = np.empty(int(latent), np.float32)
    st = _lib.load().bdh_rope_freqs(int(latent), float(theta),
                                    out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    if not _lib.check(st):
        raise ValueError(_lib.last_error())
    return out


def active_rows_mask(x, position: int, freqs):
    """x [..., N] torch f32 (unrotated), freqs torch f32 [N] on x's device."""
    import torch
    partner = x.view(*x.shape[:-1], -1, 2).flip(-1).reshape(x.shape)
    p = torch.tensor(float(position), dtype=torch.float32, device=x.device)
    raw = p * freqs
    frac_nonzero = (raw - torch.floor(raw)) != 0
    return (x != 0) | ((partner != 0) & frac_nonzero)
