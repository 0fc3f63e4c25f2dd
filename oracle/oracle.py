"""numpy/ctypes front end of the CPU oracle (oracle/bdh_oracle.c).

TEST INFRASTRUCTURE ONLY.  tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of bench.py use it as the checker; nothing in the
product package imports it.  Each wrapper names the reference function the C
code restates (paths relative to the burn_dragon v0.21.8 checkout).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libbdh_oracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64 = ctypes.c_int64


def build() -> str:
    """Compile the oracle with its committed Makefile (gcc)."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.bdh_oracle_rope_freqs.argtypes = [_i64, ctypes.c_float, _f32p]
        L.bdh_oracle_rope_rotate.argtypes = [_f32p, _i64, _i64, _i64, _i64, ctypes.c_int32,
                                             ctypes.c_float, _f32p]
        L.bdh_oracle_active_rows.argtypes = [_f32p, _i64, _i64, _f32p, _i32p]
        L.bdh_oracle_active_rows.restype = ctypes.c_int32
        for name in ("bdh_oracle_recurrent_f32",):
            getattr(L, name).argtypes = [_f32p, _f32p, _f32p, _f32p] + [_i64] * 6 + [_f32p, _f32p]
        for name in ("bdh_oracle_recurrent_f64", "bdh_oracle_dense_score_f64"):
            getattr(L, name).argtypes = [_f32p, _f32p, _f32p, _f32p] + [_i64] * 6 + [_f64p, _f64p]
        L.bdh_oracle_decode_step_f32.argtypes = [_f32p, _f32p, _f32p] + [_i64] * 6 + [
            ctypes.c_float, _f32p, _i32p, _i32p]
        L.bdh_oracle_round_bf16.argtypes = [_f32p, _f32p, _i64]
        L.bdh_oracle_ndarray_recurrent_f32.argtypes = [_f32p, _f32p, _f32p, _f32p] + [_i64] * 6 + [
            _f32p, _f32p, ctypes.c_int32]
        L.bdh_oracle_ndarray_recurrent_f32.restype = ctypes.c_double
        L.bdh_oracle_ndarray_dense_f32.argtypes = [_f32p, _f32p] + [_i64] * 6 + [_f32p, ctypes.c_int32]
        L.bdh_oracle_ndarray_dense_f32.restype = ctypes.c_double
        _lib = L
    return _lib


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(_f32p)


def _opt_f32(a):
    if a is None:
        return None, None
    return _f32(a)


def rope_freqs(latent: int, theta: float = 65536.0) -> np.ndarray:
    """Attention::build_freqs, Rope arm (attention.rs:552-576)."""
    out = np.empty(latent, np.float32)
    lib().bdh_oracle_rope_freqs(latent, theta, out.ctypes.data_as(_f32p))
    return out


def rope_rotate(x, pos0: int = 0, mode: int = 0, theta: float = 65536.0) -> np.ndarray:
    """rotate_positions (mode 0) / rotate_positions_fixed (mode 1) on x[..., T, N]
    (attention.rs:339-349, 512-550, 488-501)."""
    x, xp = _f32(x)
    T, N = x.shape[-2], x.shape[-1]
    rows = x.size // (T * N)
    out = np.empty_like(x)
    lib().bdh_oracle_rope_rotate(xp, rows, T, N, pos0, mode, theta, out.ctypes.data_as(_f32p))
    return out


def active_rows(x_row, pos: int, theta: float = 65536.0) -> np.ndarray:
    """Structural active set {i : rot(x)_i not identically zero} at position pos."""
    x_row, xp = _f32(x_row)
    N = x_row.shape[-1]
    freqs = rope_freqs(N, theta)
    idx = np.empty(N, np.int32)
    cnt = lib().bdh_oracle_active_rows(xp, N, pos, freqs.ctypes.data_as(_f32p),
                                       idx.ctypes.data_as(_i32p))
    return idx[:cnt].copy()


def _dims(q, v):
    B, H, T, N = q.shape
    Bv, Hv, Tv, D = v.shape
    assert Bv == B and Tv == T and Hv in (1, H), (q.shape, v.shape)
    return B, H, Hv, T, N, D


def recurrent_f32(q, v, rho0=None, decay=None):
    """recurrent_attention_reference (linear.rs:18-60), op-for-op in f32."""
    q, qp = _f32(q)
    v, vp = _f32(v)
    rho0, rp = _opt_f32(rho0)
    decay, dp = _opt_f32(decay)
    B, H, Hv, T, N, D = _dims(q, v)
    ctx = np.empty((B, H, T, D), np.float32)
    rho = np.empty((B, H, N, D), np.float32)
    lib().bdh_oracle_recurrent_f32(qp, vp, rp, dp, B, H, Hv, T, N, D,
                                   ctx.ctypes.data_as(_f32p), rho.ctypes.data_as(_f32p))
    return ctx, rho


def recurrent_f64(q, v, rho0=None, decay=None):
    """The same recurrence carried in f64."""
    q, qp = _f32(q)
    v, vp = _f32(v)
    rho0, rp = _opt_f32(rho0)
    decay, dp = _opt_f32(decay)
    B, H, Hv, T, N, D = _dims(q, v)
    ctx = np.empty((B, H, T, D), np.float64)
    rho = np.empty((B, H, N, D), np.float64)
    lib().bdh_oracle_recurrent_f64(qp, vp, rp, dp, B, H, Hv, T, N, D,
                                   ctx.ctypes.data_as(_f64p), rho.ctypes.data_as(_f64p))
    return ctx, rho


def dense_score_f64(q, v, rho0=None, decay=None, want_ctx=True, want_rho=True):
    """Dense-score form (linear.rs:221-364) in f64."""
    q, qp = _f32(q)
    v, vp = _f32(v)
    rho0, rp = _opt_f32(rho0)
    decay, dp = _opt_f32(decay)
    B, H, Hv, T, N, D = _dims(q, v)
    ctx = np.empty((B, H, T, D), np.float64) if want_ctx else None
    rho = np.empty((B, H, N, D), np.float64) if want_rho else None
    lib().bdh_oracle_dense_score_f64(
        qp, vp, rp, dp, B, H, Hv, T, N, D,
        ctx.ctypes.data_as(_f64p) if ctx is not None else None,
        rho.ctypes.data_as(_f64p) if rho is not None else None)
    return ctx, rho


def decode_step_f32(x, v, rho, pos: int, theta: float = 65536.0):
    """One T=1 step with RoPE at pos (sequence_dispatch.rs:97-124 ->
    linear.rs:43-57).  rho [B,H,N,D] is updated in place (must be float32,
    C-contiguous).  Returns (a [B,H,D], active_idx [B,H,N], active_cnt [B,H])."""
    x, xp = _f32(x)
    v, vp = _f32(v)
    assert rho.dtype == np.float32 and rho.flags.c_contiguous
    B, H, N = x.shape
    Hv, D = v.shape[1], v.shape[2]
    a = np.empty((B, H, D), np.float32)
    idx = np.empty((B, H, N), np.int32)
    cnt = np.empty((B, H), np.int32)
    lib().bdh_oracle_decode_step_f32(xp, vp, rho.ctypes.data_as(_f32p), B, H, Hv, N, D, pos,
                                     theta, a.ctypes.data_as(_f32p), idx.ctypes.data_as(_i32p),
                                     cnt.ctypes.data_as(_i32p))
    return a, idx, cnt


def round_bf16(a) -> np.ndarray:
    """Round-to-nearest-even to bf16, returned as exact float32."""
    a, ap = _f32(a)
    out = np.empty_like(a)
    lib().bdh_oracle_round_bf16(ap, out.ctypes.data_as(_f32p), a.size)
    return out


def ndarray_recurrent_f32(q, v, rho0=None, decay=None, threads: int = 0):
    """CPU baseline: the NdArray op sequence of linear.rs:43-57 with
    materialised [N, D] temporaries, OpenMP over (b, h).  Returns
    (ctx, rho, wall_seconds)."""
    q, qp = _f32(q)
    v, vp = _f32(v)
    rho0, rp = _opt_f32(rho0)
    decay, dp = _opt_f32(decay)
    B, H, Hv, T, N, D = _dims(q, v)
    ctx = np.empty((B, H, T, D), np.float32)
    rho = np.empty((B, H, N, D), np.float32)
    secs = lib().bdh_oracle_ndarray_recurrent_f32(qp, vp, rp, dp, B, H, Hv, T, N, D,
                                                  ctx.ctypes.data_as(_f32p),
                                                  rho.ctypes.data_as(_f32p), threads)
    return ctx, rho, secs


def ndarray_dense_f32(q, v, threads: int = 0):
    """CPU baseline, dense-score form without state or decay: the NdArray op
    sequence of linear.rs:241, 321 ((Q Q^T).tril(-1) materialised, then
    scores V), fp32, OpenMP over (b, h).  Returns (ctx, wall_seconds)."""
    q, qp = _f32(q)
    v, vp = _f32(v)
    B, H, Hv, T, N, D = _dims(q, v)
    ctx = np.empty((B, H, T, D), np.float32)
    secs = lib().bdh_oracle_ndarray_dense_f32(qp, vp, B, H, Hv, T, N, D, ctx.ctypes.data_as(_f32p), threads)
    return ctx, secs


def layer_norm_f64(x, eps: float = 1e-5) -> np.ndarray:
    """DragonNorm::forward, LayerNorm arm with gamma = 1, beta = 0
    (crates/burn_dragon_core/src/model/norm.rs:302-328): (x - mean) /
    sqrt(var + eps) over the last axis, var the biased variance
    (var_mean_bias).  f64."""
    x = np.asarray(x, np.float64)
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps)


def decode_y_neuron_tail_f64(y, decoder) -> np.ndarray:
    """decode_y_neuron_tail (residual_stream.rs:309-321): y [B,H,T,N] ->
    swap_dims(1, 2) -> [B*T, H*N] @ decoder [H*N, D] -> [B,T,D]."""
    y = np.asarray(y, np.float64)
    B, H, T, N = y.shape
    dec = np.asarray(decoder, np.float64)
    return (y.transpose(0, 2, 1, 3).reshape(B * T, H * N) @ dec).reshape(B, T, dec.shape[1])


def lowrank_layer_f64(cur, encoder, encoder_v, decoder, pos0=0, theta: float = 65536.0,
                      rho0=None, relu_threshold: float = 0.0, latent_mask=None):
    """lowrank_residual_step_impl (residual_stream.rs:323-572), dropout off,
    with its ReLU threshold and sparse latent mask (relu_lowrank.rs
    reference_forward, kernel/relu_lowrank.rs:100-135: project, subtract the
    threshold, ReLU, times the mask; the layer passes no bias, :387-400,
    :443-456):
      x = ReLU(cur @ E_h - th) * mask                      (:377-410)
      attn = recurrent attention of rope(x) with value cur  (:398;
             sequence_dispatch.rs:97-111; linear.rs:18-60)
      attn = LN(attn)                                      (:422)
      y = x * (ReLU(attn @ Ev_h - th) * mask)              (:440-486)
      mlp = LN(decode_y_neuron_tail(y, Dec))               (:488, :499)
      next = LN(cur + mlp)                                 (:517)
    cur [B,T,D]; encoder, encoder_v [H,D,N]; decoder [H*N,D]; latent_mask
    [N] (BlockPattern1d::mask, block_sparse.rs:49-64, or any [N] mask) or
    None; pos0 None = no RoPE.  RoPE runs in the reference's f32 op order,
    everything else in f64.  Returns (next [B,T,D], rho [B,H,N,D])."""
    cur = np.asarray(cur, np.float64)
    enc = np.asarray(encoder, np.float64)
    encv = np.asarray(encoder_v, np.float64)
    mask = None if latent_mask is None else np.asarray(latent_mask, np.float64)
    x = np.maximum(np.matmul(cur[:, None], enc[None]) - relu_threshold, 0.0)  # [B,H,T,N]
    if mask is not None:
        x = x * mask
    q = rope_rotate(x.astype(np.float32), pos0=pos0, theta=theta) if pos0 is not None else x
    ctx, rho = recurrent_f64(q, cur[:, None].astype(np.float32), rho0)
    a = layer_norm_f64(ctx)
    gate = np.maximum(np.matmul(a, encv[None]) - relu_threshold, 0.0)
    if mask is not None:
        gate = gate * mask
    y = x * gate
    mlp = layer_norm_f64(decode_y_neuron_tail_f64(y, decoder))
    return layer_norm_f64(cur + mlp), rho


def block_pattern_mask(latent: int, block_size: int, active_blocks=None) -> np.ndarray:
    """BlockPattern1d::mask (kernel/block_sparse.rs:49-64): 1 on the active
    blocks of block_size latents (all when active_blocks is None), else 0."""
    m = np.zeros(latent, np.float32)
    bs = max(1, block_size)
    for blk in range((latent + bs - 1) // bs):
        if active_blocks is None or blk in active_blocks:
            m[blk * bs:min(latent, (blk + 1) * bs)] = 1.0
    return m


def model_forward_f64(tokens, embed, encoder, encoder_v, decoder, lm_head, n_layer: int,
                      pos0=0, theta: float = 65536.0, rho0s=None, return_state: bool = False,
                      relu_threshold: float = 0.0, latent_mask=None):
    """DragonModel sequence forward with shared low-rank weights and the
    vanilla residual connector (dragon.rs:3340-3420): current =
    LN(embed[tokens]) (:3352), n_layer x lowrank_layer_f64 with the same
    positions, then logits = current @ lm_head (project_hidden_to_logits,
    :4033-4055).  tokens [B,T]; returns logits [B,T,vocab] f64.
    rho0s: per-layer carried states (each layer's LayerState.rho,
    dragon.rs:3437-3446), None = zeros; with return_state the per-layer
    successor states are returned too.  relu_threshold and latent_mask go to
    every layer."""
    emb = np.asarray(embed, np.float64)
    cur = layer_norm_f64(emb[np.asarray(tokens)])
    rhos = []
    for layer in range(n_layer):
        rho0 = rho0s[layer] if rho0s is not None else None
        cur, rho = lowrank_layer_f64(cur, encoder, encoder_v, decoder, pos0=pos0, theta=theta,
                                     rho0=rho0, relu_threshold=relu_threshold,
                                     latent_mask=latent_mask)
        rhos.append(rho)
    logits = cur @ np.asarray(lm_head, np.float64)
    return (logits, rhos) if return_state else logits


def rel_l2(a, b) -> float:
    """||a - b||_2 / ||b||_2 in f64 (b is the reference)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b.ravel())
    num = np.linalg.norm((a - b).ravel())
    return float(num / den) if den > 0 else float(num)


def attention_vjp_f64(q, v, grad_out, decay=None, rho0=None, safe: str = "dense"):
    """VJP of the causal linear attention (the context only) in f64:
    ctx = tril(-1)(Q Q^T * d^(r-c)) V + (Q * d^t) rho0, Q = K = query.
    Restates dense_causal_attention_vjp_with_initial_rho
    (kernel/src/dense_causal_attention/backward_runtime.rs:36-148), which the
    recurrent backward (kernel/src/recurrent/backward_runtime.rs:336-502,
    state history + reverse-time adjoint) equals in closed form:
      S  = tril(-1)(Q Q^T) * D,  D[r, c] = d^(r-c)          (:70-72)
      GS = tril(-1)(G V^T)                                   (:90-93)
      grad_v = S^T G  (summed over heads when value heads = 1)  (:80-89)
      grad_q = (GS*D + (GS*D)^T) Q  [+ (G rho0^T) * d^t]     (:94-98, :124-125)
      grad_d = sum(GS * gap * S) / sd  [+ sum(G * (Q d^t rho0) * t) / sd]
      grad_rho0 = (Q * d^t)^T G                               (:137)
    sd = d + 1e-12 (safe="dense", :100) or, for |d| < 1e-8, 1e-8
    (safe="recurrent", recurrent/backward_runtime.rs:458-465).
    q [B,H,T,N], v [B,Hv,T,D], grad_out [B,H,T,D], decay [H] (None = ones),
    rho0 [B,H,N,D] or None.  Returns (grad_q, grad_v, grad_decay, grad_rho0)."""
    q = np.asarray(q, np.float64)
    v = np.asarray(v, np.float64)
    g = np.asarray(grad_out, np.float64)
    B, H, T, N = q.shape
    Hv, D = v.shape[1], v.shape[3]
    d = np.ones(H) if decay is None else np.asarray(decay, np.float64)
    if safe == "dense":
        sd = d + 1e-12
    else:
        sd = np.where((d < 1e-8) & (d > -1e-8), 1e-8, d)
    vh = np.broadcast_to(v, (B, H, T, D)) if Hv == 1 else v
    r = np.arange(T)[:, None]
    c = np.arange(T)[None, :]
    gap = np.where(r > c, r - c, 0).astype(np.float64)
    below = r > c
    Dm = np.power(d[:, None, None], gap[None])              # [H, T, T]
    S = np.where(below, q @ q.transpose(0, 1, 3, 2), 0.0) * Dm[None]
    GS = np.where(below, g @ vh.transpose(0, 1, 3, 2), 0.0)
    W = GS * Dm[None]
    gq = (W + W.transpose(0, 1, 3, 2)) @ q
    gv = S.transpose(0, 1, 3, 2) @ g
    if Hv == 1:
        gv = gv.sum(axis=1, keepdims=True)
    gd = ((GS * gap[None, None]) * S / sd[None, :, None, None]).sum(axis=(0, 2, 3))
    grho = None
    if rho0 is not None:
        rho = np.asarray(rho0, np.float64)
        pos = np.arange(T, dtype=np.float64)
        sdec = np.power(d[:, None], pos[None])[None, :, :, None]   # [1, H, T, 1]
        sq = q * sdec
        ic = sq @ rho
        gq = gq + (g @ rho.transpose(0, 1, 3, 2)) * sdec
        gd = gd + ((g * ic) * pos[None, None, :, None] / sd[None, :, None, None]).sum(axis=(0, 2, 3))
        grho = sq.transpose(0, 1, 3, 2) @ g
    return gq, gv, gd, grho
