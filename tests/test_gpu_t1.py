"""One-token (T = 1) calls through the reference surface and the decode step.

The reference decodes through the same fused op it uses for prefill
(sequence_dispatch.rs:109-124) and picks its kernel by T
(recurrent/forward_runtime.rs:235-256).  Here a T = 1 fp32 call of
bdh_recurrent_attention[_rope]_fwd runs the one-token step: the sparse row
gather in place, one dense pass otherwise (out of place, zero state, decay).
Checked against the oracle's f32 recurrence (rel-L2 1e-5), with the rows
outside the active set bit-identical where nothing scales them."""
import ctypes

import numpy as np
import pytest

from tests import refcases as rc
from tests.gpu_util import TOL_F32, announce, dev, host, need_gpu, rel_l2

pytestmark = pytest.mark.gpu


def _kernel_launches(lib, _lib, kind):
    ms, n = ctypes.c_double(), ctypes.c_int64()
    assert lib.bdh_profile_kernel_get(kind, ctypes.byref(ms), ctypes.byref(n)) == _lib.BDH_OK
    return n.value


def _inactive(idx, cnt, N):
    mask = np.ones(N, bool)
    mask[idx[:cnt]] = False
    return mask


@pytest.mark.parametrize("B,H,Hv,N,D,pos", [
    (2, 4, 1, 8192, 256, 37),    # the C3 head shape
    (1, 2, 2, 1024, 64, 0),      # position 0, per-head values
    (2, 2, 1, 2048, 96, 1000),   # D not a multiple of 256
])
def test_t1_rope_route_in_place_and_out_of_place(oracle, B, H, Hv, N, D, pos):
    torch = need_gpu()
    import burn_dragon_amd as bd
    from burn_dragon_amd import _lib
    lib = _lib.load()
    rng = np.random.default_rng(4100 + N + D + pos)
    x = rc.sparse_relu(rng, (B, H, 1, N))
    v = rc.gaussian(rng, (B, Hv, 1, D), 1 / 16)
    rho0 = rc.gaussian(rng, (B, H, N, D), 0.5)
    rho_ref = rho0.copy()
    a_ref, idx_ref, cnt_ref = oracle.decode_step_f32(x[:, :, 0], v[:, :, 0], rho_ref, pos)

    announce("t1 route in place", B, H, Hv, N, D, pos)
    xd, vd, rd = dev(torch, x), dev(torch, v), dev(torch, rho0)
    assert lib.bdh_profile_kernel_timing(1) == _lib.BDH_OK
    out = bd.try_fused_recurrent_attention_rope(xd, vd, rd, position=pos, inplace=True)
    torch.cuda.synchronize()
    n_dec = _kernel_launches(lib, _lib, _lib.BDH_KERNEL_DECODE)
    n_pf = _kernel_launches(lib, _lib, _lib.BDH_KERNEL_PREFILL)
    assert lib.bdh_profile_kernel_timing(0) == _lib.BDH_OK
    assert (n_dec, n_pf) == (1, 0), "T = 1 must run the decode kernel, not the prefill"
    assert out.rho.data_ptr() == rd.data_ptr()
    assert rel_l2(host(out.context)[:, :, 0], a_ref) <= TOL_F32
    got = host(rd)
    assert rel_l2(got, rho_ref) <= TOL_F32
    for b in range(B):
        for h in range(H):
            m = _inactive(idx_ref[b, h], cnt_ref[b, h], N)
            assert np.array_equal(got[b, h][m], rho0[b, h][m])

    announce("t1 route out of place", B, H, Hv, N, D, pos)
    rd = dev(torch, rho0)
    out = bd.try_fused_recurrent_attention_rope(xd, vd, rd, position=pos)
    torch.cuda.synchronize()
    assert out.rho.data_ptr() != rd.data_ptr()
    assert np.array_equal(host(rd), rho0), "the caller's rho must not be written"
    assert rel_l2(host(out.context)[:, :, 0], a_ref) <= TOL_F32
    got = host(out.rho)
    assert rel_l2(got, rho_ref) <= TOL_F32
    for b in range(B):
        for h in range(H):
            m = _inactive(idx_ref[b, h], cnt_ref[b, h], N)
            assert np.array_equal(got[b, h][m], rho0[b, h][m])

    announce("t1 route zero state", B, H, Hv, N, D, pos)
    out = bd.try_fused_recurrent_attention_rope(xd, vd, None, position=pos)
    torch.cuda.synchronize()
    q = oracle.rope_rotate(x, pos0=pos)
    cref, rref = oracle.recurrent_f32(q, v)
    assert np.array_equal(host(out.context), np.zeros_like(cref))
    assert rel_l2(host(out.rho), rref) <= TOL_F32


def test_t1_rotated_query_entry(oracle):
    # bdh_recurrent_attention_fwd: the query is already rotated, so the
    # active set is {i : q_i != 0}.
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(4201)
    B, H, N, D = 2, 3, 4096, 128
    q = oracle.rope_rotate(rc.sparse_relu(rng, (B, H, 1, N)), pos0=11)
    v = rc.gaussian(rng, (B, 1, 1, D), 1 / 16)
    rho0 = rc.gaussian(rng, (B, H, N, D))
    cref, rref = oracle.recurrent_f32(q, v, rho0)
    announce("t1 rotated query")
    for inplace in (True, False):
        rd = dev(torch, rho0)
        out = bd.try_fused_recurrent_attention(dev(torch, q), dev(torch, v), rd, inplace=inplace)
        torch.cuda.synchronize()
        assert rel_l2(host(out.context), cref) <= TOL_F32
        assert rel_l2(host(out.rho), rref) <= TOL_F32
        if not inplace:
            assert np.array_equal(host(rd), rho0)


@pytest.mark.parametrize("inplace", [True, False])
def test_t1_decay_route(oracle, inplace):
    # ALiBi-style decay through the reference surface at T = 1: every row of
    # rho is scaled (recurrent.rs:415), so the step is one dense pass.
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(4301 + inplace)
    B, H, N, D = 2, 4, 2048, 64
    x = rc.sparse_relu(rng, (B, H, 1, N))
    v = rc.gaussian(rng, (B, 1, 1, D), 1 / 16)
    rho0 = rc.gaussian(rng, (B, H, N, D))
    decay = np.array([0.95, 0.9, 0.85, 0.8], np.float32)
    cref, rref = oracle.recurrent_f32(x, v, rho0, decay)
    announce("t1 decay", inplace)
    rd = dev(torch, rho0)
    out = bd.try_fused_recurrent_attention(dev(torch, x), dev(torch, v), rd, dev(torch, decay),
                                           inplace=inplace)
    torch.cuda.synchronize()
    assert rel_l2(host(out.context), cref) <= TOL_F32
    assert rel_l2(host(out.rho), rref) <= TOL_F32
    if not inplace:
        assert np.array_equal(host(rd), rho0)


def test_decode_step_with_decay_over_16_steps(oracle):
    # bdh_decode_step with decay [0.95, 0.9, ...] over 16 RoPE steps against
    # the f64 recurrence of the same 16 tokens (attention.rs:201-208,
    # linear.rs:53-56).
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(4401)
    B, H, N, D, K, P = 2, 4, 1024, 64, 16, 100
    xs = rc.sparse_relu(rng, (B, H, K, N))
    vs = rc.gaussian(rng, (B, 1, K, D), 1 / 16)
    rho0 = rc.gaussian(rng, (B, H, N, D), 0.5)
    decay = np.array([0.95, 0.9, 0.85, 0.8], np.float32)
    cref, rref = oracle.recurrent_f64(oracle.rope_rotate(xs, pos0=P), vs, rho0, decay)
    announce("decode decay 16 steps")
    rd = dev(torch, rho0)
    dd = dev(torch, decay)
    outs = []
    for k in range(K):
        o = bd.decode_step(dev(torch, xs[:, :, k]), dev(torch, vs[:, :, k]), rd, position=P + k,
                           decay=dd)
        outs.append(host(o.readout))
    torch.cuda.synchronize()
    assert rel_l2(np.stack(outs, 2), cref) <= TOL_F32
    assert rel_l2(host(rd), rref) <= TOL_F32


@pytest.mark.parametrize("D", [320, 512, 2304])
def test_decode_step_wide_rows(oracle, D):
    # Rows wider than one 256-column block: the sparse step recompacts per
    # column block (embd 320, 512, and past the old 2048 limit).
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(4500 + D)
    B, H, N, pos = 2, 2, 2048, 21
    x = rc.sparse_relu(rng, (B, H, N))
    v = rc.gaussian(rng, (B, 1, D), 1 / 16)
    rho0 = rc.gaussian(rng, (B, H, N, D), 0.5)
    rho_ref = rho0.copy()
    a_ref, idx_ref, cnt_ref = oracle.decode_step_f32(x, v, rho_ref, pos)
    announce("decode wide", D)
    rd = dev(torch, rho0)
    out = bd.decode_step(dev(torch, x), dev(torch, v), rd, position=pos, want_active=True)
    torch.cuda.synchronize()
    assert rel_l2(host(out.readout), a_ref) <= TOL_F32
    assert rel_l2(host(rd), rho_ref) <= TOL_F32
    assert np.array_equal(out.active_idx.cpu().numpy(), idx_ref)
    assert np.array_equal(out.active_cnt.cpu().numpy(), cnt_ref)


def test_t1_route_full_c3_shape(oracle):
    # BASELINE config 3's shape (B 64, nh 4, N 8192, D 256) through the
    # reference surface, in place: two sampled streams against the oracle,
    # and every stream's inactive rows unchanged.
    torch = need_gpu()
    import burn_dragon_amd as bd
    B, H, N, D, pos = 64, 4, 8192, 256, 1024
    g = torch.Generator(device="cuda").manual_seed(4601)
    rho = torch.randn(B, H, N, D, generator=g, device="cuda") * 0.25
    x = torch.relu(torch.randn(B, H, 1, N, generator=g, device="cuda") - 1.645)
    v = torch.randn(B, 1, 1, D, generator=g, device="cuda") / 16
    picks = [(0, 0), (63, 3)]
    rho_s = {p: host(rho[p[0], p[1]]) for p in picks}
    announce("t1 route C3 shape")
    before = rho.clone()
    out = bd.try_fused_recurrent_attention_rope(x, v, rho, position=pos, inplace=True)
    torch.cuda.synchronize()
    xh, vh = host(x), host(v)
    for (b, h) in picks:
        r = rho_s[(b, h)][None, None].copy()
        a_ref, idx_ref, cnt_ref = oracle.decode_step_f32(xh[b:b + 1, h:h + 1, 0], vh[b:b + 1, :, 0], r, pos)
        assert rel_l2(host(out.context[b, h, 0]), a_ref[0, 0]) <= TOL_F32
        assert rel_l2(host(rho[b, h]), r[0, 0]) <= TOL_F32
    changed = (rho != before).any(dim=-1)          # [B, H, N] rows touched
    xr = x[:, :, 0]
    partner = xr.view(B, H, N // 2, 2).flip(-1).reshape(B, H, N)
    may_change = (xr != 0) | (partner != 0)        # superset of the active set
    assert not bool((changed & ~may_change).any())
