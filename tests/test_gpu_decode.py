"""Sparse decode kernel vs the CPU oracle: readout and updated rho within
rel-L2 1e-5 (fp32), active-row sets bit-exact, rows outside the active set
untouched bit for bit."""
import numpy as np
import pytest

from tests import refcases as rc
from tests.gpu_util import TOL_F32, announce, dev, host, need_gpu, rel_l2

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,H,Hv,N,D,pos", [
    (2, 2, 1, 1024, 64, 0),        # position 0: active set = nonzero x
    (2, 4, 1, 8192, 256, 37),      # BASELINE head shape, 8 segments per stream
    (1, 3, 3, 512, 256, 1000),     # per-head values, one segment
    (2, 2, 1, 2048, 96, 5),        # D not a multiple of 256
    (1, 2, 2, 640, 10, 77),        # D not a multiple of 4 (scalar path)
    (3, 1, 1, 4096, 128, 65535),   # large position
])
def test_decode_step_matches_oracle(oracle, B, H, Hv, N, D, pos):
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(1000 + N + D + pos)
    x = rc.sparse_relu(rng, (B, H, N))
    v = rc.gaussian(rng, (B, Hv, D), 1 / 16)
    rho0 = rc.gaussian(rng, (B, H, N, D), 0.5)
    rho_ref = rho0.copy()
    a_ref, idx_ref, cnt_ref = oracle.decode_step_f32(x, v, rho_ref, pos)

    announce("decode", B, H, Hv, N, D, pos)
    rho_d = dev(torch, rho0)
    out = bd.decode_step(dev(torch, x), dev(torch, v), rho_d, position=pos, want_active=True)
    torch.cuda.synchronize()
    assert out is not None
    a = host(out.readout)
    assert rel_l2(a, a_ref) <= TOL_F32
    assert rel_l2(host(rho_d), rho_ref) <= TOL_F32
    assert np.array_equal(out.active_cnt.cpu().numpy(), cnt_ref)
    assert np.array_equal(out.active_idx.cpu().numpy(), idx_ref)
    # inactive rows are bit-identical to the input state
    rho_new = host(rho_d)
    for b in range(B):
        for h in range(H):
            mask = np.ones(N, bool)
            mask[idx_ref[b, h, :cnt_ref[b, h]]] = False
            assert np.array_equal(rho_new[b, h][mask], rho0[b, h][mask])


def test_decode_prerotated_query(oracle):
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(7)
    B, H, N, D = 2, 2, 1024, 64
    q = oracle.rope_rotate(rc.sparse_relu(rng, (B, H, 1, N)), pos0=9)[:, :, 0]
    v = rc.gaussian(rng, (B, 1, D), 1 / 16)
    rho0 = rc.gaussian(rng, (B, H, N, D))
    ctx, rho_ref = oracle.recurrent_f32(q[:, :, None], v[:, :, None], rho0)
    announce("decode prerotated")
    rho_d = dev(torch, rho0)
    out = bd.decode_step(dev(torch, q), dev(torch, v), rho_d, position=None, want_active=True)
    torch.cuda.synchronize()
    assert rel_l2(host(out.readout), ctx[:, :, 0]) <= TOL_F32
    assert rel_l2(host(rho_d), rho_ref) <= TOL_F32
    cnt = out.active_cnt.cpu().numpy()
    for b in range(B):
        for h in range(H):
            nz = np.nonzero(q[b, h])[0]
            assert cnt[b, h] == len(nz)
            assert np.array_equal(out.active_idx.cpu().numpy()[b, h, :len(nz)], nz)


def test_decode_sequence_equals_prefill(oracle):
    """K decode steps == one K-token recurrent call (same rotated inputs)."""
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(11)
    B, H, N, D, K, pos0 = 2, 2, 2048, 128, 8, 100
    xs = rc.sparse_relu(rng, (B, H, K, N))
    vs = rc.gaussian(rng, (B, 1, K, D), 1 / 16)
    rho0 = rc.gaussian(rng, (B, H, N, D))
    q = oracle.rope_rotate(xs, pos0=pos0)
    ctx_ref, rho_ref = oracle.recurrent_f64(q, vs, rho0)
    announce("decode sequence")
    rho_d = dev(torch, rho0)
    outs = []
    for k in range(K):
        o = bd.decode_step(dev(torch, xs[:, :, k]), dev(torch, vs[:, :, k]), rho_d, position=pos0 + k)
        outs.append(host(o.readout))
    torch.cuda.synchronize()
    assert rel_l2(np.stack(outs, 2), ctx_ref) <= TOL_F32
    assert rel_l2(host(rho_d), rho_ref) <= TOL_F32


def test_decode_empty_and_full_rows(oracle):
    """Edge cases: an all-zero x (no active row) and a dense x (all rows)."""
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(13)
    B, H, N, D = 1, 2, 1024, 64
    x = np.zeros((B, H, N), np.float32)
    x[0, 1] = np.abs(rng.standard_normal(N)).astype(np.float32) + 0.1
    v = rc.gaussian(rng, (B, 1, D))
    rho0 = rc.gaussian(rng, (B, H, N, D))
    rho_ref = rho0.copy()
    a_ref, idx_ref, cnt_ref = oracle.decode_step_f32(x, v, rho_ref, 3)
    announce("decode empty/full")
    rho_d = dev(torch, rho0)
    out = bd.decode_step(dev(torch, x), dev(torch, v), rho_d, position=3, want_active=True)
    torch.cuda.synchronize()
    cnt = out.active_cnt.cpu().numpy()
    assert cnt[0, 0] == 0 and cnt[0, 1] == N
    assert np.array_equal(out.active_idx.cpu().numpy(), idx_ref)
    assert np.all(host(out.readout)[0, 0] == 0.0)
    assert rel_l2(host(out.readout), a_ref) <= TOL_F32
    assert rel_l2(host(rho_d), rho_ref) <= TOL_F32


def test_decode_step_with_pointers_off_16_byte_alignment(oracle):
    # Tensors that are contiguous views at a 4-byte offset (a storage offset
    # of one float): the step takes its scalar-column kernel rather than the
    # float4 one, and matches the oracle; rows outside the active set stay
    # bit-identical.
    torch = need_gpu()
    import burn_dragon_amd as bd
    B, H, N, D, pos = 2, 2, 1024, 64, 9
    rng = np.random.default_rng(4242)
    x = rc.sparse_relu(rng, (B, H, N))
    v = rc.gaussian(rng, (B, 1, D), 1 / 16)
    rho0 = rc.gaussian(rng, (B, H, N, D), 0.5)
    rho_ref = rho0.copy()
    a_ref, _, _ = oracle.decode_step_f32(x, v, rho_ref, pos)

    def shifted(a):
        flat = torch.zeros(a.size + 1, device="cuda")
        flat[1:] = torch.from_numpy(np.ascontiguousarray(a, np.float32).reshape(-1)).cuda()
        view = flat[1:].view(a.shape)
        assert view.data_ptr() % 16 == 4
        return view
    xd, vd, rd = shifted(x), shifted(v), shifted(rho0)
    announce("decode off 16-byte alignment")
    out = bd.decode_step(xd, vd, rd, position=pos)
    torch.cuda.synchronize()
    assert out is not None
    assert rel_l2(host(out.readout), a_ref) <= TOL_F32
    assert rel_l2(host(rd), rho_ref) <= TOL_F32
    partner = x.reshape(B, H, N // 2, 2)[..., ::-1].reshape(B, H, N)
    untouched = (x == 0) & (partner == 0)
    assert np.array_equal(host(rd)[untouched], rho0[untouched])


@pytest.mark.parametrize("B,H,N,D,pos,density", [
    (64, 4, 256, 16, 9, 0.02),      # 256 streams of a few rows each
    (1, 1, 65536, 64, 3, 0.3),      # one long stream (several compaction passes)
    (8, 16, 512, 32, 77, 0.0),      # no active row at all
    (2048, 1, 64, 8, 5, 0.05),      # many short streams
    (2049, 1, 32, 8, 6, 0.1),
])
def test_decode_stream_counts(oracle, B, H, N, D, pos, density):
    # Streams with few, many or no active rows, one stream alone and over two
    # thousand streams: every readout, row and list matches the oracle, and
    # the step without lists equals the step with them.
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(5000 + N + B)
    x = (rng.random((B, H, N)) < density).astype(np.float32) * rng.random((B, H, N)).astype(np.float32)
    x[::3] = 0.0  # whole streams without an active row between active ones
    v = rc.gaussian(rng, (B, 1, D), 1 / 16)
    rho0 = rc.gaussian(rng, (B, H, N, D), 0.5)
    rho_ref = rho0.copy()
    a_ref, idx_ref, cnt_ref = oracle.decode_step_f32(x, v, rho_ref, pos)
    announce("decode stream counts", B, H, N, D, pos, density)
    rho_d = dev(torch, rho0)
    out = bd.decode_step(dev(torch, x), dev(torch, v), rho_d, position=pos, want_active=True)
    torch.cuda.synchronize()
    assert np.array_equal(out.active_cnt.cpu().numpy(), cnt_ref)
    assert np.array_equal(out.active_idx.cpu().numpy(), idx_ref)
    a = host(out.readout)
    assert np.all(a[cnt_ref == 0] == 0.0)
    if np.abs(a_ref).sum() > 0:
        assert rel_l2(a, a_ref) <= TOL_F32
    assert rel_l2(host(rho_d), rho_ref) <= TOL_F32
    # and without the lists (the step keeps its own)
    rho_d2 = dev(torch, rho0)
    out2 = bd.decode_step(dev(torch, x), dev(torch, v), rho_d2, position=pos)
    torch.cuda.synchronize()
    assert torch.equal(out2.readout, out.readout) and torch.equal(rho_d2, rho_d)
