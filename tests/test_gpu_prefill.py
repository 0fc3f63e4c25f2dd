"""Prefill paths vs the CPU oracle at sizes the oracle finishes in seconds.

fp32 path: rel-L2 <= 1e-5 against the f64 recurrence (the reference's own
test shapes and index-formula inputs, decay, initial state, shared and
per-head values, RoPE fused).  bf16 MFMA path: rel-L2 <= 1e-2 against the
f64 recurrence evaluated on the bf16-rounded inputs."""
import numpy as np
import pytest

from tests import refcases as rc
from tests.gpu_util import TOL_BF16, TOL_F32, announce, dev, host, need_gpu, rel_l2

pytestmark = pytest.mark.gpu


def _run(torch, bd, q, v, rho0, decay, dtype=None, rope=None):
    dt = dtype or torch.float32
    qd, vd = dev(torch, q, dt), dev(torch, v, dt)
    rd = dev(torch, rho0) if rho0 is not None else None
    dd = dev(torch, decay) if decay is not None else None
    if rope is None:
        out = bd.try_fused_recurrent_attention(qd, vd, rd, dd)
    else:
        out = bd.try_fused_recurrent_attention_rope(qd, vd, rd, dd, position=rope[0], fixed=rope[1])
    torch.cuda.synchronize()
    assert out is not None
    return host(out.context), host(out.rho)


# ---- fp32 path ---------------------------------------------------------------

@pytest.mark.parametrize("case", range(len(rc.RECURRENT_TEST_SHAPES)))
def test_f32_reference_test_shapes(oracle, case):
    # recurrent/tests.rs:158-206, 290-336 shapes; our generator, same law N(0,1).
    torch = need_gpu()
    import burn_dragon_amd as bd
    qs, vs, rs, dec = rc.RECURRENT_TEST_SHAPES[case]
    rng = np.random.default_rng(100 + case)
    q = rc.gaussian(rng, qs)
    v = rc.gaussian(rng, vs)
    rho0 = rc.gaussian(rng, rs) if rs else None
    decay = np.array(dec, np.float32) if dec else None
    announce("f32 shapes", qs, vs)
    ctx, rho = _run(torch, bd, q, v, rho0, decay)
    cref, rref = oracle.recurrent_f64(q, v, rho0, decay)
    assert rel_l2(ctx, cref) <= TOL_F32
    assert rel_l2(rho, rref) <= TOL_F32


def test_f32_index_formula_invariant_inputs(oracle):
    # linear.rs:485-533 inputs: T=320 (crosses the 256-token state interval).
    torch = need_gpu()
    import burn_dragon_amd as bd
    q, v, rho0, decay, _ = rc.chunked_decay_state_case()
    announce("f32 linear.rs:485")
    ctx, rho = _run(torch, bd, q, v, rho0, decay)
    cref, rref = oracle.dense_score_f64(q, v, rho0, decay)
    assert rel_l2(ctx, cref) <= TOL_F32 and rel_l2(rho, rref) <= TOL_F32
    q, v, _ = rc.chunked_no_decay_case()
    announce("f32 linear.rs:451")
    ctx, rho = _run(torch, bd, q, v, None, None)
    cref, rref = oracle.dense_score_f64(q, v)
    assert rel_l2(ctx, cref) <= TOL_F32 and rel_l2(rho, rref) <= TOL_F32
    # known answer, linear.rs:433-449
    q, v, rho_exp, ctx_exp = rc.signed_rho_case()
    ctx, rho = _run(torch, bd, q, v, None, None)
    assert np.array_equal(rho, rho_exp) and np.array_equal(ctx, ctx_exp)


def test_f32_c1_config_rope(oracle):
    # B1 nh4 T256 N1024 D64, RoPE theta 65536, V ~ N(0,1).
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(rc.config_seed(1))
    x = rc.sparse_relu(rng, (1, 4, 256, 1024))
    v = rc.gaussian(rng, (1, 1, 256, 64))
    announce("f32 C1 rope")
    ctx, rho = _run(torch, bd, x, v, None, None, rope=(0, False))
    q = oracle.rope_rotate(x, pos0=0)
    cref, rref = oracle.recurrent_f64(q, v)
    assert rel_l2(ctx, cref) <= TOL_F32 and rel_l2(rho, rref) <= TOL_F32
    # the f32 op-order mirror agrees too
    c32, r32 = oracle.recurrent_f32(q, v)
    assert rel_l2(ctx, c32) <= TOL_F32


def test_f32_rope_fixed_and_offset(oracle):
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(21)
    x = rc.sparse_relu(rng, (2, 2, 40, 64))
    v = rc.gaussian(rng, (2, 2, 40, 24))
    rho0 = rc.gaussian(rng, (2, 2, 64, 24))
    for pos, fixed in ((5, False), (123, True)):
        announce("f32 rope", pos, fixed)
        ctx, rho = _run(torch, bd, x, v, rho0, None, rope=(pos, fixed))
        q = oracle.rope_rotate(x, pos0=pos, mode=1 if fixed else 0)
        cref, rref = oracle.recurrent_f64(q, v, rho0)
        assert rel_l2(ctx, cref) <= TOL_F32 and rel_l2(rho, rref) <= TOL_F32


# ---- bf16 MFMA path -----------------------------------------------------------

def _bf16_case(rng, B, H, Hv, T, N, D, with_rho):
    x = rc.sparse_relu(rng, (B, H, T, N))
    v = rc.gaussian(rng, (B, Hv, T, D), 1 / 16)
    rho0 = rc.gaussian(rng, (B, H, N, D), 0.05) if with_rho else None
    return x, v, rho0


@pytest.mark.parametrize("B,H,Hv,T,N,D,with_rho,decay,pos", [
    (1, 2, 1, 128, 256, 64, False, None, 0),          # one chunk
    (2, 2, 1, 512, 512, 256, False, None, 0),         # 4 chunks, one interval
    (1, 2, 2, 300, 256, 96, True, None, 17),          # ragged T, per-head V, rho_in
    (1, 2, 1, 1100, 256, 128, True, None, 3),         # 3 state intervals (512+512+76)
    (1, 4, 1, 256, 256, 64, True, [0.99, 0.98, 0.97, 0.96], 0),  # ALiBi-style decay
    (1, 2, 1, 700, 512, 320, True, [0.995, 0.99], 9),  # D > 256, not a multiple of 256; 2 intervals
    (2, 2, 1, 600, 2304, 64, False, None, 5),          # x rotated once: rows of 4 streams, N % 2048 != 0
    (1, 1, 1, 1027, 256, 64, True, None, 2),           # x rotated once: B H T not a multiple of 4 rows
])
def test_bf16_rope_prefill_matches_oracle(oracle, B, H, Hv, T, N, D, with_rho, decay, pos):
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(T * 7 + N + D)
    x, v, rho0 = _bf16_case(rng, B, H, Hv, T, N, D, with_rho)
    dec = np.array(decay, np.float32) if decay else None
    xb, vb = oracle.round_bf16(x), oracle.round_bf16(v)
    announce("bf16 rope", B, H, Hv, T, N, D, with_rho, decay, pos)
    ctx, rho = _run(torch, bd, xb, vb, rho0, dec, dtype=torch.bfloat16, rope=(pos, False))
    q = oracle.rope_rotate(xb, pos0=pos)
    cref, rref = oracle.recurrent_f64(q, vb, rho0, dec)
    e_ctx, e_rho = rel_l2(ctx, cref), rel_l2(rho, rref)
    print(f"rel-L2 ctx {e_ctx:.2e} rho {e_rho:.2e}")
    assert e_ctx <= TOL_BF16 and e_rho <= TOL_BF16


@pytest.mark.parametrize("T", [384, 1100])  # one interval (rotated in the tile loads); three (x rotated once)
def test_bf16_rope_fixed_mode(oracle, T):
    # rotate_positions_fixed (attention.rs:512-550): every token at one position.
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(41)
    x, v, rho0 = _bf16_case(rng, 1, 2, 1, T, 256, 64, True)
    xb, vb = oracle.round_bf16(x), oracle.round_bf16(v)
    announce("bf16 rope fixed", 1, 2, T, 256, 64)
    ctx, rho = _run(torch, bd, xb, vb, rho0, None, dtype=torch.bfloat16, rope=(1000, True))
    q = oracle.rope_rotate(xb, pos0=1000, mode=1)
    cref, rref = oracle.recurrent_f64(q, vb, rho0)
    assert rel_l2(ctx, cref) <= TOL_BF16 and rel_l2(rho, rref) <= TOL_BF16


def test_bf16_alibi_dense_score_short_context(oracle):
    # DenseScoreShortContext with ALiBi (sequence_dispatch.rs:137-198): the
    # fused dense context + initial_context(rho0) + final_rho of the
    # reference are one call here, with decay = exp(-slope) (default slopes),
    # rho = the layer's state and no rotation (the ALiBi arm's frequencies
    # are zero, attention.rs:569).  Checked against the dense-score closed
    # form (linear.rs:221-364).
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(57)
    B, H, T, N, D = 2, 4, 300, 512, 64
    x, v, rho0 = _bf16_case(rng, B, H, 1, T, N, D, True)
    dec = bd.alibi_decay(bd.default_alibi_slopes(H)).numpy()
    xb, vb = oracle.round_bf16(x), oracle.round_bf16(v)
    announce("bf16 alibi dense-score", B, H, T, N, D)
    ctx, rho = _run(torch, bd, xb, vb, rho0, dec, dtype=torch.bfloat16)
    cref, rref = oracle.dense_score_f64(xb, vb, rho0, dec)
    e_ctx, e_rho = rel_l2(ctx, cref), rel_l2(rho, rref)
    print(f"rel-L2 ctx {e_ctx:.2e} rho {e_rho:.2e}")
    assert e_ctx <= TOL_BF16 and e_rho <= TOL_BF16


def test_bf16_rope_positions_across_calls(oracle):
    # Each call rotates at its own positions (nothing is kept between calls):
    # calls at positions 5, 5, 9, 5 and a longer call at 5 must each match
    # the oracle.
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(61)
    x, v, _ = _bf16_case(rng, 1, 2, 1, 256, 256, 64, False)
    xl, vl, _ = _bf16_case(rng, 1, 2, 1, 384, 256, 64, False)
    xb, vb, xlb, vlb = (oracle.round_bf16(t) for t in (x, v, xl, vl))
    announce("bf16 rope positions across calls")
    for xx, vv, pos in ((xb, vb, 5), (xb, vb, 5), (xb, vb, 9), (xb, vb, 5), (xlb, vlb, 5)):
        ctx, rho = _run(torch, bd, xx, vv, None, None, dtype=torch.bfloat16, rope=(pos, False))
        cref, rref = oracle.recurrent_f64(oracle.rope_rotate(xx, pos0=pos), vv)
        assert rel_l2(ctx, cref) <= TOL_BF16 and rel_l2(rho, rref) <= TOL_BF16, pos


@pytest.mark.parametrize("chunk", [128, 256, 384, 1024])
def test_bf16_row_chunk(oracle, chunk):
    # The row chunk (the reference's dense_score_row_chunk, linear.rs:117-118)
    # only moves where rho is materialised: T = 1100 with rho in and decay is
    # 9, 5, 3 or 2 state intervals, each within the bf16 tolerance of the
    # oracle.
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(71 + chunk)
    x, v, rho0 = _bf16_case(rng, 1, 2, 1, 1100, 256, 64, True)
    dec = np.array([0.999, 0.998], np.float32)
    xb, vb = oracle.round_bf16(x), oracle.round_bf16(v)
    announce("bf16 row chunk", chunk)
    out = bd.try_fused_recurrent_attention_rope(
        dev(torch, xb, torch.bfloat16), dev(torch, vb, torch.bfloat16), dev(torch, rho0),
        dev(torch, dec), position=4, chunk=chunk)
    torch.cuda.synchronize()
    assert out is not None
    cref, rref = oracle.recurrent_f64(oracle.rope_rotate(xb, pos0=4), vb, rho0, dec)
    assert rel_l2(host(out.context), cref) <= TOL_BF16 and rel_l2(host(out.rho), rref) <= TOL_BF16


@pytest.mark.parametrize("rope,decay,chunk,T", [
    (None, [0.9, -0.8], 256, 700),        # pre-rotated queries, a negative decay, 3 intervals
    ((6, False), [0.5, 0.25], 128, 1100),  # strong decay: powers underflow inside an interval
    ((0, False), [1.0, 0.97], 384, 900),   # a decay of exactly 1 beside a decaying head
])
def test_bf16_state_carry_with_decay(oracle, rope, decay, chunk, T):
    # Decay in the state-carry form (two or more intervals): each token's row
    # of q^T weighted by d^(end - t), the carried block scaled by d^Lc at
    # each interval start, d^(r - c) on the scores and d^r on the readouts.
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(83 + T + chunk)
    x, v, rho0 = _bf16_case(rng, 1, 2, 1, T, 256, 64, True)
    dec = np.array(decay, np.float32)
    xb, vb = oracle.round_bf16(x), oracle.round_bf16(v)
    if rope is None:
        xb = oracle.round_bf16(oracle.rope_rotate(xb, pos0=0))
    announce("bf16 state carry decay", rope, decay, chunk, T)
    xd, vd = dev(torch, xb, torch.bfloat16), dev(torch, vb, torch.bfloat16)
    if rope is None:
        out = bd.try_fused_recurrent_attention(xd, vd, dev(torch, rho0), dev(torch, dec), chunk=chunk)
        q = xb
    else:
        out = bd.try_fused_recurrent_attention_rope(xd, vd, dev(torch, rho0), dev(torch, dec),
                                                    position=rope[0], chunk=chunk)
        q = oracle.rope_rotate(xb, pos0=rope[0])
    torch.cuda.synchronize()
    assert out is not None
    cref, rref = oracle.recurrent_f64(q, vb, rho0, dec)
    e_ctx, e_rho = rel_l2(host(out.context), cref), rel_l2(host(out.rho), rref)
    print(f"rel-L2 ctx {e_ctx:.2e} rho {e_rho:.2e}")
    assert e_ctx <= TOL_BF16 and e_rho <= TOL_BF16


def test_bf16_row_chunk_outside_the_abi_is_refused():
    torch = need_gpu()
    import burn_dragon_amd as bd
    x = torch.zeros(1, 2, 256, 256, device="cuda", dtype=torch.bfloat16)
    v = torch.zeros(1, 1, 256, 64, device="cuda", dtype=torch.bfloat16)
    announce("bf16 row chunk refused")
    for chunk in (-128, 100, 8192):
        assert bd.try_fused_recurrent_attention_rope(x, v, chunk=chunk) is None, chunk
    assert bd.try_fused_recurrent_attention_rope(x, v, chunk=4096) is not None


def test_bf16_prerotated_query(oracle):
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(31)
    x, v, rho0 = _bf16_case(rng, 2, 2, 1, 256, 256, 64, True)
    q = oracle.round_bf16(oracle.rope_rotate(x, pos0=0))
    vb = oracle.round_bf16(v)
    announce("bf16 prerotated")
    ctx, rho = _run(torch, bd, q, vb, rho0, None, dtype=torch.bfloat16)
    cref, rref = oracle.recurrent_f64(q, vb, rho0)
    assert rel_l2(ctx, cref) <= TOL_BF16 and rel_l2(rho, rref) <= TOL_BF16


def test_bf16_unsupported_shape_returns_none():
    torch = need_gpu()
    import burn_dragon_amd as bd
    q = torch.zeros(1, 1, 8, 100, dtype=torch.bfloat16, device="cuda")
    v = torch.zeros(1, 1, 8, 64, dtype=torch.bfloat16, device="cuda")
    assert bd.try_fused_recurrent_attention(q, v) is None


# ---- dense causal attention ----------------------------------------------------

@pytest.mark.parametrize("case", range(len(rc.DENSE_TEST_SHAPES)))
def test_dense_causal_attention_f32(oracle, case):
    # dense_causal_attention/tests.rs:185-204 shapes and decays.
    torch = need_gpu()
    import burn_dragon_amd as bd
    qs, vs, dec = rc.DENSE_TEST_SHAPES[case]
    rng = np.random.default_rng(200 + case)
    q, v = rc.gaussian(rng, qs), rc.gaussian(rng, vs)
    decay = np.array(dec, np.float32)
    announce("dense f32", qs)
    out = bd.try_fused_dense_causal_attention(dev(torch, q), dev(torch, v), dev(torch, decay))
    torch.cuda.synchronize()
    cref, _ = oracle.dense_score_f64(q, v, None, decay, want_rho=False)
    assert rel_l2(host(out), cref) <= TOL_F32


def test_dense_causal_attention_bf16_and_limits(oracle):
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(41)
    q = oracle.round_bf16(oracle.rope_rotate(rc.sparse_relu(rng, (2, 2, 384, 256))))
    v = oracle.round_bf16(rc.gaussian(rng, (2, 1, 384, 64), 1 / 16))
    decay = np.ones(2, np.float32)
    announce("dense bf16")
    out = bd.try_fused_dense_causal_attention(dev(torch, q, torch.bfloat16),
                                              dev(torch, v, torch.bfloat16), dev(torch, decay))
    torch.cuda.synchronize()
    cref, _ = oracle.dense_score_f64(q, v, None, None, want_rho=False)
    assert rel_l2(host(out), cref) <= TOL_BF16
    big = torch.zeros(1, 1, 1025, 8, device="cuda")
    assert bd.try_fused_dense_causal_attention(big, big, torch.ones(1, device="cuda")) is None
    # decay of the wrong shape -> None (dense_causal_attention.rs:209-211)
    qd = dev(torch, q, torch.bfloat16)
    vd = dev(torch, v, torch.bfloat16)
    assert bd.try_fused_dense_causal_attention(qd, vd, torch.ones(3, device="cuda")) is None


@pytest.mark.parametrize("B,H,T,N,D", [
    (1, 2, 1000, 512, 64),    # 4 row blocks, the last ragged (232 rows)
    (2, 1, 1024, 256, 320),   # whole row blocks, two 256-column context blocks
])
def test_dense_causal_attention_bf16_several_tiles(oracle, B, H, T, N, D):
    # Context only on pre-rotated queries with a decay (ones) given, as the
    # entry point requires: several gram row blocks, ragged or whole.
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(T + N + D)
    q = oracle.round_bf16(oracle.rope_rotate(rc.sparse_relu(rng, (B, H, T, N))))
    v = oracle.round_bf16(rc.gaussian(rng, (B, 1, T, D), 1 / 16))
    announce("dense bf16", B, H, T, N, D)
    out = bd.try_fused_dense_causal_attention(dev(torch, q, torch.bfloat16),
                                              dev(torch, v, torch.bfloat16), dev(torch, np.ones(H, np.float32)))
    torch.cuda.synchronize()
    cref, _ = oracle.dense_score_f64(q, v, None, None, want_rho=False)
    assert rel_l2(host(out), cref) <= TOL_BF16


@pytest.mark.parametrize("decay", [[0.0, 0.9], [-0.9, 0.5], [-0.5, 0.0]])
def test_bf16_decay_zero_and_negative(oracle, decay):
    # Decay powers d^e as repeated products give them (recurrent.rs:415):
    # d = 0 keeps d^0 = 1 (row 0 of the readout, the carried state at e = 0)
    # and makes every higher power 0; d < 0 alternates sign.  Two intervals
    # and a carried state exercise the gram, readout and state units.
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(6100 + int(decay[0] * 10))
    B, H, T, N, D = 1, 2, 640, 512, 64
    x = oracle.round_bf16(rc.sparse_relu(rng, (B, H, T, N)))
    v = oracle.round_bf16(rc.gaussian(rng, (B, 1, T, D), 1 / 16))
    rho0 = rc.gaussian(rng, (B, H, N, D), 0.1)
    dec = np.array(decay, np.float32)
    cref, rref = oracle.recurrent_f64(oracle.rope_rotate(x, pos0=2), v, rho0, dec)
    announce("bf16 decay", decay)
    ctx, rho = _run(torch, bd, x, v, rho0, dec, torch.bfloat16, rope=(2, False))
    assert np.isfinite(ctx).all() and np.isfinite(rho).all()
    assert rel_l2(ctx, cref) <= TOL_BF16
    assert rel_l2(rho, rref) <= TOL_BF16


@pytest.mark.parametrize("B,H,Hv,T,N,D,with_rho,chunk,rope,inplace", [
    (1, 2, 1, 1100, 256, 64, True, 128, (4, False), False),    # 9 intervals, ragged last
    (1, 2, 2, 1100, 512, 320, False, 256, (9, False), False),  # two column blocks, per-head V, no rho
    (2, 2, 1, 1024, 256, 96, True, 384, (1000, True), False),  # L not a multiple of 256, fixed positions
    (1, 2, 1, 700, 256, 64, True, 256, None, False),           # pre-rotated query
    (1, 2, 1, 1100, 256, 64, True, 512, (3, False), True),     # rho updated in place
])
def test_bf16_state_carry_path(oracle, B, H, Hv, T, N, D, with_rho, chunk, rope, inplace):
    # Two or more intervals without decay run the state-carry kernel (every
    # rho block carried across the intervals in registers, bf16 snapshots at
    # the interval starts) and one launch of every interval's gram tiles and
    # readouts.
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(T + N + D + chunk)
    x, v, rho0 = _bf16_case(rng, B, H, Hv, T, N, D, with_rho)
    xb, vb = oracle.round_bf16(x), oracle.round_bf16(v)
    if rope is None:
        xb = oracle.round_bf16(oracle.rope_rotate(xb, pos0=0))
        q = xb
    else:
        q = oracle.rope_rotate(xb, pos0=rope[0], mode=1 if rope[1] else 0)
    announce("bf16 state carry", B, H, Hv, T, N, D, with_rho, chunk, rope, inplace)
    xd, vd = dev(torch, xb, torch.bfloat16), dev(torch, vb, torch.bfloat16)
    rd = dev(torch, rho0) if with_rho else None
    if rope is None:
        out = bd.try_fused_recurrent_attention(xd, vd, rd, None, inplace=inplace, chunk=chunk)
    else:
        out = bd.try_fused_recurrent_attention_rope(xd, vd, rd, None, position=rope[0], fixed=rope[1],
                                                    inplace=inplace, chunk=chunk)
    torch.cuda.synchronize()
    assert out is not None
    if inplace:
        assert out.rho.data_ptr() == rd.data_ptr()
    cref, rref = oracle.recurrent_f64(q, vb, rho0)
    e_ctx, e_rho = rel_l2(host(out.context), cref), rel_l2(host(out.rho), rref)
    print(f"rel-L2 ctx {e_ctx:.2e} rho {e_rho:.2e}")
    assert e_ctx <= TOL_BF16 and e_rho <= TOL_BF16


@pytest.mark.parametrize("B,H,Hv,T,N,D,decay,rope", [
    (1, 2, 1, 300, 256, 96, None, (17, False)),                 # ragged T inside one 512-token interval
    (1, 2, 2, 700, 512, 320, None, (5, False)),                 # three 256-row blocks, two column blocks
    (2, 2, 1, 512, 256, 64, [0.97, 0.95], (0, False)),          # decay (gram and state weights)
    (1, 2, 1, 1024, 256, 64, None, (2000, True)),               # four row blocks, fixed positions
])
def test_bf16_one_interval_cases(oracle, B, H, Hv, T, N, D, decay, rope):
    # One interval (row chunk 1024) with RoPE in the tile loads and no carried
    # state: ragged lengths, several 256-row blocks and column blocks, decay,
    # fixed positions.
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(T + N + 3 * D)
    x, v, _ = _bf16_case(rng, B, H, Hv, T, N, D, False)
    xb, vb = oracle.round_bf16(x), oracle.round_bf16(v)
    dec = np.array(decay, np.float32) if decay else None
    announce("bf16 one interval", B, H, Hv, T, N, D, decay, rope)
    out = bd.try_fused_recurrent_attention_rope(
        dev(torch, xb, torch.bfloat16), dev(torch, vb, torch.bfloat16), None,
        dev(torch, dec) if dec is not None else None, position=rope[0], fixed=rope[1], chunk=1024)
    torch.cuda.synchronize()
    assert out is not None
    q = oracle.rope_rotate(xb, pos0=rope[0], mode=1 if rope[1] else 0)
    cref, rref = oracle.recurrent_f64(q, vb, None, dec)
    e_ctx, e_rho = rel_l2(host(out.context), cref), rel_l2(host(out.rho), rref)
    print(f"rel-L2 ctx {e_ctx:.2e} rho {e_rho:.2e}")
    assert e_ctx <= TOL_BF16 and e_rho <= TOL_BF16
