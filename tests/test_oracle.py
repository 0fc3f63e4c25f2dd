"""Pins the CPU oracle (oracle/bdh_oracle.c) before anything is checked
against it.  Each check is one the mathematics or the reference's own tests
fix independently of the oracle's code: the reference's known answers and
index-formula invariants, closed forms evaluated with numpy's matmul (a
library routine), textbook rotations, brute force on tiny inputs, and torch's
bf16 rounding.  A final group plants plausible mistakes in the oracle's math
(on the CPU) and shows that the checks catch them.
"""
import math

import numpy as np
import pytest

from tests import refcases as rc


def maxabs(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def closed_form_np(q, v, rho0=None, decay=None, include_diag=False):
    """numpy matmul closed form of the recurrence (f64): the independent
    formulation the dense-score executor uses (linear.rs:221-364)."""
    q = q.astype(np.float64)
    v = v.astype(np.float64)
    B, H, T, N = q.shape
    v = np.broadcast_to(v, (B, H, T, v.shape[-1])) if v.shape[1] == 1 else v
    d = np.ones(H) if decay is None else decay.astype(np.float64)
    r = np.arange(T)
    expo = r[:, None] - r[None, :]
    mask = (expo >= 0) if include_diag else (expo > 0)
    ctx = np.zeros((B, H, T, v.shape[-1]))
    rho = np.zeros((B, H, N, v.shape[-1]))
    for h in range(H):
        dec = np.where(mask, d[h] ** np.maximum(expo, 0), 0.0)
        s = q[:, h] @ np.swapaxes(q[:, h], -1, -2) * dec
        ctx[:, h] = s @ v[:, h]
        rho[:, h] = np.swapaxes(q[:, h] * (d[h] ** (T - r))[:, None], -1, -2) @ v[:, h]
        if rho0 is not None:
            ctx[:, h] += (q[:, h] * (d[h] ** r)[:, None]) @ rho0[:, h].astype(np.float64)
            rho[:, h] += rho0[:, h].astype(np.float64) * d[h] ** T
    return ctx, rho


# --- recurrence ------------------------------------------------------------

def test_signed_rho_known_answer(oracle):
    # linear.rs:433-449: q=[0.5,1], v=[2,-3,4] => rho = q^T v, ctx_0 = 0.
    q, v, rho_exp, ctx_exp = rc.signed_rho_case()
    for fn in (oracle.recurrent_f32, oracle.recurrent_f64):
        ctx, rho = fn(q, v)
        assert np.array_equal(np.asarray(rho, np.float32), rho_exp)
        assert np.array_equal(np.asarray(ctx, np.float32), ctx_exp)
        assert (np.asarray(rho) < 0).any()


def test_chunked_equals_full_without_decay(oracle):
    # linear.rs:451-483 inputs; recurrence == dense-score closed form.
    q, v, _ = rc.chunked_no_decay_case()
    ctx32, rho32 = oracle.recurrent_f32(q, v)
    ctx64, rho64 = oracle.dense_score_f64(q, v)
    cref, rref = closed_form_np(q, v)
    assert maxabs(ctx64, cref) < 1e-9 * max(1.0, np.abs(cref).max())
    assert maxabs(rho64, rref) < 1e-9 * max(1.0, np.abs(rref).max())
    # The reference's own tolerance for this invariant is 1e-4 absolute; the
    # values here reach ~1e2, so compare relatively.
    assert oracle.rel_l2(ctx32, cref) < 1e-6
    assert oracle.rel_l2(rho32, rref) < 1e-6


def test_chunked_equals_full_with_decay_and_state(oracle):
    # linear.rs:485-533 inputs (decay [0.91..0.97], rho state ramps).
    q, v, rho0, decay, _ = rc.chunked_decay_state_case()
    ctx32, rho32 = oracle.recurrent_f32(q, v, rho0, decay)
    ctx64, rho64 = oracle.recurrent_f64(q, v, rho0, decay)
    cds, rds = oracle.dense_score_f64(q, v, rho0, decay)
    cref, rref = closed_form_np(q, v, rho0, decay)
    assert maxabs(ctx64, cref) < 1e-9
    assert maxabs(rho64, rref) < 1e-9
    assert maxabs(cds, cref) < 1e-9
    assert maxabs(rds, rref) < 1e-9
    assert maxabs(ctx32, cref) < 2e-4 and maxabs(rho32, rref) < 2e-4


def test_cached_decay_inputs(oracle):
    # linear.rs:535-587 inputs: decay = exp(-slope), T=16, two heads.
    q, v, rho0, decay = rc.cached_decay_case()
    ctx32, rho32 = oracle.recurrent_f32(q, v, rho0, decay)
    cref, rref = closed_form_np(q, v, rho0, decay)
    assert maxabs(ctx32, cref) < 1e-5 and maxabs(rho32, rref) < 1e-5


def test_ramp_inputs_value_heads(oracle):
    # recurrent/tests.rs:216-245 ramps; Hv=1 must equal Hv=H with repeated v.
    q, v, rho, _, decay = rc.ramp_grad_case()
    c1, r1 = oracle.recurrent_f32(q, v, rho, decay)
    vH = np.repeat(v, 2, axis=1)
    c2, r2 = oracle.recurrent_f32(q, vH, rho, decay)
    assert np.array_equal(c1, c2) and np.array_equal(r1, r2)
    cref, rref = closed_form_np(q, v, rho, decay)
    assert maxabs(c1, cref) < 1e-6 and maxabs(r1, rref) < 1e-6


def test_brute_force_tiny(oracle):
    # Pure-Python loop over scalars on a tiny input (read-before-update).
    rng = np.random.default_rng(5)
    B, H, T, N, D = 1, 2, 4, 3, 2
    q = rng.standard_normal((B, H, T, N)).astype(np.float32)
    v = rng.standard_normal((B, 1, T, D)).astype(np.float32)
    decay = np.array([0.5, 0.25], np.float32)
    ctx, rho = oracle.recurrent_f64(q, v, None, decay)
    for h in range(H):
        state = [[0.0] * D for _ in range(N)]
        for t in range(T):
            out = [sum(state[l][e] * float(q[0, h, t, l]) for l in range(N)) for e in range(D)]
            for e in range(D):
                assert abs(out[e] - ctx[0, h, t, e]) < 1e-12
            for l in range(N):
                for e in range(D):
                    state[l][e] = (state[l][e] + float(q[0, h, t, l]) * float(v[0, 0, t, e])) * float(decay[h])
        assert maxabs(np.array(state), rho[0, h]) < 1e-12


def test_f32_mirror_matches_ndarray_baseline_bitwise(oracle):
    rng = np.random.default_rng(7)
    q = oracle.rope_rotate(rc.sparse_relu(rng, (2, 2, 8, 64)), pos0=3)
    v = rc.gaussian(rng, (2, 1, 8, 16))
    rho0 = rc.gaussian(rng, (2, 2, 64, 16))
    c1, r1 = oracle.recurrent_f32(q, v, rho0)
    c2, r2, secs = oracle.ndarray_recurrent_f32(q, v, rho0, threads=2)
    # Skipping zero rows only changes the sign of zeros.
    assert np.array_equal(c1 + 0.0, c2 + 0.0) and np.array_equal(r1 + 0.0, r2 + 0.0)
    assert secs >= 0.0
    decay = np.array([0.9, 0.8], np.float32)
    c1, r1 = oracle.recurrent_f32(q, v, rho0, decay)
    c2, r2, _ = oracle.ndarray_recurrent_f32(q, v, rho0, decay)
    assert np.array_equal(c1, c2) and np.array_equal(r1, r2)


def test_dense_score_baseline_matches_numpy_closed_form(oracle):
    """The dense-score CPU baseline (fp32, [T, T] scores materialised)
    against the f64 numpy closed form, C1's distributions at a reduced size,
    per-head and shared values; a dropped tril (diagonal kept) fails."""
    rng = np.random.default_rng(17)
    q = oracle.rope_rotate(rc.sparse_relu(rng, (1, 4, 64, 256)))
    for v in (rc.gaussian(rng, (1, 1, 64, 32)), rc.gaussian(rng, (1, 4, 64, 32))):
        ctx, secs = oracle.ndarray_dense_f32(q, v, threads=2)
        want, _ = closed_form_np(q, v)
        assert oracle.rel_l2(ctx, want) < 1e-6 and secs >= 0.0
        diag, _ = closed_form_np(q, v, include_diag=True)
        assert oracle.rel_l2(ctx, diag) > 1e-2


# --- RoPE -------------------------------------------------------------------

def test_rope_freqs_closed_form(oracle):
    for N, theta in ((8, 65536.0), (1024, 65536.0), (8192, 65536.0), (6, 10000.0)):
        f = oracle.rope_freqs(N, theta)
        i = np.arange(N)
        ref = theta ** (-(2 * (i // 2)) / N) / (2 * math.pi)
        assert np.all(f[0::2] == f[1::2])
        assert np.max(np.abs(f / ref - 1.0)) < 4e-7


def test_rope_textbook_rotation(oracle):
    # N=2, x=(1,0): rot = (cos phi, sin phi), phi = 2*pi*frac(p*f0) = frac(p/2pi)*2pi.
    for p in (0, 1, 2, 7, 100):
        out = oracle.rope_rotate(np.array([[[1.0, 0.0]]], np.float32), pos0=p)
        f0 = np.float32(1.0) / np.float32(2 * np.float32(math.pi))
        raw = np.float32(p) * f0
        phi = float((raw - np.floor(raw)) * np.float32(2 * np.float32(math.pi)))
        assert abs(out[0, 0, 0] - math.cos(phi)) < 2e-7 and abs(out[0, 0, 1] - math.sin(phi)) < 2e-7
        # (0,1) rotates to (-sin, cos): the [-odd, even] convention (attention.rs:496).
        out = oracle.rope_rotate(np.array([[[0.0, 1.0]]], np.float32), pos0=p)
        assert abs(out[0, 0, 0] + math.sin(phi)) < 2e-7 and abs(out[0, 0, 1] - math.cos(phi)) < 2e-7


def test_rope_invariants(oracle):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((3, 5, 64)).astype(np.float32)
    # position 0 is the identity, bit for bit.
    assert np.array_equal(oracle.rope_rotate(x, pos0=0, mode=1), x)
    # Sequential positions: row t is rotated by pos0 + t; Fixed: all by pos0.
    seq = oracle.rope_rotate(x, pos0=4, mode=0)
    for t in range(5):
        fixed = oracle.rope_rotate(x[:, t:t + 1], pos0=4 + t, mode=1)
        assert np.array_equal(seq[:, t:t + 1], fixed)
    # Pairwise norms are preserved.
    pr = (seq.reshape(3, 5, 32, 2) ** 2).sum(-1)
    px = (x.reshape(3, 5, 32, 2) ** 2).sum(-1)
    assert np.max(np.abs(pr - px) / (px + 1e-6)) < 1e-5
    # <R_p a, R_q b> depends on q - p only (small positions: f32 phase exact enough).
    a = x[0, 0:1][None]
    b = x[1, 0:1][None]
    d1 = float(np.sum(oracle.rope_rotate(a, 3, 1) * oracle.rope_rotate(b, 5, 1)))
    d2 = float(np.sum(oracle.rope_rotate(a, 10, 1) * oracle.rope_rotate(b, 12, 1)))
    assert abs(d1 - d2) < 1e-4 * max(1.0, abs(d1))


def test_active_rows_brute_force(oracle):
    rng = np.random.default_rng(13)
    N = 1024
    for pos in (0, 1, 5, 123, 1000, 4095):
        x = rc.sparse_relu(rng, (N,))
        r = oracle.rope_rotate(x[None, None], pos0=pos)[0, 0]
        brute = np.nonzero(r != 0.0)[0].astype(np.int32)
        act = oracle.active_rows(x, pos)
        assert np.array_equal(act, brute), pos
        if pos == 0:
            assert np.array_equal(act, np.nonzero(x)[0])


def test_active_fraction_matches_binomial(oracle):
    rng = np.random.default_rng(17)
    N = 8192
    x = rc.sparse_relu(rng, (N,))
    frac = len(oracle.active_rows(x, 77)) / N
    assert abs(frac - rc.expected_active_fraction()) < 0.01


# --- decode -----------------------------------------------------------------

def test_decode_steps_equal_prefill_recurrence(oracle):
    rng = np.random.default_rng(19)
    B, H, N, D, K, pos0 = 2, 3, 128, 16, 6, 41
    xs = rc.sparse_relu(rng, (B, H, K, N))
    vs = rc.gaussian(rng, (B, 1, K, D), 1 / 16)
    rho0 = rc.gaussian(rng, (B, H, N, D))
    q = oracle.rope_rotate(xs, pos0=pos0)
    ctx, rho_ref = oracle.recurrent_f32(q, vs, rho0)
    rho = rho0.copy()
    for k in range(K):
        a, idx, cnt = oracle.decode_step_f32(xs[:, :, k], vs[:, :, k], rho, pos0 + k)
        assert np.array_equal(a + 0.0, ctx[:, :, k] + 0.0)
        for b in range(B):
            for h in range(H):
                exp = oracle.active_rows(xs[b, h, k], pos0 + k)
                assert cnt[b, h] == len(exp)
                assert np.array_equal(idx[b, h, :cnt[b, h]], exp)
                assert np.all(idx[b, h, cnt[b, h]:] == -1)
    assert np.array_equal(rho + 0.0, rho_ref + 0.0)


# --- bf16 rounding -----------------------------------------------------------

def test_round_bf16_matches_torch(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(23)
    a = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 100,
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.4e38, -1e-40], np.float32)])
    ref = torch.from_numpy(a).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(oracle.round_bf16(a), ref)


# --- planted mistakes: the checks above must catch them ----------------------

def test_checks_catch_planted_mistakes(oracle):
    q, v, rho0, decay, _ = rc.chunked_decay_state_case()
    ctx, rho = oracle.recurrent_f64(q, v, rho0, decay)
    # (1) update-before-read: the diagonal term leaks into ctx.
    c_bad, _ = closed_form_np(q, v, rho0, decay, include_diag=True)
    assert maxabs(ctx, c_bad) > 1e-2
    # (2) decay applied before the add: rho' = rho*d + q v.
    r_bad = rho0.astype(np.float64).copy()
    for t in range(q.shape[2]):
        r_bad = r_bad * decay[None, :, None, None] + np.einsum(
            "bhn,bd->bhnd", q[:, :, t].astype(np.float64), v[:, 0, t].astype(np.float64))
    assert maxabs(rho, r_bad) > 1e-3
    # (3) transposed operand: q^T v swapped to v^T q shape cannot match.
    _, rref = closed_form_np(q, v, rho0, decay)
    assert maxabs(rho, rref) < 1e-9
    # (4) wrong RoPE sign convention ([odd, -even]) is caught by the textbook test.
    x = np.array([[[0.0, 1.0]]], np.float32)
    good = oracle.rope_rotate(x, pos0=1)
    assert good[0, 0, 0] < 0  # -sin(phi) for phi in (0, pi)


def test_alibi_helpers_match_reference_formulas():
    # default_alibi_slopes (kernel/linear_attention.rs:149-160): 1 / 2^(h/H);
    # decay = exp(-slope) (attention.rs:201-208), e.g. the cached-decay test's
    # slopes [0.25, 0.75] (linear.rs:535-587).
    import math
    from burn_dragon_amd.recurrent import alibi_decay, default_alibi_slopes
    s4 = default_alibi_slopes(4)
    assert [round(v, 6) for v in s4] == [round(2.0 ** (-h / 4), 6) for h in range(4)]
    assert s4[0] == 1.0 and default_alibi_slopes(0) == []
    d = alibi_decay([0.25, 0.75]).numpy()
    assert abs(d[0] - math.exp(-0.25)) < 1e-7 and abs(d[1] - math.exp(-0.75)) < 1e-7
