"""Pins the oracle's attention VJP (oracle.attention_vjp_f64) before the GPU
VJP is checked against it.  The reference's own test
(dense_causal_attention/tests.rs:105-183) checks its VJP against autodiff of
the stateful forward on ramp inputs; here the same inputs (and random ones)
check the closed form against central finite differences of the oracle's
f64 forward, L = sum(ctx * G).  The forward differenced is the numpy f64
closed form of the recurrence that test_oracle.py pins against the oracle's
recurrence (linear.rs:18-60, 221-364); the C recurrence itself takes f32
inputs, too coarse for a difference step.  Planted mistakes in the VJP
(on the CPU) must fail the same check."""
import numpy as np
import pytest

from tests import refcases as rc
from tests.test_oracle import closed_form_np


def _loss(oracle, q, v, rho0, decay, g):
    ctx, _ = closed_form_np(np.asarray(q, np.float64), np.asarray(v, np.float64),
                            None if rho0 is None else np.asarray(rho0, np.float64),
                            None if decay is None else np.asarray(decay, np.float64))
    return float(np.sum(ctx * g))


def _fd(oracle, name, q, v, rho0, decay, g, h=1e-5):
    """Central differences of L with respect to one input (f64 inputs)."""
    args = {"q": q, "v": v, "rho0": rho0, "decay": decay}
    x = np.array(args[name], np.float64)
    out = np.zeros_like(x)
    for i in np.ndindex(x.shape):
        xp, xm = x.copy(), x.copy()
        xp[i] += h
        xm[i] -= h
        ap, am = dict(args), dict(args)
        ap[name], am[name] = xp, xm
        out[i] = (_loss(oracle, ap["q"], ap["v"], ap["rho0"], ap["decay"], g)
                  - _loss(oracle, am["q"], am["v"], am["rho0"], am["decay"], g)) / (2 * h)
    return out


def _all_fd(oracle, q, v, rho0, decay, g):
    return (_fd(oracle, "q", q, v, rho0, decay, g), _fd(oracle, "v", q, v, rho0, decay, g),
            _fd(oracle, "decay", q, v, rho0, decay, g),
            _fd(oracle, "rho0", q, v, rho0, decay, g) if rho0 is not None else None)


def _check(got, want, tol=1e-6):
    for a, b in zip(got, want):
        if b is None:
            assert a is None
            continue
        assert np.max(np.abs(np.asarray(a) - b)) <= tol * max(1.0, np.max(np.abs(b)))


def _cases():
    # dense_causal_attention/tests.rs:105-140 ramps (grad_output i*0.02-0.1)
    q, v, _, rho_state, decay = rc.ramp_grad_case()
    g = rc.ramp_lin((1, 2, 3, 6), 0.02, -0.1)
    yield "ramps", q.astype(np.float64), v.astype(np.float64), rho_state.astype(np.float64), \
        decay.astype(np.float64), g.astype(np.float64)
    rng = np.random.default_rng(11)
    yield "random per-head values", rng.standard_normal((2, 2, 5, 4)), \
        rng.standard_normal((2, 2, 5, 3)), rng.standard_normal((2, 2, 4, 3)), \
        np.array([0.8, 0.97]), rng.standard_normal((2, 2, 5, 3))
    yield "random no state", rng.standard_normal((1, 3, 6, 5)), rng.standard_normal((1, 1, 6, 2)), \
        None, np.array([0.9, 1.0, 0.7]), rng.standard_normal((1, 3, 6, 2))


@pytest.mark.parametrize("case", list(_cases()), ids=lambda c: c[0])
def test_vjp_matches_finite_differences(oracle, case):
    _, q, v, rho0, decay, g = case
    got = oracle.attention_vjp_f64(q, v, g, decay, rho0)
    _check(got, _all_fd(oracle, q, v, rho0, decay, g))


def test_vjp_without_decay_is_the_ones_case(oracle):
    rng = np.random.default_rng(12)
    q, v, g = rng.standard_normal((1, 2, 4, 3)), rng.standard_normal((1, 1, 4, 2)), \
        rng.standard_normal((1, 2, 4, 2))
    a = oracle.attention_vjp_f64(q, v, g, None, None)
    b = oracle.attention_vjp_f64(q, v, g, np.ones(2), None)
    for x, y in zip(a[:3], b[:3]):
        assert np.allclose(x, y, rtol=0, atol=1e-12)


def test_checks_catch_planted_vjp_mistakes(oracle):
    _, q, v, rho0, decay, g = next(iter(_cases()))
    fd = _all_fd(oracle, q, v, rho0, decay, g)
    gq, gv, gd, grho = oracle.attention_vjp_f64(q, v, g, decay, rho0)
    B, H, T, N = q.shape
    # (1) grad_q without the transposed (key-side) term: Q is also the key.
    r = np.arange(T)[:, None] - np.arange(T)[None, :]
    W = np.where(r > 0, g @ np.broadcast_to(v, g.shape).transpose(0, 1, 3, 2), 0.0) * \
        np.power(decay[:, None, None], np.maximum(r, 0))[None]
    gq_bad = W @ q + (g @ rho0.transpose(0, 1, 3, 2)) * np.power(decay[:, None], np.arange(T))[None, :, :, None]
    assert np.max(np.abs(gq_bad - fd[0])) > 1e-4
    assert np.max(np.abs(gq - fd[0])) < 1e-6
    # (2) grad_v not summed over heads (value heads = 1): head 0 only.
    Sm = np.where(r > 0, q @ q.transpose(0, 1, 3, 2), 0.0) * np.power(decay[:, None, None], np.maximum(r, 0))[None]
    gv_bad = (Sm.transpose(0, 1, 3, 2) @ g)[:, :1]
    assert np.max(np.abs(gv_bad - fd[1])) > 1e-4
    # (3) state decay exponent off by one: d^(t+1) on rho0.
    grho_bad = (q * np.power(decay[:, None], np.arange(T) + 1)[None, :, :, None]).transpose(0, 1, 3, 2) @ g
    assert np.max(np.abs(grho_bad - fd[3])) > 1e-5
