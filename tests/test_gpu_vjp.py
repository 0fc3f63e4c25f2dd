"""Attention VJP (fp32) on the GPU against the oracle's f64 closed form
(oracle.attention_vjp_f64, pinned by finite differences in
test_oracle_vjp.py): the reference test's ramp inputs
(dense_causal_attention/tests.rs:105-183), random shapes with shared and
per-head values, with and without an initial state, ragged tiles, sequences
longer than one 1024-token interval (the reverse scan of the state
gradient), and the recurrent backward's decay defaults.  Bar: rel-L2 <= 1e-5
(fp32)."""
import numpy as np
import pytest

from tests import refcases as rc
from tests.gpu_util import TOL_F32, announce, dev, host, need_gpu, rel_l2

pytestmark = pytest.mark.gpu


def _cmp(got, want, tol=TOL_F32):
    names = ("grad_query", "grad_value", "grad_decay", "grad_rho")
    errs = {}
    for n, a, b in zip(names, got, want):
        if b is None:
            assert a is None, n
            continue
        errs[n] = rel_l2(host(a), b)
    print("rel-L2", {k: f"{v:.2e}" for k, v in errs.items()})
    for n, e in errs.items():
        assert e <= tol, (n, e)


def test_vjp_reference_ramps(oracle):
    torch = need_gpu()
    import burn_dragon_amd as bd
    q, v, _, rho_state, decay = rc.ramp_grad_case()
    g = rc.ramp_lin((1, 2, 3, 6), 0.02, -0.1)
    announce("vjp ramps")
    out = bd.dense_causal_attention_vjp_with_initial_rho(dev(torch, g), dev(torch, q), dev(torch, v),
                                                         dev(torch, decay), dev(torch, rho_state))
    torch.cuda.synchronize()
    assert out is not None
    want = oracle.attention_vjp_f64(q, v, g, decay, rho_state)
    _cmp((out.grad_query, out.grad_value, out.grad_decay, out.grad_initial_rho), want)


@pytest.mark.parametrize("B,H,Hv,T,N,D,with_rho,decay", [
    (2, 4, 1, 16, 32, 24, True, [0.97, 0.93, 0.89, 0.85]),   # dense test shape + state
    (1, 2, 2, 70, 96, 40, False, [0.95, 0.9]),                # ragged tiles, per-head values
    (2, 2, 1, 300, 256, 96, True, [0.999, 0.99]),
    (1, 4, 1, 512, 1024, 256, False, None),                   # decay ones
    (1, 2, 1, 1100, 64, 32, True, [0.999, 0.998]),            # 2 intervals (1024 + 76): reverse scan
    (1, 2, 2, 2100, 64, 24, False, [0.9995, 0.999]),          # 3 intervals, per-head values
    (2, 1, 1, 2048, 128, 64, True, None),                     # 2 whole intervals, decay ones
])
def test_vjp_matches_oracle(oracle, B, H, Hv, T, N, D, with_rho, decay):
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(7700 + T + N)
    q = rc.gaussian(rng, (B, H, T, N), 1 / np.sqrt(N))
    v = rc.gaussian(rng, (B, Hv, T, D))
    g = rc.gaussian(rng, (B, H, T, D))
    rho0 = rc.gaussian(rng, (B, H, N, D), 0.1) if with_rho else None
    dec = np.array(decay, np.float32) if decay is not None else None
    announce("vjp", B, H, Hv, T, N, D, with_rho, decay)
    out = bd.dense_causal_attention_vjp_with_initial_rho(
        dev(torch, g), dev(torch, q), dev(torch, v), dev(torch, dec) if dec is not None else None,
        dev(torch, rho0) if rho0 is not None else None)
    torch.cuda.synchronize()
    assert out is not None
    want = oracle.attention_vjp_f64(q, v, g, dec, rho0)
    _cmp((out.grad_query, out.grad_value, out.grad_decay, out.grad_initial_rho), want)


def test_recurrent_vjp_defaults_and_state(oracle):
    # The recurrent backward: decay absent (ones), the incoming rho's
    # gradient, and its decay guard (equal to the dense one away from 0).
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(7801)
    B, H, T, N, D = 2, 2, 40, 64, 32
    q = rc.gaussian(rng, (B, H, T, N), 0.2)
    v = rc.gaussian(rng, (B, 1, T, D))
    g = rc.gaussian(rng, (B, H, T, D))
    rho = rc.gaussian(rng, (B, H, N, D), 0.1)
    announce("recurrent vjp")
    out = bd.recurrent_attention_vjp(dev(torch, g), dev(torch, q), dev(torch, v), dev(torch, rho))
    torch.cuda.synchronize()
    want = oracle.attention_vjp_f64(q, v, g, None, rho, safe="recurrent")
    _cmp((out.grad_query, out.grad_value, out.grad_decay, out.grad_rho), want)
    out = bd.recurrent_attention_vjp(dev(torch, g), dev(torch, q), dev(torch, v), None,
                                     dev(torch, np.array([0.9, 0.8], np.float32)))
    torch.cuda.synchronize()
    assert out.grad_rho is None
    want = oracle.attention_vjp_f64(q, v, g, np.array([0.9, 0.8]), None, safe="recurrent")
    _cmp((out.grad_query, out.grad_value, out.grad_decay, None), want)


def test_vjp_none_cases():
    torch = need_gpu()
    import burn_dragon_amd as bd
    q = torch.zeros(1, 2, 8, 16, device="cuda")
    v = torch.zeros(1, 1, 8, 4, device="cuda")
    g = torch.zeros(1, 2, 8, 4, device="cuda")
    d = torch.ones(2, device="cuda")
    announce("vjp none cases")
    assert bd.dense_causal_attention_vjp(g, q, v, d) is not None
    assert bd.dense_causal_attention_vjp(g.bfloat16(), q.bfloat16(), v.bfloat16(), d) is None
    assert bd.dense_causal_attention_vjp(g, q, torch.zeros(1, 3, 8, 4, device="cuda"), d) is None
    assert bd.dense_causal_attention_vjp(g, q, v, torch.ones(3, device="cuda")) is None
    # Any length is served (five intervals here); zero inputs give zero gradients.
    big = torch.zeros(1, 1, 4097, 8, device="cuda")
    out = bd.dense_causal_attention_vjp(torch.zeros(1, 1, 4097, 4, device="cuda"), big,
                                        torch.zeros(1, 1, 4097, 4, device="cuda"), torch.ones(1, device="cuda"))
    torch.cuda.synchronize()
    assert out is not None
    assert not out.grad_query.any() and not out.grad_value.any() and not out.grad_decay.any()


def test_recurrent_vjp_over_several_intervals(oracle):
    # The recurrent backward past one interval: the incoming rho's gradient
    # comes back through three interval states.
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(7901)
    B, H, T, N, D = 1, 2, 2500, 64, 32
    q = rc.gaussian(rng, (B, H, T, N), 0.1)
    v = rc.gaussian(rng, (B, 1, T, D))
    g = rc.gaussian(rng, (B, H, T, D))
    rho = rc.gaussian(rng, (B, H, N, D), 0.1)
    dec = np.array([0.9993, 0.9985], np.float32)
    announce("recurrent vjp intervals", T)
    out = bd.recurrent_attention_vjp(dev(torch, g), dev(torch, q), dev(torch, v), dev(torch, rho),
                                     dev(torch, dec))
    torch.cuda.synchronize()
    assert out is not None
    gq, gv, gd, gr = oracle.attention_vjp_f64(q, v, g, dec, rho, safe="recurrent")
    _cmp((out.grad_query, out.grad_value, out.grad_decay, out.grad_rho), (gq, gv, gd, gr))
