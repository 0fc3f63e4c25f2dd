"""The wave-role prefill launch (burn_dragon_amd/csrc/roles_prefill.hip), which
one-interval RoPE calls without decay or a carried state take when
BDH_PREFILL_ROLES=1 is set: its cases against the oracle, and C2 at full size
against the default launch.  There rho must match bit for bit (the same
rotated bf16 words, the same MFMA instruction and order of the token steps),
while the context may differ in its last bits (the gram tiles anchor their
(cos, sin) advances at other rows), which also shows that the other launch
ran."""
import os

import numpy as np
import pytest

from tests import refcases as rc
from tests.gpu_util import TOL_BF16, announce, dev, host, need_gpu, rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture
def roles_env():
    old = os.environ.get("BDH_PREFILL_ROLES")

    def set_roles(on):
        os.environ["BDH_PREFILL_ROLES"] = "1" if on else "0"

    yield set_roles
    if old is None:
        os.environ.pop("BDH_PREFILL_ROLES", None)
    else:
        os.environ["BDH_PREFILL_ROLES"] = old


def _rope_call(torch, bd, xd, vd, pos=0, fixed=False):
    out = bd.try_fused_recurrent_attention_rope(xd, vd, None, None, position=pos, fixed=fixed)
    torch.cuda.synchronize()
    assert out is not None
    return out


@pytest.mark.parametrize("B,H,Hv,T,N,D,pos,fixed", [
    (1, 2, 1, 256, 256, 64, 0, False),      # one diagonal tile, D < 256
    (2, 2, 2, 512, 512, 96, 17, False),     # an off-diagonal tile, per-head V
    (1, 2, 1, 512, 256, 256, 1000, True),   # every token at one position
    (1, 1, 1, 512, 768, 128, 5, False),     # N a multiple of 256, not of 512
])
def test_roles_prefill_matches_oracle(oracle, roles_env, B, H, Hv, T, N, D, pos, fixed):
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(T + 3 * N + D)
    xb = oracle.round_bf16(rc.sparse_relu(rng, (B, H, T, N)))
    vb = oracle.round_bf16(rc.gaussian(rng, (B, Hv, T, D), 1 / 16))
    announce("roles prefill", B, H, Hv, T, N, D, pos, fixed)
    roles_env(True)
    out = _rope_call(torch, bd, dev(torch, xb, torch.bfloat16), dev(torch, vb, torch.bfloat16), pos, fixed)
    q = oracle.rope_rotate(xb, pos0=pos, mode=1 if fixed else 0)
    cref, rref = oracle.recurrent_f64(q, vb)
    e_ctx, e_rho = rel_l2(host(out.context), cref), rel_l2(host(out.rho), rref)
    print(f"rel-L2 ctx {e_ctx:.2e} rho {e_rho:.2e}")
    assert e_ctx <= TOL_BF16 and e_rho <= TOL_BF16


def test_roles_prefill_c2_against_the_default_launch(oracle, roles_env):
    torch = need_gpu()
    import burn_dragon_amd as bd
    B, H, T, N, D = 8, 4, 512, 8192, 256
    g = torch.Generator(device="cuda").manual_seed(rc.config_seed(2))
    x = torch.relu(torch.randn(B, H, T, N, generator=g, device="cuda") - 1.645).to(torch.bfloat16)
    v = (torch.randn(B, 1, T, D, generator=g, device="cuda") / 16).to(torch.bfloat16)
    announce("C2 roles vs default")
    roles_env(False)
    ref = _rope_call(torch, bd, x, v)
    ctx0, rho0 = ref.context.clone(), ref.rho.clone()
    roles_env(True)
    out = _rope_call(torch, bd, x, v)
    assert torch.equal(out.rho, rho0)
    assert not torch.equal(out.context, ctx0)
    assert rel_l2(host(out.context), host(ctx0)) <= 1e-3
    xs, vs = host(x[7:8, 3:4]), host(v[7:8])
    cref, _ = oracle.recurrent_f64(oracle.rope_rotate(xs, pos0=0), vs)
    assert rel_l2(host(out.context[7:8, 3:4]), cref) <= TOL_BF16
