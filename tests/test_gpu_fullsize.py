"""BASELINE configurations at full size.  The oracle checks sampled streams
(it finishes a whole stream in seconds); properties independent of size cover
every stream:
  * C2 (B8 T512 N8192 D256 bf16): prefill split in two calls carrying rho ==
    one call (state carry across chunks and intervals);
  * C3 (B64 decode): rows outside the active set are bit-identical after a
    step, sampled streams match the oracle, active sets bit-exact;
  * C4 (B1 T8192 bf16) at the automatic row chunk and at the config's chunk
    256: every chunk boundary and the final rho against the oracle for all
    four heads; with decay, two heads."""
import numpy as np
import pytest

from tests import refcases as rc
from tests.gpu_util import TOL_BF16, TOL_F32, announce, host, need_gpu, rel_l2

pytestmark = pytest.mark.gpu


def _bf16_inputs(torch, seed, B, H, T, N, D):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.relu(torch.randn(B, H, T, N, generator=g, device="cuda") - 1.645).to(torch.bfloat16)
    v = (torch.randn(B, 1, T, D, generator=g, device="cuda") / 16).to(torch.bfloat16)
    return x, v


def test_c2_prefill_full_size(oracle):
    torch = need_gpu()
    import burn_dragon_amd as bd
    B, H, T, N, D = 8, 4, 512, 8192, 256
    x, v = _bf16_inputs(torch, rc.config_seed(2), B, H, T, N, D)
    announce("C2 full prefill")
    out = bd.try_fused_recurrent_attention_rope(x, v, position=0)
    torch.cuda.synchronize()
    assert out is not None
    # sampled streams vs the oracle (bf16 inputs, f32 RoPE, f64 recurrence)
    for b, h in ((0, 0), (7, 3)):
        xs = host(x[b:b + 1, h:h + 1])
        vs = host(v[b:b + 1])
        q = oracle.rope_rotate(xs, pos0=0)
        cref, rref = oracle.recurrent_f64(q, vs)
        e1 = rel_l2(host(out.context[b:b + 1, h:h + 1]), cref)
        e2 = rel_l2(host(out.rho[b:b + 1, h:h + 1]), rref)
        print(f"C2 stream ({b},{h}) rel-L2 ctx {e1:.2e} rho {e2:.2e}")
        assert e1 <= TOL_BF16 and e2 <= TOL_BF16
    # property on every stream: two calls carrying rho == one call
    announce("C2 split prefill")
    o1 = bd.try_fused_recurrent_attention_rope(x[:, :, :256].contiguous(), v[:, :, :256].contiguous(),
                                               position=0)
    o2 = bd.try_fused_recurrent_attention_rope(x[:, :, 256:].contiguous(), v[:, :, 256:].contiguous(),
                                               o1.rho, position=256)
    torch.cuda.synchronize()
    ctx_split = torch.cat([o1.context, o2.context], dim=2)
    assert rel_l2(host(ctx_split), host(out.context)) <= TOL_BF16
    assert rel_l2(host(o2.rho), host(out.rho)) <= 1e-5   # rho sums are exact fp32 of bf16 products
    assert torch.isfinite(out.context).all() and torch.isfinite(out.rho).all()


def test_c3_decode_full_size(oracle):
    torch = need_gpu()
    import burn_dragon_amd as bd
    B, H, N, D = 64, 4, 8192, 256
    g = torch.Generator(device="cuda").manual_seed(rc.config_seed(3))
    rho = torch.randn(B, H, N, D, generator=g, device="cuda") * 0.05
    samples = ((0, 0), (31, 2), (63, 3))
    for k in range(3):
        pos = 1024 + k
        x = torch.relu(torch.randn(B, H, N, generator=g, device="cuda") - 1.645)
        v = torch.randn(B, 1, D, generator=g, device="cuda") / 16
        before = {s: host(rho[s[0], s[1]]) for s in samples}
        rho_prev = rho.clone()
        announce("C3 decode step", pos)
        out = bd.decode_step(x, v, rho, position=pos, want_active=True)
        torch.cuda.synchronize()
        cnt = out.active_cnt
        frac = float(cnt.float().mean()) / N
        assert abs(frac - rc.expected_active_fraction()) < 0.01
        # rows outside the active set: bit-identical, on every stream
        changed = (rho != rho_prev).any(dim=-1)
        idx = out.active_idx.long()
        idx = torch.where(idx >= 0, idx, torch.full_like(idx, N))  # padding -> spare column N
        act = torch.zeros(B, H, N + 1, dtype=torch.bool, device="cuda")
        act.scatter_(2, idx, True)
        act = act[:, :, :N]
        assert int(act.sum()) == int(cnt.sum())
        assert not (changed & ~act).any()
        for (b, h) in samples:
            r0 = before[(b, h)][None, None].copy()
            a_ref, idx_ref, cnt_ref = oracle.decode_step_f32(host(x[b:b + 1, h:h + 1]),
                                                             host(v[b:b + 1]), r0, pos)
            assert cnt[b, h].item() == cnt_ref[0, 0]
            assert np.array_equal(out.active_idx[b, h].cpu().numpy(), idx_ref[0, 0])
            assert rel_l2(host(out.readout[b, h]), a_ref[0, 0]) <= TOL_F32
            assert rel_l2(host(rho[b, h]), r0[0, 0]) <= TOL_F32
        del rho_prev


def test_c4_long_context_full_size(oracle):
    # The automatic row chunk (512) and the config's chunk 256 (31 bf16 rho
    # snapshots), both against one oracle run: every chunk boundary, the whole
    # context and the final rho of all four heads.
    torch = need_gpu()
    import burn_dragon_amd as bd
    B, H, T, N, D = 1, 4, 8192, 8192, 256
    x, v = _bf16_inputs(torch, rc.config_seed(4), B, H, T, N, D)
    q = oracle.rope_rotate(host(x), pos0=0)
    cref, rref = oracle.recurrent_f64(q, host(v))
    bounds = sorted({t for c in range(1, T // 256) for t in (256 * c - 1, 256 * c)} | {T - 1})
    for chunk in (0, 256):
        announce("C4 long prefill", chunk)
        out = bd.try_fused_recurrent_attention_rope(x, v, position=0, chunk=chunk)
        torch.cuda.synchronize()
        ctx = host(out.context)
        e_b = rel_l2(ctx[:, :, bounds], cref[:, :, bounds])
        e_all = rel_l2(ctx, cref)
        e_rho = rel_l2(host(out.rho), rref)
        print(f"C4 chunk {chunk} rel-L2 boundaries {e_b:.2e} all {e_all:.2e} rho {e_rho:.2e}")
        assert e_b <= TOL_BF16 and e_all <= TOL_BF16 and e_rho <= TOL_BF16
        del out


def test_c4_long_context_with_decay_full_size(oracle):
    # C4's shape with ALiBi-like decay per head (the state-carry form with
    # decay): heads 0 and 3 against the oracle, at every chunk boundary and
    # on the final rho.
    torch = need_gpu()
    import burn_dragon_amd as bd
    B, H, T, N, D = 1, 4, 8192, 8192, 256
    x, v = _bf16_inputs(torch, rc.config_seed(4) + 7, B, H, T, N, D)
    dec = np.array([0.999, 0.998, 0.997, 0.996], np.float32)
    announce("C4 long prefill with decay")
    out = bd.try_fused_recurrent_attention_rope(x, v, decay=torch.from_numpy(dec).cuda(), position=0)
    torch.cuda.synchronize()
    assert out is not None
    xh, vh = host(x), host(v)
    bounds = sorted({t for c in range(1, T // 256) for t in (256 * c - 1, 256 * c)} | {T - 1})
    for h in (0, 3):
        q = oracle.rope_rotate(xh[:, h:h + 1], pos0=0)
        cref, rref = oracle.recurrent_f64(q, vh, None, dec[h:h + 1])
        ctx = host(out.context[:, h:h + 1])
        e_b = rel_l2(ctx[:, :, bounds], cref[:, :, bounds])
        e_rho = rel_l2(host(out.rho[:, h:h + 1]), rref)
        print(f"C4 decay head {h} rel-L2 boundaries {e_b:.2e} all {rel_l2(ctx, cref):.2e} rho {e_rho:.2e}")
        assert e_b <= TOL_BF16 and rel_l2(ctx, cref) <= TOL_BF16 and e_rho <= TOL_BF16


def test_c3_decode_after_1024_token_prefill(oracle):
    # Config 3 as specified: rho prefilled by a 1024-token synthetic prefill,
    # then 32 decode steps (positions 1024..1055).  Two sampled streams follow
    # the oracle step by step from the prefilled state; every stream's rows
    # outside the step's possible active set stay bit-identical.
    torch = need_gpu()
    import burn_dragon_amd as bd
    B, H, N, D, P, K = 64, 4, 8192, 256, 1024, 32
    g = torch.Generator(device="cuda").manual_seed(rc.config_seed(3) + 1)
    xp = torch.relu(torch.randn(B, H, P, N, generator=g, device="cuda") - 1.645).to(torch.bfloat16)
    vp = (torch.randn(B, 1, P, D, generator=g, device="cuda") / 16).to(torch.bfloat16)
    announce("C3 1024-token prefill")
    pre = bd.try_fused_recurrent_attention_rope(xp, vp, position=0)
    torch.cuda.synchronize()
    assert pre is not None
    del xp, vp
    rho = pre.rho
    samples = ((0, 0), (63, 3))
    ref = {s: host(rho[s[0], s[1]])[None, None].copy() for s in samples}
    for k in range(K):
        pos = P + k
        x = torch.relu(torch.randn(B, H, N, generator=g, device="cuda") - 1.645)
        v = torch.randn(B, 1, D, generator=g, device="cuda") / 16
        rho_prev = rho.clone() if k % 8 == 0 else None
        announce("C3 decode after prefill", pos)
        out = bd.decode_step(x, v, rho, position=pos)
        torch.cuda.synchronize()
        for (b, h) in samples:
            a_ref, _, _ = oracle.decode_step_f32(host(x[b:b + 1, h:h + 1]), host(v[b:b + 1]),
                                                 ref[(b, h)], pos)
            assert rel_l2(host(out.readout[b, h]), a_ref[0, 0]) <= TOL_F32, (k, b, h)
        if rho_prev is not None:
            changed = (rho != rho_prev).any(dim=-1)
            partner = x.view(B, H, N // 2, 2).flip(-1).reshape(B, H, N)
            assert not bool((changed & ~((x != 0) | (partner != 0))).any()), k
            del rho_prev
    for (b, h) in samples:
        e = rel_l2(host(rho[b, h]), ref[(b, h)][0, 0])
        print(f"C3 stream ({b},{h}) rho after {K} steps rel-L2 {e:.2e}")
        assert e <= TOL_F32
