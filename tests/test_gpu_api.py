"""Behaviour of the drop-in surface on the GPU: the reference's None cases,
defaults (rho -> zeros, decay -> ones), the private rho copy vs in-place,
plan reuse, profiling counters and repeated-call memory stability
(recurrent.rs:175-259, recurrent/tests.rs:290-336)."""
import numpy as np
import pytest

from tests import refcases as rc
from tests.gpu_util import TOL_F32, announce, dev, host, need_gpu, rel_l2

pytestmark = pytest.mark.gpu


def test_none_cases_match_reference():
    torch = need_gpu()
    import burn_dragon_amd as bd
    q = torch.zeros(2, 4, 6, 16, device="cuda")
    v = torch.zeros(2, 1, 6, 24, device="cuda")
    announce("api none cases")
    assert bd.try_fused_recurrent_attention(q, v) is not None
    assert bd.try_fused_recurrent_attention(q[:, :, :0], v[:, :, :0]) is None       # zero time
    assert bd.try_fused_recurrent_attention(q, torch.zeros(2, 2, 6, 24, device="cuda")) is None
    assert bd.try_fused_recurrent_attention(q, torch.zeros(1, 1, 6, 24, device="cuda")) is None
    assert bd.try_fused_recurrent_attention(q, torch.zeros(2, 1, 5, 24, device="cuda")) is None
    assert bd.try_fused_recurrent_attention(q.half(), v.half()) is None              # dtype
    assert bd.try_fused_recurrent_attention(q.cpu(), v.cpu()) is None                # backend
    plan = bd.CompiledRecurrentAttentionPlan.new(2, 4, 1, 6, 16, 24)
    assert bd.try_fused_recurrent_attention_with_plan(q, v, None, None, plan) is not None
    bad = bd.CompiledRecurrentAttentionPlan.new(2, 4, 1, 7, 16, 24)
    assert bd.try_fused_recurrent_attention_with_plan(q, v, None, None, bad) is None


def test_defaults_and_private_rho_copy(oracle):
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(3)
    q = rc.gaussian(rng, (1, 2, 5, 8))
    v = rc.gaussian(rng, (1, 2, 5, 10))
    rho0 = rc.gaussian(rng, (1, 2, 8, 10))
    announce("api defaults")
    qd, vd, rd = dev(torch, q), dev(torch, v), dev(torch, rho0)
    # wrong-shaped rho -> zeros; wrong-shaped decay -> ones (recurrent.rs:243-250)
    out = bd.try_fused_recurrent_attention(qd, vd, torch.zeros(3, device="cuda"),
                                           torch.ones(5, device="cuda"))
    cref, rref = oracle.recurrent_f64(q, v)
    assert rel_l2(host(out.context), cref) <= TOL_F32 and rel_l2(host(out.rho), rref) <= TOL_F32
    # the caller's rho is not written ...
    out = bd.try_fused_recurrent_attention(qd, vd, rd, None)
    torch.cuda.synchronize()
    assert np.array_equal(host(rd), rho0)
    cref, rref = oracle.recurrent_f64(q, v, rho0)
    assert rel_l2(host(out.rho), rref) <= TOL_F32
    # ... unless in place is asked for
    out2 = bd.try_fused_recurrent_attention(qd, vd, rd, None, inplace=True)
    torch.cuda.synchronize()
    assert out2.rho.data_ptr() == rd.data_ptr()
    assert rel_l2(host(rd), rref) <= TOL_F32


def test_profile_counts_calls_and_launches():
    torch = need_gpu()
    import burn_dragon_amd as bd
    bd.recurrent_profile_enable(True)
    bd.recurrent_profile_reset()
    q = torch.zeros(1, 2, 4, 8, device="cuda")
    v = torch.zeros(1, 1, 4, 8, device="cuda")
    announce("api profile")
    for _ in range(3):
        bd.try_fused_recurrent_attention(q, v)
    snap = bd.recurrent_profile_snapshot()
    bd.recurrent_profile_enable(False)
    assert snap.calls == 3 and snap.launches >= 9 and snap.total_ns > 0


def test_profile_allocation_metadata_and_rollout_counters():
    """The counters recurrent.rs:206-215, 344-356 fills: a first call of a
    (latent, theta) no other test uses uploads its RoPE table and allocates;
    the same call again allocates nothing and finds the table resident; a
    T = 1 in-place fp32 step counts one resident rollout step; copy_ns stays 0
    (the private rho copy is fused into the kernel writing rho_out)."""
    torch = need_gpu()
    import ctypes
    import burn_dragon_amd as bd
    from burn_dragon_amd import _lib
    N, D, theta = 24, 8, 777.25
    rng = np.random.default_rng(31)
    x = dev(torch, rc.sparse_relu(rng, (1, 2, 3, N)))
    v = dev(torch, rc.gaussian(rng, (1, 1, 3, D)))
    x1 = dev(torch, rc.sparse_relu(rng, (1, 2, 1, N)))
    v1 = dev(torch, rc.gaussian(rng, (1, 1, 1, D)))
    side = torch.cuda.Stream()  # a fresh stream: its scratch starts empty
    side.wait_stream(torch.cuda.current_stream())
    announce("api profile counters")
    bd.recurrent_profile_enable(True)
    try:
        with torch.cuda.stream(side):
            bd.recurrent_profile_reset()
            out = bd.try_fused_recurrent_attention_rope(x, v, theta=theta)
            s1 = bd.recurrent_profile_snapshot()
            out = bd.try_fused_recurrent_attention_rope(x, v, theta=theta)
            s2 = bd.recurrent_profile_snapshot()
            rho = out.rho.clone()
            bd.try_fused_recurrent_attention_rope(x1, v1, rho, position=3, theta=theta, inplace=True)
            s3 = bd.recurrent_profile_snapshot()
        side.synchronize()
    finally:
        bd.recurrent_profile_enable(False)
        assert _lib.load().bdh_scratch_release(ctypes.c_void_p(side.cuda_stream)) == _lib.BDH_OK
    assert s1.calls == 1 and s1.transient_allocations >= 1
    assert s1.metadata_upload_bytes == 4 * N and s1.metadata_reuse_hits == 0
    assert s2.calls == 2 and s2.transient_allocations == s1.transient_allocations
    assert s2.metadata_reuse_hits == 1 and s2.metadata_reuse_bytes == 4 * N
    assert s2.metadata_upload_bytes == 4 * N
    assert s3.calls == 3 and s3.resident_rollout_steps == 1
    assert s3.copy_ns == 0 and s3.setup_ns > 0 and s3.dispatch_ns > 0


def test_memory_stays_bounded_across_repeated_calls():
    # recurrent/tests.rs:290-336: 32 calls carrying rho must not grow memory.
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(23)
    q = dev(torch, rc.gaussian(rng, (2, 4, 16, 8)))
    v = dev(torch, rc.gaussian(rng, (2, 1, 16, 12)))
    decay = dev(torch, np.array([0.9, 0.91, 0.92, 0.93], np.float32))
    rho = torch.zeros(2, 4, 8, 12, device="cuda")
    announce("api memory")
    for _ in range(2):
        rho = bd.try_fused_recurrent_attention(q, v, rho, decay).rho
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    for _ in range(32):
        rho = bd.try_fused_recurrent_attention(q, v, rho, decay).rho
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() - base <= 64 * 1024 * 1024
    assert torch.isfinite(rho).all()


def test_kernel_timing_records_the_dominant_kernels():
    # bdh_profile_kernel_timing / _get: events around prefill_mfma_kernel and
    # decode_kernel launches; nothing recorded while off.
    import ctypes
    torch = need_gpu()
    import burn_dragon_amd as bd
    from burn_dragon_amd import _lib
    lib = _lib.load()

    def got(kind):
        ms, n = ctypes.c_double(), ctypes.c_int64()
        assert lib.bdh_profile_kernel_get(kind, ctypes.byref(ms), ctypes.byref(n)) == _lib.BDH_OK
        return ms.value, n.value

    x = torch.relu(torch.randn(1, 2, 256, 256, device="cuda") - 1.0).to(torch.bfloat16)
    v = (torch.randn(1, 1, 256, 64, device="cuda") / 16).to(torch.bfloat16)
    xd = torch.relu(torch.randn(1, 2, 256, device="cuda") - 1.0)
    vd = torch.randn(1, 1, 64, device="cuda")
    announce("api kernel timing")
    assert lib.bdh_profile_kernel_timing(1) == _lib.BDH_OK
    out = bd.try_fused_recurrent_attention_rope(x, v, position=0)
    bd.decode_step(xd, vd, out.rho, position=256)
    torch.cuda.synchronize()
    pm, pn = got(_lib.BDH_KERNEL_PREFILL)
    dm, dn = got(_lib.BDH_KERNEL_DECODE)
    assert pn == 1 and pm > 0 and dn == 1 and dm > 0
    assert lib.bdh_profile_kernel_timing(0) == _lib.BDH_OK
    bd.try_fused_recurrent_attention_rope(x, v, position=0)
    torch.cuda.synchronize()
    assert got(_lib.BDH_KERNEL_PREFILL) == (0.0, 0)
