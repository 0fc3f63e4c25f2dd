"""bdh_decode_step_noalloc (buffers in a file-scope device array, no
allocation) against bdh_decode_step (scratch-backed) through the C ABI: two
calls in a row, the second with a smaller input, each bit-identical to the
existing entry point (same kernels), with lists, RoPE, decay and streams
split into row ranges; plus the size limit."""
import ctypes

import numpy as np
import pytest

from tests import refcases as rc
from tests.gpu_util import TOL_F32, announce, dev, host, need_gpu, rel_l2

pytestmark = pytest.mark.gpu


def _call(lib, _lib, fn, torch, x, v, rho, decay, pos, lists):
    B, H, N = x.shape
    Hv, D = v.shape[1], v.shape[2]
    a = torch.empty((B, H, D), device="cuda", dtype=torch.float32)
    idx = torch.empty((B, H, N), device="cuda", dtype=torch.int32) if lists else None
    cnt = torch.empty((B, H), device="cuda", dtype=torch.int32) if lists else None
    rope = _lib.BdhRope(_lib.BDH_ROPE_SEQUENTIAL, 0, pos, 65536.0) if pos is not None else None
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    st = getattr(lib, fn)(B, H, Hv, N, D, p(x), p(v), p(rho), p(decay),
                          ctypes.byref(rope) if rope is not None else None, p(a), p(idx), p(cnt),
                          ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == _lib.BDH_OK, _lib.last_error()
    return a, idx, cnt


CASES = [
    # (B, H, Hv, N, D, pos, decay, lists): first call, then a smaller one
    ((2, 2, 1, 8192, 256, 1024, False, True), (1, 2, 2, 2048, 64, 5, False, True)),
    ((2, 4, 1, 4096, 128, 300, True, True), (1, 2, 1, 1024, 96, 7, True, False)),
    ((4, 4, 1, 8192, 256, None, False, False), (1, 1, 1, 512, 32, None, False, True)),
]


@pytest.mark.parametrize("first,second", CASES)
def test_noalloc_matches_decode_step(oracle, first, second):
    torch = need_gpu()
    from burn_dragon_amd import _lib
    lib = _lib.load()
    for k, (B, H, Hv, N, D, pos, with_decay, lists) in enumerate((first, second)):
        rng = np.random.default_rng(7000 + 10 * k + N + D)
        x = dev(torch, rc.sparse_relu(rng, (B, H, N)))
        v = dev(torch, rc.gaussian(rng, (B, Hv, D), 1 / 16))
        rho0 = rc.gaussian(rng, (B, H, N, D), 0.5)
        decay = dev(torch, np.linspace(0.95, 0.8, H).astype(np.float32)) if with_decay else None
        announce("noalloc", k, B, H, Hv, N, D, pos, with_decay, lists)
        r_ref, r_new = dev(torch, rho0), dev(torch, rho0)
        a_ref, i_ref, c_ref = _call(lib, _lib, "bdh_decode_step", torch, x, v, r_ref, decay, pos, lists)
        a_new, i_new, c_new = _call(lib, _lib, "bdh_decode_step_noalloc", torch, x, v, r_new, decay,
                                    pos, lists)
        torch.cuda.synchronize()
        assert torch.equal(a_new, a_ref)
        assert torch.equal(r_new, r_ref)
        if lists:
            assert torch.equal(i_new, i_ref) and torch.equal(c_new, c_ref)
        if pos is not None and not with_decay:
            # and against the oracle (fp32 bar)
            rho_o = rho0.copy()
            ao, io, co = oracle.decode_step_f32(host(x), host(v), rho_o, pos)
            assert rel_l2(host(a_new), ao) <= TOL_F32 and rel_l2(host(r_new), rho_o) <= TOL_F32


def test_noalloc_rejects_sizes_beyond_its_array():
    torch = need_gpu()
    from burn_dragon_amd import _lib
    lib = _lib.load()
    x = torch.zeros(1, 1, 8, device="cuda")
    p = ctypes.c_void_p(x.data_ptr())
    announce("noalloc limits")
    # latent beyond one frequency-table slot: refused before any launch
    st = lib.bdh_decode_step_noalloc(1, 1, 1, (1 << 20) + 2, 8, p, p, p, None, None, p, None, None,
                                     None)
    assert st == _lib.BDH_UNSUPPORTED and "latent" in _lib.last_error()
    # 64 streams of 65536 rows with lists: split into row ranges (two per
    # stream on a GPU of at least 128 CUs), their range lists take 16 MiB,
    # beyond the 8 MiB range region.  Every buffer has its declared size, so a
    # missed refusal would run the step and fail the assertion, not fault.
    if torch.cuda.get_device_properties(0).multi_processor_count < 128:
        pytest.skip("64 streams are not split into row ranges on fewer than 128 CUs")
    B, H, N, D = 16, 4, 1 << 16, 8
    xs = torch.zeros(B, H, N, device="cuda")
    vs = torch.zeros(B, 1, D, device="cuda")
    rho = torch.zeros(B, H, N, D, device="cuda")
    a = torch.zeros(B, H, D, device="cuda")
    idx = torch.zeros(B, H, N, device="cuda", dtype=torch.int32)
    cnt = torch.zeros(B, H, device="cuda", dtype=torch.int32)
    q = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    st = lib.bdh_decode_step_noalloc(B, H, 1, N, D, q(xs), q(vs), q(rho), None, None, q(a), q(idx),
                                     q(cnt), None)
    assert st == _lib.BDH_UNSUPPORTED and "MiB" in _lib.last_error()


def test_noalloc_graph_keeps_its_table_after_other_keys():
    # A graph captured at one (latent, theta) keeps reading that key's table
    # after eager calls at other keys: table slots are never overwritten.
    torch = need_gpu()
    from burn_dragon_amd import _lib
    lib = _lib.load()
    B, H, N, D, pos, theta = 2, 2, 3072, 64, 777, 10000.0
    rng = np.random.default_rng(7100)
    x = dev(torch, rc.sparse_relu(rng, (B, H, N)))
    v = dev(torch, rc.gaussian(rng, (B, 1, D), 1 / 16))
    rho0 = dev(torch, rc.gaussian(rng, (B, H, N, D), 0.5))
    p = lambda t: ctypes.c_void_p(t.data_ptr()) if t is not None else None  # noqa: E731
    rope = _lib.BdhRope(_lib.BDH_ROPE_SEQUENTIAL, 0, pos, theta)
    a = torch.empty((B, H, D), device="cuda", dtype=torch.float32)
    idx = torch.empty((B, H, N), device="cuda", dtype=torch.int32)
    cnt = torch.empty((B, H), device="cuda", dtype=torch.int32)

    def step(fn, rho, ao, io, co, stream):
        return getattr(lib, fn)(B, H, 1, N, D, p(x), p(v), p(rho), None, ctypes.byref(rope), p(ao),
                                p(io), p(co), ctypes.c_void_p(stream.cuda_stream))

    announce("noalloc graph", B, H, N, D, pos, theta)
    r_ref = rho0.clone()
    a_ref = torch.empty_like(a)
    i_ref, c_ref = torch.empty_like(idx), torch.empty_like(cnt)
    cur = torch.cuda.current_stream()
    assert step("bdh_decode_step", r_ref, a_ref, i_ref, c_ref, cur) == _lib.BDH_OK, _lib.last_error()
    rho = rho0.clone()
    assert step("bdh_decode_step_noalloc", rho, a, idx, cnt, cur) == _lib.BDH_OK  # uploads the table
    torch.cuda.synchronize()
    cap = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        st = step("bdh_decode_step_noalloc", rho, a, idx, cnt, cap)
    assert st == _lib.BDH_OK, _lib.last_error()
    for i, (n2, th2) in enumerate(((2048, 65536.0), (4096, 500.0), (N, 65536.0))):
        # an eager call at another key, then a replay from the same state
        x2 = dev(torch, rc.sparse_relu(rng, (1, 1, n2)))
        v2 = dev(torch, rc.gaussian(rng, (1, 1, D), 1 / 16))
        r2 = dev(torch, rc.gaussian(rng, (1, 1, n2, D), 0.5))
        a2 = torch.empty((1, 1, D), device="cuda", dtype=torch.float32)
        rope2 = _lib.BdhRope(_lib.BDH_ROPE_SEQUENTIAL, 0, 3 + i, th2)
        st = lib.bdh_decode_step_noalloc(1, 1, 1, n2, D, p(x2), p(v2), p(r2), None,
                                         ctypes.byref(rope2), p(a2), None, None,
                                         ctypes.c_void_p(cur.cuda_stream))
        assert st == _lib.BDH_OK, _lib.last_error()
        rho.copy_(rho0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(a, a_ref) and torch.equal(rho, r_ref), i
        assert torch.equal(idx, i_ref) and torch.equal(cnt, c_ref), i
