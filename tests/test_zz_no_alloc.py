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
    # latent beyond the frequency-table region: refused before any launch
    st = lib.bdh_decode_step_noalloc(1, 1, 1, (1 << 20) + 2, 8, p, p, p, None, None, p, None, None,
                                     None)
    assert st == _lib.BDH_UNSUPPORTED and "latent" in _lib.last_error()
    # range lists of 64 streams split into row ranges, 2^20 rows each
    # (256 MiB), exceed the array: refused before any launch
    st = lib.bdh_decode_step_noalloc(16, 4, 1, 1 << 20, 8, p, p, p, None, None, p, p, None, None)
    assert st == _lib.BDH_UNSUPPORTED and "MiB" in _lib.last_error()
