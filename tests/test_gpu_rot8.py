"""The hand-written RoPE rotation of the bf16 prefill (rot8_bf16 / rot8_f32,
three-operand v_dot2_f32_bf16 with neg_hi and hand-placed wait states)
against the same rotation through the compiler's dot-product builtin, bit
for bit, and against an exact scalar rotation: the two products of bf16
values are exact in f64 and so is their sum.  v_dot2_f32_bf16 adds its
accumulator (+0.0 here), so an exact -0 comes out +0; its f32 result is
within one ulp of the exact sum rounded once (measured on MI355X: 582 of
2,097,152 lanes of this sample sit one ulp away, the rest are the correctly
rounded value), and the bf16 words the prefill stores equal the exact
rotation rounded to nearest even in every lane of this sample.  262,144
chunks of random words, plus signed zeros."""
import ctypes

import numpy as np
import pytest

from tests.gpu_util import announce, need_gpu

pytestmark = pytest.mark.gpu


def _bf16_bits(a):
    """f32 -> bf16 bits, round to nearest even (values are finite)."""
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint32)


def _from_bf16(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def test_rot8_asm_matches_builtin_and_exact_rotation():
    torch = need_gpu()
    from burn_dragon_amd import _lib
    lib = _lib.load()
    rng = np.random.default_rng(99)
    n = 1 << 18
    xv = rng.standard_normal(n * 8).astype(np.float32)
    xv[rng.random(n * 8) < 0.3] = 0.0
    xv[:8] = -0.0
    ang = rng.uniform(0, 2 * np.pi, n * 4)
    cs = np.empty(n * 8, np.float32)
    cs[0::2], cs[1::2] = np.cos(ang), np.sin(ang)
    xb, cb = _bf16_bits(xv), _bf16_bits(cs)
    xw = (xb[0::2] | (xb[1::2] << 16)).astype(np.uint32)   # (even lo, odd hi) per pair
    cw = (cb[0::2] | (cb[1::2] << 16)).astype(np.uint32)   # (cos lo, sin hi)
    dx = torch.from_numpy(xw.view(np.int32)).cuda()
    dc = torch.from_numpy(cw.view(np.int32)).cuda()
    ba = torch.empty(n * 4, dtype=torch.int32, device="cuda")
    bb = torch.empty_like(ba)
    fa = torch.empty(n * 8, dtype=torch.float32, device="cuda")
    fb = torch.empty_like(fa)
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    announce("rot8 selftest", n)
    st = lib.bdh_selftest_rot8(p(dx), p(dc), p(ba), p(bb), p(fa), p(fb), n,
                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == _lib.BDH_OK, _lib.last_error()
    torch.cuda.synchronize()
    assert torch.equal(ba, bb), "asm bf16 rotation differs from the builtin"
    assert torch.equal(fa.view(torch.int32), fb.view(torch.int32)), "asm f32 rotation differs"
    # exact scalar rotation: even' = e c - o s, odd' = o c + e s
    e, o = _from_bf16(xb[0::2]).astype(np.float64), _from_bf16(xb[1::2]).astype(np.float64)
    c, s = _from_bf16(cb[0::2]).astype(np.float64), _from_bf16(cb[1::2]).astype(np.float64)
    ref = np.empty(n * 8, np.float32)
    ref[0::2] = ((e * c - o * s) + 0.0).astype(np.float32)
    ref[1::2] = ((o * c + e * s) + 0.0).astype(np.float32)
    got = fa.cpu().numpy()
    assert not np.signbit(got[got == 0]).any(), "a zero result kept its sign"
    ulp = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert ulp.max() <= 1, np.argwhere(ulp > 1)[:5]
    assert np.count_nonzero(ulp) < got.size // 1000, np.count_nonzero(ulp)
    got_b = ba.cpu().numpy().view(np.uint32)
    ref_b = _bf16_bits(ref)
    assert np.array_equal(got_b & 0xFFFF, ref_b[0::2]) and np.array_equal(got_b >> 16, ref_b[1::2])
