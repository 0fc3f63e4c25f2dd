"""Two calls of different shapes running at once on two streams of the same
(default) priority: each stream has its own scratch, so neither disturbs the
other (the reference gives every call its own buffers, recurrent.rs:
221-359).  Both results must equal the oracle, and releasing one stream's
scratch must leave the other working."""
import numpy as np
import pytest

from tests import refcases as rc
from tests.gpu_util import TOL_BF16, announce, host, need_gpu, rel_l2

pytestmark = pytest.mark.gpu


def test_two_streams_at_once(oracle):
    torch = need_gpu()
    import burn_dragon_amd as bd
    from burn_dragon_amd import _lib
    rng = np.random.default_rng(5001)
    shapes = [(2, 2, 640, 512, 64), (1, 4, 300, 256, 96)]
    cases = []
    for (B, H, T, N, D) in shapes:
        x = oracle.round_bf16(rc.sparse_relu(rng, (B, H, T, N)))
        v = oracle.round_bf16(rc.gaussian(rng, (B, 1, T, D), 1 / 16))
        cref, rref = oracle.recurrent_f64(oracle.rope_rotate(oracle.round_bf16(x), pos0=5), v)
        cases.append((torch.from_numpy(x).cuda().to(torch.bfloat16),
                      torch.from_numpy(v).cuda().to(torch.bfloat16), cref, rref))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    announce("streams concurrent", shapes)
    outs = [[], []]
    for rep in range(3):  # launches of both streams interleave without host waits
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                outs[i].append(bd.try_fused_recurrent_attention_rope(cases[i][0], cases[i][1], position=5))
    torch.cuda.synchronize()
    for i, (_, _, cref, rref) in enumerate(cases):
        for o in outs[i]:
            assert o is not None
            assert rel_l2(host(o.context), cref) <= TOL_BF16
            assert rel_l2(host(o.rho), rref) <= TOL_BF16
        assert torch.equal(outs[i][0].context, outs[i][-1].context)

    announce("streams release")
    lib = _lib.load()
    assert lib.bdh_scratch_release(ctypes_stream(streams[0])) == _lib.BDH_OK
    with torch.cuda.stream(streams[1]):
        again = bd.try_fused_recurrent_attention_rope(cases[1][0], cases[1][1], position=5)
    with torch.cuda.stream(streams[0]):
        regrown = bd.try_fused_recurrent_attention_rope(cases[0][0], cases[0][1], position=5)
    torch.cuda.synchronize()
    assert torch.equal(again.context, outs[1][0].context)
    assert torch.equal(regrown.context, outs[0][0].context)


def ctypes_stream(s):
    import ctypes
    return ctypes.c_void_p(s.cuda_stream)
