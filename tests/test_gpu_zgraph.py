"""HIP graph capture of the bf16 prefill.

Scratch is kept per stream: the capture stream is warmed by one eager call,
then captured.  Between replays run eager calls at other positions and at a
larger T on the capture stream itself, which grows that stream's scratch:
the buffers the graph holds are retired, not freed, so every replay still
equals the eager result."""
import pytest

from tests.gpu_util import announce, need_gpu

pytestmark = pytest.mark.gpu


def test_prefill_replays_from_a_hip_graph():
    torch = need_gpu()
    import burn_dragon_amd as bd
    g = torch.Generator(device="cuda").manual_seed(4)
    x = torch.relu(torch.randn(2, 2, 300, 512, generator=g, device="cuda") - 1.5).to(torch.bfloat16)
    v = (torch.randn(2, 1, 300, 64, generator=g, device="cuda") / 16).to(torch.bfloat16)
    xl = torch.relu(torch.randn(2, 2, 1100, 512, generator=g, device="cuda") - 1.5).to(torch.bfloat16)
    vl = (torch.randn(2, 1, 1100, 64, generator=g, device="cuda") / 16).to(torch.bfloat16)
    announce("api graph replay")
    ref = bd.try_fused_recurrent_attention_rope(x, v, position=3)
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        bd.try_fused_recurrent_attention_rope(x, v, position=3)  # grows this stream's scratch
    torch.cuda.current_stream().wait_stream(cap)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        out = bd.try_fused_recurrent_attention_rope(x, v, position=3)
    assert out is not None
    for i in range(4):
        out.context.zero_()
        out.rho.zero_()
        bd.try_fused_recurrent_attention_rope(x, v, position=7)  # eager work between replays
        with torch.cuda.stream(cap):
            # a larger shape on the capture stream: its scratch grows
            big = bd.try_fused_recurrent_attention_rope(xl, vl, position=i)
        torch.cuda.synchronize()
        assert big is not None
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.context, ref.context) and torch.equal(out.rho, ref.rho), i


def test_capture_without_warm_scratch_is_refused():
    # A stream whose scratch would have to grow during capture gets the
    # reference's None (BDH_UNSUPPORTED), not an allocation inside the graph.
    torch = need_gpu()
    import burn_dragon_amd as bd
    from burn_dragon_amd import _lib
    x = torch.relu(torch.randn(1, 2, 256, 512, device="cuda") - 1.5).to(torch.bfloat16)
    v = (torch.randn(1, 1, 256, 64, device="cuda") / 16).to(torch.bfloat16)
    bd.try_fused_recurrent_attention_rope(x, v, position=0)  # frequency table resident
    torch.cuda.synchronize()
    cold = torch.cuda.Stream()
    announce("api capture cold stream")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cold):
        out = bd.try_fused_recurrent_attention_rope(x, v, position=0)
    assert out is None
    assert "capture" in _lib.last_error()
    del graph
    torch.cuda.synchronize()


def test_replay_on_another_stream_overlaps_eager_work_on_the_capture_stream(oracle):
    # A graph captured on stream A is replayed on stream B while an eager call
    # of the same shape runs on A, with no synchronisation between the two:
    # the eager call takes fresh scratch (the captured set belongs to the
    # graph), so both results are exact.
    import numpy as np
    torch = need_gpu()
    import burn_dragon_amd as bd
    from tests.gpu_util import TOL_BF16, dev, host, rel_l2
    rng = np.random.default_rng(41)
    B, H, T, N, D = 4, 4, 512, 2048, 128

    def inputs():
        x = oracle.round_bf16(np.maximum(rng.standard_normal((B, H, T, N), dtype=np.float32) - 1.645,
                                         0))
        v = oracle.round_bf16(rng.standard_normal((B, 1, T, D), dtype=np.float32) / 16)
        return x, v

    (xa, va), (xb, vb) = inputs(), inputs()
    ta, tva = dev(torch, xa, torch.bfloat16), dev(torch, va, torch.bfloat16)
    tb, tvb = dev(torch, xb, torch.bfloat16), dev(torch, vb, torch.bfloat16)
    announce("graph replay on B, eager on A", B, H, T, N, D)
    ref_a = bd.try_fused_recurrent_attention_rope(ta, tva, position=11)
    ref_b = bd.try_fused_recurrent_attention_rope(tb, tvb, position=5)
    stream_a, stream_b = torch.cuda.Stream(), torch.cuda.Stream()
    stream_a.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream_a):
        bd.try_fused_recurrent_attention_rope(tb, tvb, position=5)  # warms A's scratch
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream_a):
        out = bd.try_fused_recurrent_attention_rope(tb, tvb, position=5)
    assert out is not None
    torch.cuda.synchronize()
    for i in range(3):
        with torch.cuda.stream(stream_a):
            eager = bd.try_fused_recurrent_attention_rope(ta, tva, position=11)
        with torch.cuda.stream(stream_b):
            graph.replay()
        torch.cuda.synchronize()
        assert eager is not None
        assert torch.equal(eager.context, ref_a.context) and torch.equal(eager.rho, ref_a.rho), i
        assert torch.equal(out.context, ref_b.context) and torch.equal(out.rho, ref_b.rho), i
    # and the exact results match the oracle
    for x, v, pos, r in ((xa, va, 11, ref_a), (xb, vb, 5, ref_b)):
        c_ref, rho_ref = oracle.recurrent_f64(oracle.rope_rotate(x, pos0=pos), v)
        assert rel_l2(host(r.context), c_ref) <= TOL_BF16
        assert rel_l2(host(r.rho), rho_ref) <= TOL_BF16
