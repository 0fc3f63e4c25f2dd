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
