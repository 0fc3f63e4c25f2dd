"""HIP graph capture of the bf16 prefill: replays interleaved with eager
calls at other positions, so the RoPE table (kept across calls and named by
a key in device memory) is rebuilt and reused in both directions."""
import pytest

from tests.gpu_util import announce, need_gpu

pytestmark = pytest.mark.gpu


def test_prefill_replays_from_a_hip_graph():
    # The bf16 RoPE prefill records no memset and allocates nothing once its
    # scratch is warm, so it can be captured; every replay (with eager work
    # and synchronisations between them) must equal the eager result.
    torch = need_gpu()
    import burn_dragon_amd as bd
    g = torch.Generator(device="cuda").manual_seed(4)
    x = torch.relu(torch.randn(2, 2, 300, 512, generator=g, device="cuda") - 1.5).to(torch.bfloat16)
    v = (torch.randn(2, 1, 300, 64, generator=g, device="cuda") / 16).to(torch.bfloat16)
    announce("api graph replay")
    ref = bd.try_fused_recurrent_attention_rope(x, v, position=3)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        bd.try_fused_recurrent_attention_rope(x, v, position=3)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = bd.try_fused_recurrent_attention_rope(x, v, position=3)
    for i in range(3):
        out.context.zero_()
        out.rho.zero_()
        bd.try_fused_recurrent_attention_rope(x, v, position=7)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.context, ref.context) and torch.equal(out.rho, ref.rho), i
