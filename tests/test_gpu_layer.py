"""Low-rank layer body (bdh_lowrank_layer_fwd) vs the CPU oracle
(oracle.lowrank_layer_f64, pinned in tests/test_oracle_layer.py): rel-L2 <=
1e-2 on next and on rho, bf16 MFMA with fp32 accumulation.  The oracle gets
the bf16-rounded weights the packed layout holds and the f32 layer input."""
import numpy as np
import pytest

from tests.gpu_util import TOL_BF16, announce, dev, host, need_gpu, rel_l2

pytestmark = pytest.mark.gpu


def _case(rng, B, H, T, N, D):
    cur = rng.standard_normal((B, T, D)).astype(np.float32)
    enc = (rng.standard_normal((H, D, N)) * 0.02 * 8 / np.sqrt(D / 64)).astype(np.float32)
    encv = (rng.standard_normal((H, D, N)) * 0.02 * 8 / np.sqrt(D / 64)).astype(np.float32)
    dec = (rng.standard_normal((H * N, D)) * 0.02).astype(np.float32)
    return cur, enc, encv, dec


@pytest.mark.parametrize("B,H,T,N,D,pos,want_rho", [
    (2, 2, 200, 256, 64, 5, False),     # ragged rows (M = 400), context-only attention
    (1, 4, 300, 512, 128, 0, True),     # rho out: one 300-token state interval
    (1, 2, 640, 256, 256, 17, True),    # two state intervals (512 + 128), D = 256
    (1, 2, 24, 256, 64, 11, True),      # few-row GEMMs, two 16-row blocks
    (3, 2, 16, 512, 128, 2, False),     # few-row GEMMs, four 16-row blocks (M = 48)
    (1, 1, 40, 256, 2048, 3, True),     # widest embd: 32 values a lane in the LayerNorms
    (2, 1, 160, 256, 1024, 0, False),   # wide embd on the 256 x 128 tiles (M = 320)
    (1, 2, 1000, 512, 64, 3, False),    # context only over 4 gram row blocks, the last ragged
    # T % 256 == 0 and D <= 256: GEMM Y fused into the decoder (y never stored)
    (2, 2, 256, 256, 64, 5, False),     # 4 latent chunks over 2 heads in one workgroup per token tile
    (1, 3, 512, 256, 192, 3, True),     # D = 192 (decoder rows past D clamped), 6 chunks over 3 heads
    (1, 4, 512, 512, 256, 0, True),     # D = 256, 16 chunks in 4 splits
    (1, 2, 512, 512, 128, 4, False),    # context only on 4-wave gram tiles: an off-diagonal tile, 4 N ranges
])
def test_layer_matches_oracle(oracle, B, H, T, N, D, pos, want_rho):
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(B * 1000 + T + N + D)
    cur, enc, encv, dec = _case(rng, B, H, T, N, D)
    w = bd.LowRankWeights.pack(dev(torch, enc[None]), dev(torch, encv[None]), dev(torch, dec))
    assert w is not None
    announce("layer", B, H, T, N, D, pos, want_rho)
    out = bd.lowrank_layer_forward(dev(torch, cur), w, position=pos, want_rho=want_rho)
    torch.cuda.synchronize()
    assert out is not None
    nref, rref = oracle.lowrank_layer_f64(cur, oracle.round_bf16(enc), oracle.round_bf16(encv),
                                          oracle.round_bf16(dec), pos0=pos)
    e_next = rel_l2(host(out.next), nref)
    msg = f"rel-L2 next {e_next:.2e}"
    if want_rho:
        e_rho = rel_l2(host(out.rho), rref)
        msg += f" rho {e_rho:.2e}"
        assert e_rho <= TOL_BF16, msg
    print(msg)
    assert e_next <= TOL_BF16, msg


def test_layer_without_rope(oracle):
    # rope = NULL: the attention sees x itself (no rotated copy is written).
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(8)
    B, H, T, N, D = 1, 2, 256, 256, 64
    cur, enc, encv, dec = _case(rng, B, H, T, N, D)
    w = bd.LowRankWeights.pack(dev(torch, enc), dev(torch, encv), dev(torch, dec))
    announce("layer no rope", B, H, T, N, D)
    out = bd.lowrank_layer_forward(dev(torch, cur), w, position=None)
    torch.cuda.synchronize()
    nref, _ = oracle.lowrank_layer_f64(cur, oracle.round_bf16(enc), oracle.round_bf16(encv),
                                       oracle.round_bf16(dec), pos0=None)
    assert rel_l2(host(out.next), nref) <= TOL_BF16


def test_layer_pack_layouts(oracle):
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(2)
    H, D, N = 2, 64, 256
    enc = rng.standard_normal((H, D, N)).astype(np.float32)
    encv = rng.standard_normal((H, D, N)).astype(np.float32)
    dec = rng.standard_normal((H * N, D)).astype(np.float32)
    announce("layer pack")
    w = bd.LowRankWeights.pack(dev(torch, enc), dev(torch, encv), dev(torch, dec))
    torch.cuda.synchronize()
    assert np.array_equal(host(w.encoder), oracle.round_bf16(enc.transpose(0, 2, 1)))
    assert np.array_equal(host(w.encoder_v), oracle.round_bf16(encv.transpose(0, 2, 1)))
    # decoder: the transpose [D, H N] in 128-latent chunks, [H N / 128, D, 128]
    chunks = oracle.round_bf16(dec.T).reshape(D, H * N // 128, 128).transpose(1, 0, 2)
    assert np.array_equal(host(w.decoder), chunks)


def test_layer_unsupported_shapes_return_none():
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(3)
    # embd not a multiple of 64 -> None (the caller keeps its Burn-op path)
    cur, enc, encv, dec = _case(rng, 1, 2, 64, 256, 96)
    w = bd.LowRankWeights.pack(dev(torch, enc), dev(torch, encv), dev(torch, dec))
    announce("layer unsupported")
    assert bd.lowrank_layer_forward(dev(torch, cur), w) is None
    # embd mismatch between input and weights -> None
    cur2 = rng.standard_normal((1, 64, 64)).astype(np.float32)
    assert bd.lowrank_layer_forward(dev(torch, cur2), w) is None


@pytest.mark.parametrize("T", [130, 256])  # 256: GEMM Y fused into the decoder
def test_model_forward_matches_oracle(oracle, T):
    # embed -> LN -> 2 shared layers -> logits (vocab 256), every step on the GPU.
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(77)
    B, V, D, H, N, L = 2, 256, 64, 2, 256, 2
    _, enc, encv, dec = _case(rng, 1, H, 1, N, D)
    embed = (rng.standard_normal((V, D)) * 0.02).astype(np.float32)
    head = (rng.standard_normal((D, V)) * 0.02).astype(np.float32)
    tokens = rng.integers(0, V, (B, T)).astype(np.int32)
    w = bd.pack_model(dev(torch, embed), dev(torch, enc[None]), dev(torch, encv[None]),
                      dev(torch, dec), dev(torch, head), L)
    assert w is not None
    announce("model forward", B, T, V, D, H, N, L)
    logits = bd.model_forward_logits(dev(torch, tokens), w, position=0)
    torch.cuda.synchronize()
    assert logits is not None
    ref = oracle.model_forward_f64(tokens, embed, oracle.round_bf16(enc), oracle.round_bf16(encv),
                                   oracle.round_bf16(dec), oracle.round_bf16(head), L)
    e = rel_l2(host(logits), ref)
    print(f"rel-L2 logits {e:.2e}")
    assert e <= TOL_BF16


@pytest.mark.parametrize("B,H,T,N,D,pos,mode", [
    (2, 2, 150, 256, 64, 7, "copy"),       # carried rho in, successor to a new buffer
    (1, 2, 600, 256, 128, 3, "inplace"),   # two state intervals, successor over rho
    (2, 2, 100, 256, 64, 4, "nokeep"),     # carried rho, successor not kept
    (3, 2, 1, 512, 128, 9, "inplace"),     # one token in place: the sparse decode step
    (3, 2, 1, 512, 128, 9, "copy"),        # one token to a new buffer: the MFMA path
])
def test_layer_carried_state_matches_oracle(oracle, B, H, T, N, D, pos, mode):
    # LayerState.rho in (sequence_dispatch.rs:83-136): the attention starts
    # from rho0 instead of zeros.
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(B * 100 + T + N + D)
    cur, enc, encv, dec = _case(rng, B, H, T, N, D)
    rho0 = (rng.standard_normal((B, H, N, D)) * 0.05).astype(np.float32)
    w = bd.LowRankWeights.pack(dev(torch, enc[None]), dev(torch, encv[None]), dev(torch, dec))
    rho_t = dev(torch, rho0)
    announce("layer carried state", B, H, T, N, D, pos, mode)
    out = bd.lowrank_layer_forward(dev(torch, cur), w, position=pos, rho=rho_t,
                                   inplace=mode == "inplace", want_rho=mode == "copy")
    torch.cuda.synchronize()
    assert out is not None
    nref, rref = oracle.lowrank_layer_f64(cur, oracle.round_bf16(enc), oracle.round_bf16(encv),
                                          oracle.round_bf16(dec), pos0=pos, rho0=rho0)
    e_next = rel_l2(host(out.next), nref)
    msg = f"rel-L2 next {e_next:.2e}"
    if mode == "nokeep":
        assert out.rho is None
    else:
        e_rho = rel_l2(host(out.rho), rref)
        msg += f" rho {e_rho:.2e}"
        assert e_rho <= TOL_BF16, msg
    if mode != "inplace":
        assert np.array_equal(host(rho_t), rho0)  # the caller's state is not written
    print(msg)
    assert e_next <= TOL_BF16, msg


def test_model_incremental_matches_full_sequence(oracle):
    # linear_attention_incremental_forward_matches_full_sequence
    # (dragon.rs:5028-5057): tokens 1..6 one per forward_with_state call from
    # the initial state equal the full-sequence forward; position ends at 6.
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(92)
    V, D, H, N, L = 256, 64, 2, 256, 2
    _, enc, encv, dec = _case(rng, 1, H, 1, N, D)
    embed = (rng.standard_normal((V, D)) * 0.02).astype(np.float32)
    head = (rng.standard_normal((D, V)) * 0.02).astype(np.float32)
    tokens = np.array([[1, 2, 3, 4, 5, 6]], np.int32)
    w = bd.pack_model(dev(torch, embed), dev(torch, enc[None]), dev(torch, encv[None]),
                      dev(torch, dec), dev(torch, head), L)
    tok = dev(torch, tokens)
    announce("model incremental vs full", V, D, H, N, L)
    full = bd.model_forward_logits(tok, w, position=0)
    state = bd.new_model_state(w, 1, tok.device)
    pieces = [bd.model_forward_logits(tok[:, i:i + 1], w, state=state) for i in range(6)]
    torch.cuda.synchronize()
    assert state.position == 6
    inc = np.concatenate([host(p) for p in pieces], axis=1)
    ref = oracle.model_forward_f64(tokens, embed, oracle.round_bf16(enc), oracle.round_bf16(encv),
                                   oracle.round_bf16(dec), oracle.round_bf16(head), L)
    e_full, e_inc, e_pair = rel_l2(host(full), ref), rel_l2(inc, ref), rel_l2(inc, host(full))
    print(f"rel-L2 full {e_full:.2e}, incremental {e_inc:.2e}, incremental vs full {e_pair:.2e}")
    assert e_full <= TOL_BF16 and e_inc <= TOL_BF16 and e_pair <= TOL_BF16


def test_model_prompt_then_decode_matches_oracle(oracle):
    # A prompt through forward_with_state, then one token per call carrying
    # every layer's rho and the position (the generation loop), against one
    # oracle forward over the whole sequence.
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(91)
    B, T0, steps, V, D, H, N, L = 2, 40, 3, 256, 64, 2, 256, 2
    _, enc, encv, dec = _case(rng, 1, H, 1, N, D)
    embed = (rng.standard_normal((V, D)) * 0.02).astype(np.float32)
    head = (rng.standard_normal((D, V)) * 0.02).astype(np.float32)
    tokens = rng.integers(0, V, (B, T0 + steps)).astype(np.int32)
    w = bd.pack_model(dev(torch, embed), dev(torch, enc[None]), dev(torch, encv[None]),
                      dev(torch, dec), dev(torch, head), L)
    tok = dev(torch, tokens)
    state = bd.new_model_state(w, B, tok.device)
    announce("model prompt + decode", B, T0, steps, V, D, H, N, L)
    parts = [bd.model_forward_logits(tok[:, :T0], w, state=state)]
    for t in range(T0, T0 + steps):
        parts.append(bd.model_forward_logits(tok[:, t:t + 1], w, state=state))
    torch.cuda.synchronize()
    assert all(p is not None for p in parts) and state.position == T0 + steps
    got = np.concatenate([host(p) for p in parts], axis=1)
    ref = oracle.model_forward_f64(tokens, embed, oracle.round_bf16(enc), oracle.round_bf16(encv),
                                   oracle.round_bf16(dec), oracle.round_bf16(head), L)
    e_all, e_steps = rel_l2(got, ref), rel_l2(got[:, T0:], ref[:, T0:])
    print(f"rel-L2 logits {e_all:.2e}, decoded tokens {e_steps:.2e}")
    assert e_all <= TOL_BF16 and e_steps <= TOL_BF16


@pytest.mark.parametrize("B,H,T,N,D,pos,mode,mask_kind", [
    (1, 2, 300, 512, 128, 3, "copy", "blocks"),     # 256 x 128 tiles, block-sparse latent mask
    (2, 2, 24, 256, 64, 5, "copy", "values"),       # few-row GEMMs, a mask of other values
    (3, 2, 1, 512, 128, 9, "inplace", "blocks"),    # one token in place: the sparse decode step
    (1, 2, 640, 256, 256, 0, "copy", None),         # the threshold alone, two state intervals
    (1, 2, 512, 256, 128, 6, "copy", "values"),     # fused Y and decoder: mask and threshold in its epilogue
])
def test_layer_threshold_and_mask_match_oracle(oracle, B, H, T, N, D, pos, mode, mask_kind):
    # relu_threshold and the sparse latent mask in both projections
    # (relu_lowrank.rs reference_forward; residual_stream.rs:377-470) against
    # the oracle pinned by scalar loops in tests/test_oracle_layer.py.
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng = np.random.default_rng(B * 300 + T + N + D)
    cur, enc, encv, dec = _case(rng, B, H, T, N, D)
    rho0 = (rng.standard_normal((B, H, N, D)) * 0.05).astype(np.float32)
    th = 0.4
    if mask_kind == "blocks":
        mask = oracle.block_pattern_mask(N, 64, {b for b in range(N // 64) if b % 3 != 1})
    elif mask_kind == "values":
        mask = rng.choice([0.0, 0.5, 1.0, 1.5], N).astype(np.float32)
    else:
        mask = None
    w = bd.LowRankWeights.pack(dev(torch, enc[None]), dev(torch, encv[None]), dev(torch, dec))
    rho_t = dev(torch, rho0)
    announce("layer threshold mask", B, H, T, N, D, pos, mode, mask_kind)
    out = bd.lowrank_layer_forward(dev(torch, cur), w, position=pos, rho=rho_t,
                                   inplace=mode == "inplace", want_rho=mode == "copy",
                                   relu_threshold=th,
                                   latent_mask=None if mask is None else dev(torch, mask[None, None, None]))
    torch.cuda.synchronize()
    assert out is not None
    nref, rref = oracle.lowrank_layer_f64(cur, oracle.round_bf16(enc), oracle.round_bf16(encv),
                                          oracle.round_bf16(dec), pos0=pos, rho0=rho0,
                                          relu_threshold=th, latent_mask=mask)
    plain, _ = oracle.lowrank_layer_f64(cur, oracle.round_bf16(enc), oracle.round_bf16(encv),
                                        oracle.round_bf16(dec), pos0=pos, rho0=rho0)
    e_next, e_rho = rel_l2(host(out.next), nref), rel_l2(host(out.rho), rref)
    print(f"rel-L2 next {e_next:.2e} rho {e_rho:.2e} (vs the unmasked layer "
          f"{rel_l2(nref, plain):.2e})")
    assert rel_l2(nref, plain) > 5 * TOL_BF16  # the options change the output
    assert e_next <= TOL_BF16 and e_rho <= TOL_BF16


def test_layer_options_are_validated():
    import ctypes
    torch = need_gpu()
    import burn_dragon_amd as bd
    from burn_dragon_amd import _lib
    rng = np.random.default_rng(3)
    cur, enc, encv, dec = _case(rng, 1, 1, 16, 256, 64)
    w = bd.LowRankWeights.pack(dev(torch, enc[None]), dev(torch, encv[None]), dev(torch, dec))
    c, nxt = dev(torch, cur), torch.empty(1, 16, 64, device="cuda")
    mask = torch.ones(257, device="cuda")
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    plan = _lib.BdhLayerPlan(1, 1, 16, 256, 64)
    announce("layer options refused")
    for th, m in ((float("nan"), None), (0.0, ctypes.c_void_p(mask.data_ptr() + 4))):
        opts = _lib.BdhLayerOptions(th, 0, m)
        st = _lib.load().bdh_lowrank_layer_fwd_ex(ctypes.byref(plan), p(c), p(w.encoder), p(w.encoder_v),
                                                   p(w.decoder), None, None, p(nxt), None,
                                                   ctypes.byref(opts), None)
        assert st == _lib.BDH_EINVAL
    # a wrongly sized mask is refused by the wrapper (the reference's None)
    assert bd.lowrank_layer_forward(c, w, latent_mask=mask) is None
