"""BASELINE config 5 at its full shape: the 6-layer BDH forward over a byte
vocabulary, B 16, T 1024, D 256, nh 4, N 8192, weights shared across layers
(std 0.02 Gaussians), random tokens (residual_stream.rs:323-572,
dragon.rs:3340-3420).

Batch rows are independent and the forward is causal (logits at t depend
on tokens <= t only), so the full-shape GPU forward is checked on a token
prefix of two batch rows against one oracle forward of that prefix alone.
The decode check runs a prompt and three one-token steps at B 16 (the
decode step then splits each stream into the row ranges of the C5 decode)
against one oracle forward over the same tokens of two rows (the
incremental == full invariant, dragon.rs:5028-5057)."""
import numpy as np
import pytest

from tests.gpu_util import TOL_BF16, announce, dev, host, need_gpu, rel_l2

pytestmark = pytest.mark.gpu

B, T, D, H, N, V, L = 16, 1024, 256, 4, 8192, 256, 6
ROWS = [0, 15]      # batch rows checked against the oracle
PREFIX = 128        # tokens of each checked row


def _weights(seed):
    rng = np.random.default_rng(seed)
    enc = (rng.standard_normal((H, D, N)) * 0.02).astype(np.float32)
    encv = (rng.standard_normal((H, D, N)) * 0.02).astype(np.float32)
    dec = (rng.standard_normal((H * N, D)) * 0.02).astype(np.float32)
    embed = (rng.standard_normal((V, D)) * 0.02).astype(np.float32)
    head = (rng.standard_normal((D, V)) * 0.02).astype(np.float32)
    return rng, enc, encv, dec, embed, head


def _pack(torch, bd, enc, encv, dec, embed, head):
    return bd.pack_model(dev(torch, embed), dev(torch, enc[None]), dev(torch, encv[None]),
                         dev(torch, dec), dev(torch, head), L)


def _oracle_logits(oracle, tokens, enc, encv, dec, embed, head):
    return oracle.model_forward_f64(tokens, embed, oracle.round_bf16(enc), oracle.round_bf16(encv),
                                    oracle.round_bf16(dec), oracle.round_bf16(head), L)


def test_c5_full_forward_prefix_matches_oracle(oracle):
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng, enc, encv, dec, embed, head = _weights(20260734)
    tokens = rng.integers(0, V, (B, T)).astype(np.int32)
    w = _pack(torch, bd, enc, encv, dec, embed, head)
    announce("C5 forward", B, T, D, H, N, L)
    logits = bd.model_forward_logits(dev(torch, tokens), w, position=0)
    torch.cuda.synchronize()
    assert logits is not None and tuple(logits.shape) == (B, T, V)
    assert bool(torch.isfinite(logits).all())
    got = host(logits[ROWS, :PREFIX])
    ref = _oracle_logits(oracle, tokens[ROWS, :PREFIX], enc, encv, dec, embed, head)
    err = rel_l2(got, ref)
    print(f"C5 forward rows {ROWS} tokens 0..{PREFIX - 1}: rel-L2 {err:.2e}")
    assert err <= TOL_BF16


def test_c5_prompt_then_decode_matches_oracle(oracle):
    torch = need_gpu()
    import burn_dragon_amd as bd
    rng, enc, encv, dec, embed, head = _weights(20260735)
    T0, steps = 48, 3
    tokens = rng.integers(0, V, (B, T0 + steps)).astype(np.int32)
    w = _pack(torch, bd, enc, encv, dec, embed, head)
    tok = dev(torch, tokens)
    state = bd.new_model_state(w, B, tok.device)
    announce("C5 prompt + decode", B, T0, steps)
    parts = [bd.model_forward_logits(tok[:, :T0], w, state=state)]
    for t in range(T0, T0 + steps):
        parts.append(bd.model_forward_logits(tok[:, t:t + 1].contiguous(), w, state=state))
    torch.cuda.synchronize()
    assert all(p is not None for p in parts) and state.position == T0 + steps
    got = np.concatenate([host(p[ROWS]) for p in parts], axis=1)
    assert np.isfinite(got).all()
    ref = _oracle_logits(oracle, tokens[ROWS], enc, encv, dec, embed, head)
    e_all, e_steps = rel_l2(got, ref), rel_l2(got[:, T0:], ref[:, T0:])
    print(f"C5 prompt + decode rows {ROWS}: rel-L2 all {e_all:.2e}, decoded tokens {e_steps:.2e}")
    assert e_all <= TOL_BF16 and e_steps <= TOL_BF16
