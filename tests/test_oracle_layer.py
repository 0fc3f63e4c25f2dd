"""Pins the layer-body oracle (oracle.lowrank_layer_f64) before the GPU layer
is checked against it: a LayerNorm known answer (biased variance, eps under
the root), the decoder tail against the headwise sum it replaces, and a
pure-Python scalar loop over a tiny layer (RoPE, read-before-update
recurrence, the order of ReLU, LayerNorm, gate and residual).  Plausible
mistakes planted in a copy of the composition must fail these checks."""
import math

import numpy as np


def _ln_list(vals, eps=1e-5):
    m = sum(vals) / len(vals)
    var = sum((u - m) ** 2 for u in vals) / len(vals)
    return [(u - m) / math.sqrt(var + eps) for u in vals]


def test_layer_norm_known_answer(oracle):
    # x = (1, 2, 3, 4): mean 2.5, biased var 1.25 (unbiased would be 5/3).
    out = oracle.layer_norm_f64(np.array([[1.0, 2.0, 3.0, 4.0]]))
    den = math.sqrt(1.25 + 1e-5)
    expect = [-1.5 / den, -0.5 / den, 0.5 / den, 1.5 / den]
    assert np.max(np.abs(out[0] - expect)) < 1e-15
    # invariants on random rows: zero mean, variance var / (var + eps)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 64)) * 3 + 1
    y = oracle.layer_norm_f64(x)
    var = x.var(axis=-1)
    assert np.max(np.abs(y.mean(axis=-1))) < 1e-12
    assert np.max(np.abs(y.var(axis=-1) - var / (var + 1e-5))) < 1e-12


def test_decode_tail_equals_headwise_sum(oracle):
    # residual_stream.rs:317 "one GEMM is the exact headwise sum".
    rng = np.random.default_rng(4)
    B, H, T, N, D = 2, 3, 5, 4, 6
    y = rng.standard_normal((B, H, T, N))
    dec = rng.standard_normal((H * N, D))
    got = oracle.decode_y_neuron_tail_f64(y, dec)
    ref = sum(np.einsum("btn,nd->btd", y[:, h], dec[h * N:(h + 1) * N]) for h in range(H))
    assert np.max(np.abs(got - ref)) < 1e-12


def _rope_list(xs, pos, theta=65536.0):
    # attention.rs:488-576 restated on Python scalars (f32 phase op order).
    N = len(xs)
    out = []
    for i in range(N):
        k = (i // 2) * 2
        f = np.float32(1.0) / np.float32(np.float32(theta) ** np.float32(np.float32(k) / np.float32(N)))
        f = np.float32(f / np.float32(2 * np.float32(math.pi)))
        raw = np.float32(np.float32(pos) * f)
        phi = float(np.float32(np.float32(raw - np.floor(raw)) * np.float32(2 * np.float32(math.pi))))
        c, s = math.cos(phi), math.sin(phi)
        other = -xs[i + 1] if i % 2 == 0 else xs[i - 1]
        out.append(xs[i] * c + other * s)
    return out


def _act(v, th, m, bad, where):
    # relu_lowrank reference_forward on one scalar: (v - th), ReLU, times m
    if bad == "threshold_after_relu":
        return (max(0.0, v) - th) * m
    if bad == "mask_before_relu":
        return max(0.0, v * m - th)
    if bad == "mask_only_x" and where == "y":
        return max(0.0, v - th)
    return max(0.0, v - th) * m


def _layer_loops(cur, enc, encv, dec, pos0, bad=None, th=0.0, mask=None):
    B, T, D = cur.shape
    H, _, N = enc.shape
    mk = [1.0] * N if mask is None else [float(v) for v in mask]
    nxt = np.zeros((B, T, D))
    for b in range(B):
        x = [[[_act(sum(cur[b, t, d] * enc[h, d, n] for d in range(D)), th, mk[n], bad, "x")
               for n in range(N)] for t in range(T)] for h in range(H)]
        attn = [[None] * T for _ in range(H)]
        for h in range(H):
            rho = [[0.0] * D for _ in range(N)]
            for t in range(T):
                q = _rope_list(x[h][t], pos0 + t)
                if bad == "update_before_read":
                    for n in range(N):
                        for d in range(D):
                            rho[n][d] += q[n] * cur[b, t, d]
                attn[h][t] = [sum(q[n] * rho[n][d] for n in range(N)) for d in range(D)]
                if bad != "update_before_read":
                    for n in range(N):
                        for d in range(D):
                            rho[n][d] += q[n] * cur[b, t, d]
        for t in range(T):
            z = [0.0] * D
            for h in range(H):
                a = attn[h][t] if bad == "no_attn_norm" else _ln_list(attn[h][t])
                for n in range(N):
                    g = sum(a[d] * encv[h, d, n] for d in range(D))
                    yv = x[h][t][n] * (g if bad == "gate_without_relu" else _act(g, th, mk[n], bad, "y"))
                    for d in range(D):
                        z[d] += yv * dec[h * N + n, d]
            mlp = z if bad == "no_mlp_norm" else _ln_list(z)
            nxt[b, t] = _ln_list([cur[b, t, d] + mlp[d] for d in range(D)])
    return nxt


def test_layer_matches_scalar_loops_and_catches_planted_mistakes(oracle):
    rng = np.random.default_rng(9)
    B, T, D, H, N = 1, 4, 4, 2, 4
    cur = rng.standard_normal((B, T, D))
    enc = rng.standard_normal((H, D, N)) * 0.7
    encv = rng.standard_normal((H, D, N)) * 0.7
    dec = rng.standard_normal((H * N, D)) * 0.5
    got, _ = oracle.lowrank_layer_f64(cur, enc, encv, dec, pos0=3)
    ref = _layer_loops(cur, enc, encv, dec, 3)
    assert np.max(np.abs(got - ref)) < 1e-5  # RoPE runs in f32 in the oracle
    for bad in ("update_before_read", "no_attn_norm", "gate_without_relu", "no_mlp_norm"):
        wrong = _layer_loops(cur, enc, encv, dec, 3, bad=bad)
        assert np.max(np.abs(got - wrong)) > 1e-3, bad


def test_layer_threshold_and_mask_match_scalar_loops(oracle):
    # The ReLU threshold and the latent mask (relu_lowrank.rs reference_forward:
    # subtract, ReLU, times the mask, in both projections): a threshold inside
    # the projections' range and a mask with values other than 0 and 1, so
    # that each plausible misplacement changes the output.
    rng = np.random.default_rng(21)
    B, T, D, H, N = 1, 4, 4, 2, 4
    cur = rng.standard_normal((B, T, D))
    enc = rng.standard_normal((H, D, N)) * 0.7
    encv = rng.standard_normal((H, D, N)) * 0.7
    dec = rng.standard_normal((H * N, D)) * 0.5
    th, mask = 0.3, np.array([1.0, 0.5, 0.0, 2.0])
    got, _ = oracle.lowrank_layer_f64(cur, enc, encv, dec, pos0=3, relu_threshold=th, latent_mask=mask)
    ref = _layer_loops(cur, enc, encv, dec, 3, th=th, mask=mask)
    assert np.max(np.abs(got - ref)) < 1e-5
    plain, _ = oracle.lowrank_layer_f64(cur, enc, encv, dec, pos0=3)
    assert np.max(np.abs(got - plain)) > 1e-3
    for bad in ("threshold_after_relu", "mask_before_relu", "mask_only_x"):
        wrong = _layer_loops(cur, enc, encv, dec, 3, bad=bad, th=th, mask=mask)
        assert np.max(np.abs(got - wrong)) > 1e-3, bad


def test_block_pattern_mask(oracle):
    # BlockPattern1d::mask (block_sparse.rs:49-64): whole blocks, the last one
    # ragged; dense when no blocks are listed.
    m = oracle.block_pattern_mask(10, 4, {0, 2})
    assert m.tolist() == [1, 1, 1, 1, 0, 0, 0, 0, 1, 1]
    assert oracle.block_pattern_mask(5, 2).tolist() == [1] * 5


def test_model_oracle_composition(oracle):
    # LN(embed[tok]) -> layer -> @ lm_head, restated with the scalar loops above.
    rng = np.random.default_rng(12)
    V, D, H, N, T = 6, 4, 2, 4, 3
    embed = rng.standard_normal((V, D))
    enc = rng.standard_normal((H, D, N)) * 0.7
    encv = rng.standard_normal((H, D, N)) * 0.7
    dec = rng.standard_normal((H * N, D)) * 0.5
    head = rng.standard_normal((D, V))
    tokens = np.array([[5, 0, 3]])
    got = oracle.model_forward_f64(tokens, embed, enc, encv, dec, head, 1, pos0=2)
    cur = np.array([[_ln_list(list(embed[t])) for t in tokens[0]]])
    hid = _layer_loops(cur, enc, encv, dec, 2)
    ref = [[sum(hid[0, t, d] * head[d, v] for d in range(D)) for v in range(V)] for t in range(T)]
    assert np.max(np.abs(got[0] - np.array(ref))) < 1e-5
    # zero layers: logits of the normalised embeddings only
    got0 = oracle.model_forward_f64(tokens, embed, enc, encv, dec, head, 0)
    assert np.max(np.abs(got0[0] - cur[0] @ head)) < 1e-12


def test_model_state_carry_splits_a_sequence(oracle):
    # forward_with_state over a prompt, then one token at a time carrying each
    # layer's rho and the position (dragon.rs:3334, :3437-3446), equals one
    # forward over the whole sequence: the invariant of the reference's
    # linear_attention_incremental_forward_matches_full_sequence
    # (dragon.rs:5028-5057).  Dropping the carried state or not
    # advancing the position must break it.
    rng = np.random.default_rng(13)
    V, D, H, N, T, L = 7, 8, 2, 8, 5, 2
    embed = rng.standard_normal((V, D))
    enc = rng.standard_normal((H, D, N)) * 0.5
    encv = rng.standard_normal((H, D, N)) * 0.5
    dec = rng.standard_normal((H * N, D)) * 0.5
    head = rng.standard_normal((D, V))
    tokens = rng.integers(0, V, (2, T))
    whole = oracle.model_forward_f64(tokens, embed, enc, encv, dec, head, L, pos0=0)

    def split(carry=True, advance=True):
        out, rhos = oracle.model_forward_f64(tokens[:, :3], embed, enc, encv, dec, head, L,
                                             pos0=0, return_state=True)
        steps = [out]
        for t in range(3, T):
            lg, new = oracle.model_forward_f64(tokens[:, t:t + 1], embed, enc, encv, dec, head, L,
                                               pos0=t if advance else 0,
                                               rho0s=rhos if carry else None, return_state=True)
            steps.append(lg)
            rhos = new
        return np.concatenate(steps, axis=1)

    scale = np.max(np.abs(whole))
    assert np.max(np.abs(split() - whole)) < 1e-5 * scale
    assert np.max(np.abs(split(carry=False) - whole)) > 1e-2 * scale
    assert np.max(np.abs(split(advance=False) - whole)) > 1e-2 * scale
