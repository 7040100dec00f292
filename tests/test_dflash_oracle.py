"""CPU pins of the f64 draft-forward oracle (oracle/dflash_oracle.py).

Each op is checked against what the mathematics fixes -- closed forms, special
cases and invariants -- chosen so that a plausible slip (a missing eps, a wrong
sign or partner index in the rotation, a wrong kv-head mapping, an off-by-one in
the causal bound) fails.  The composite is checked for the structure the block
generalisation promises: causality across tokens, its dependence on every
injected row, and reduction to the reference's one-token sequence."""
import numpy as np
import pytest

import dflash_oracle as dfo
import laguna_hip as lh
import synth


# ---- RMSNorm (kernels/rmsnorm.comp:23-34) ----

def test_rmsnorm_known_answer():
    x = np.array([[3.0, 4.0]])
    y = dfo.rmsnorm(x, np.array([1.0, 2.0]))
    r = 1.0 / np.sqrt(12.5 + 1e-5)
    np.testing.assert_allclose(y, [[3.0 * r, 8.0 * r]], rtol=1e-15)


def test_rmsnorm_eps_matters_for_small_rows():
    x = np.full((1, 16), 1e-3)
    y = dfo.rmsnorm(x, np.ones(16))
    np.testing.assert_allclose(y, 1e-3 / np.sqrt(1e-6 + 1e-5), rtol=1e-14)


def test_rmsnorm_rows_independent():
    x = synth.normal(1, 3 * 64).reshape(3, 64).astype(np.float64)
    w = synth.normal(2, 64).astype(np.float64)
    y = dfo.rmsnorm(x, w)
    x2 = x.copy()
    x2[1] *= 7.0
    y2 = dfo.rmsnorm(x2, w)
    np.testing.assert_array_equal(y[[0, 2]], y2[[0, 2]])


# ---- encoder aux norm (kernels/enc_aux_norm.comp:21-43) ----

def test_enc_aux_norm_per_chunk():
    n_feat, n_aux = 8, 3
    x = np.concatenate([np.full(n_feat, 2.0), np.full(n_feat, -0.5), np.arange(1.0, 9.0)])[None]
    w = np.concatenate([np.full(n_feat, 1.0), np.full(n_feat, 3.0), np.full(n_feat, 0.5)])
    y = dfo.enc_aux_norm(x, w, n_feat, n_aux)
    np.testing.assert_allclose(y[0, :8], 2.0 / np.sqrt(4.0 + 1e-5), rtol=1e-15)
    np.testing.assert_allclose(y[0, 8:16], -1.5 / np.sqrt(0.25 + 1e-5), rtol=1e-15)
    ms = np.mean(np.arange(1.0, 9.0) ** 2)  # 25.5
    np.testing.assert_allclose(y[0, 16:], 0.5 * np.arange(1.0, 9.0) / np.sqrt(ms + 1e-5), rtol=1e-15)


# ---- RoPE table and QK-norm + NeoX rotation (kernels/qk_norm_rope.comp:23-67) ----

def test_rope_freq_table():
    f = dfo.rope_freq(128)
    assert f.dtype == np.float32 and f.shape == (64,)
    assert f[0] == 1.0
    exact = 500000.0 ** (-2.0 * np.arange(64) / 128.0)
    np.testing.assert_allclose(f, exact, rtol=2e-6)
    assert np.all(np.diff(f) < 0)
    np.testing.assert_array_equal(f, lh.rope_freq(128))  # product-side table is the same f32 computation


def _unit_heads(rows, n_heads, hd, seed=3):
    return synth.normal(seed, rows * n_heads * hd).reshape(rows, n_heads * hd).astype(np.float64)


def test_qk_norm_rope_position_zero_is_norm_only():
    x = _unit_heads(2, 3, 16)
    w = synth.normal(4, 16).astype(np.float64)
    y = dfo.qk_norm_rope(x, w, dfo.rope_freq(16), [0, 0], 3, 16, 16)
    xh = x.reshape(2, 3, 16)
    ref = xh * w / np.sqrt(np.mean(xh * xh, axis=-1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(y, ref.reshape(2, -1), rtol=1e-14)


def test_qk_norm_rope_is_complex_rotation():
    # NeoX: (n_d + i n_{d+hd/2}) * e^{i freq[d] pos} for d < rope_dim/2 (rope_dim == head_dim)
    hd, pos = 32, 37
    x = _unit_heads(1, 2, hd)
    w = np.ones(hd)
    freq = dfo.rope_freq(hd)
    y = dfo.qk_norm_rope(x, w, freq, [pos], 2, hd, hd).reshape(2, hd)
    n = dfo.qk_norm_rope(x, w, freq, [0], 2, hd, hd).reshape(2, hd)
    ang = (freq * np.float32(pos)).astype(np.float64)
    z = (n[:, :hd // 2] + 1j * n[:, hd // 2:]) * np.exp(1j * ang)
    np.testing.assert_allclose(y[:, :hd // 2], z.real, atol=1e-13)
    np.testing.assert_allclose(y[:, hd // 2:], z.imag, atol=1e-13)


def test_qk_norm_rope_quarter_turn():
    # freq[0] chosen so position 1 turns the (0, hd/2) pair by pi/2; other pairs angle 0
    hd = 16
    x = _unit_heads(1, 2, hd)
    freq = np.array([np.pi / 2] + [0.0] * 7, np.float32)
    y = dfo.qk_norm_rope(x, np.ones(hd), freq, [1], 2, hd, hd).reshape(2, hd)
    n = dfo.qk_norm_rope(x, np.ones(hd), freq, [0], 2, hd, hd).reshape(2, hd)
    np.testing.assert_allclose(y[:, 0], -n[:, 8], atol=1e-6)   # (n0, n8) -> (-n8, n0)
    np.testing.assert_allclose(y[:, 8], n[:, 0], atol=1e-6)
    keep = [d for d in range(hd) if d not in (0, 8)]
    np.testing.assert_array_equal(y[:, keep], n[:, keep])


def test_qk_norm_rope_zero_rope_dim_is_norm_only():
    x = _unit_heads(1, 2, 16)
    y = dfo.qk_norm_rope(x, np.ones(16), np.zeros(1, np.float32), [9], 2, 16, 0)
    n = dfo.qk_norm_rope(x, np.ones(16), dfo.rope_freq(16), [0], 2, 16, 16)
    np.testing.assert_array_equal(y, n)


def test_qk_norm_rope_preserves_head_norm():
    hd = 128
    x = _unit_heads(3, 4, hd)
    freq = dfo.rope_freq(hd)
    y = dfo.qk_norm_rope(x, np.ones(hd), freq, [5, 900, 2047], 4, hd, hd).reshape(3, 4, hd)
    n = dfo.qk_norm_rope(x, np.ones(hd), freq, [0, 0, 0], 4, hd, hd).reshape(3, 4, hd)
    np.testing.assert_allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(n, axis=-1), rtol=1e-13)


# ---- attention (kernels/mha_attn.comp:28-72) ----

def test_attention_single_key_returns_its_value():
    hd = 8
    q = synth.normal(5, 2 * hd).reshape(1, 2 * hd)
    K = synth.normal(6, hd).reshape(1, hd)
    V = synth.normal(7, hd).reshape(1, hd)
    out = dfo.attention(q, K, V, [0], 2, 1, hd).reshape(2, hd)
    np.testing.assert_allclose(out, np.tile(V.astype(np.float64), (2, 1)), rtol=1e-15)


def test_attention_equal_scores_average_the_allowed_values():
    hd, S = 4, 6
    q = np.zeros((2, hd))
    K = synth.normal(8, S * hd).reshape(S, hd)
    V = synth.normal(9, S * hd).reshape(S, hd).astype(np.float64)
    out = dfo.attention(q, K, V, [2, 5], 1, 1, hd)
    np.testing.assert_allclose(out[0], V[:3].mean(0), rtol=1e-14)  # causal: positions 0..2
    np.testing.assert_allclose(out[1], V.mean(0), rtol=1e-14)
    nc = dfo.attention(q, K, V, [0, 0], 1, 1, hd, causal=False)
    np.testing.assert_allclose(nc[0], V.mean(0), rtol=1e-14)


def test_attention_gqa_head_mapping():
    # 4 query heads over 2 kv heads: heads 0,1 -> kv 0; 2,3 -> kv 1
    hd = 4
    K = np.zeros((1, 2 * hd))
    V = np.concatenate([np.full(hd, 1.0), np.full(hd, 2.0)])[None]
    out = dfo.attention(np.zeros((1, 4 * hd)), K, V, [0], 4, 2, hd).reshape(4, hd)
    np.testing.assert_array_equal(out[:, 0], [1.0, 1.0, 2.0, 2.0])


def test_attention_two_keys_closed_form():
    hd = 4
    q = np.array([[1.0, 0, 0, 0]])
    K = np.array([[2.0, 0, 0, 0], [0.0, 0, 0, 0]])
    V = np.array([[1.0, 0, 0, 0], [0.0, 1, 0, 0]])
    out = dfo.attention(q, K, V, [1], 1, 1, hd)[0]
    a = np.exp(2.0 / 2.0)  # score 2 * (1/sqrt(4))
    np.testing.assert_allclose(out[:2], [a / (a + 1), 1 / (a + 1)], rtol=1e-15)


# ---- gate, activation ----

def test_softplus_gate_threshold():
    g = np.array([0.0, 20.0, 20.5, 21.0, -30.0])
    y = dfo.softplus_gate(g)
    np.testing.assert_allclose(y[0], np.log(2.0), rtol=1e-15)
    np.testing.assert_allclose(y[1], np.log1p(np.exp(20.0)), rtol=1e-15)  # 20 is not above the threshold
    assert y[2] == 20.5 and y[3] == 21.0
    np.testing.assert_allclose(y[4], np.exp(-30.0), rtol=1e-12)


def test_gate_mul_per_head():
    a = np.ones((1, 6))
    out = dfo.gate_mul(a, np.array([[2.0, 3.0]]), 2, 3)
    np.testing.assert_array_equal(out, [[2, 2, 2, 3, 3, 3]])


def test_silu_mul_special_values():
    y = dfo.silu_mul(np.array([0.0, 40.0, -40.0]), np.array([5.0, 2.0, 2.0]))
    assert y[0] == 0.0
    np.testing.assert_allclose(y[1], 80.0, rtol=1e-15)
    assert abs(y[2]) < 1e-15


# ---- composite ----

CFG = lh.DFlashConfig(n_embd=256, n_heads=4, n_kv=2, head_dim=64, rope_dim=64, n_ff=512, n_aux=2, n_layers=2)


@pytest.fixture(scope="module")
def tiny():
    W, layers = synth.dflash_model(0x5EED0100, CFG, 2, norm_sigma=0.1)
    return W, layers


def test_block_forward_is_causal_over_tokens(tiny):
    W, layers = tiny
    M, C = 4, 3
    feat, tok, kc, vc = synth.dflash_inputs(0x5EED0101, CFG, 2, M, C)
    y = dfo.forward_block(feat, tok, W, layers, kc, vc, C, CFG)
    tok2 = tok.copy()
    tok2[2:] += 1.0
    y2 = dfo.forward_block(feat, tok2, W, layers, kc, vc, C, CFG)
    np.testing.assert_array_equal(y[:2], y2[:2])  # tokens 0, 1 do not see tokens 2, 3
    assert np.max(np.abs(y[2:] - y2[2:])) > 1e-3
    feat2 = feat.copy()
    feat2[3] += 1.0  # every token sees every injected row
    y3 = dfo.forward_block(feat2, tok, W, layers, kc, vc, C, CFG)
    assert np.all(np.max(np.abs(y3 - y), axis=1) > 1e-6)


def test_block_forward_one_token_is_the_reference_sequence(tiny):
    # M = 1, C = 0: per layer attention over [injected (pos 0), token (pos 1)] with
    # q_pos 1, written out step by step as src/dflash.rs:877-976 does it
    W, layers = tiny
    feat, tok, _, _ = synth.dflash_inputs(0x5EED0102, CFG, 2, 1, 0)
    y = dfo.forward_block(feat, tok, W, layers, [np.zeros((0, 128))] * 2, [np.zeros((0, 128))] * 2, 0, CFG)
    E, H, KV, HD = CFG.n_embd, CFG.n_heads, CFG.n_kv, CFG.head_dim
    freq = dfo.rope_freq(HD)
    enc = dfo.encode(feat, W, CFG)
    x = tok.astype(np.float64)
    for L in layers:
        en = dfo.rmsnorm(enc, L["attn_norm"])
        k_inj = dfo.qk_norm_rope(dfo.proj(en, L["attn_k"], L["attn_k_dtype"], E, KV * HD), L["attn_k_norm"], freq, [0],
                                 KV, HD, HD)
        v_inj = dfo.proj(en, L["attn_v"], L["attn_v_dtype"], E, KV * HD)
        nx = dfo.rmsnorm(x, L["attn_norm"])
        q = dfo.qk_norm_rope(dfo.proj(nx, L["attn_q"], L["attn_q_dtype"], E, H * HD), L["attn_q_norm"], freq, [1], H,
                             HD, HD)
        k = dfo.qk_norm_rope(dfo.proj(nx, L["attn_k"], L["attn_k_dtype"], E, KV * HD), L["attn_k_norm"], freq, [1], KV,
                             HD, HD)
        v = dfo.proj(nx, L["attn_v"], L["attn_v_dtype"], E, KV * HD)
        a = dfo.attention(q, np.concatenate([k_inj, k]), np.concatenate([v_inj, v]), [1], H, KV, HD)
        a = dfo.gate_mul(a, dfo.softplus_gate(dfo.proj(nx, L["attn_gate"], L["attn_gate_dtype"], E, H)), H, HD)
        x = x + dfo.proj(a, L["attn_output"], L["attn_output_dtype"], H * HD, E)
        h = dfo.rmsnorm(x, L["ffn_norm"])
        f = dfo.silu_mul(dfo.proj(h, L["ffn_gate"], L["ffn_gate_dtype"], E, CFG.n_ff),
                         dfo.proj(h, L["ffn_up"], L["ffn_up_dtype"], E, CFG.n_ff))
        x = x + dfo.proj(f, L["ffn_down"], L["ffn_down_dtype"], CFG.n_ff, E)
    x = dfo.rmsnorm(x, W["output_norm"])
    np.testing.assert_allclose(y, x, rtol=1e-12, atol=1e-12)


def _weights_f64(raw, dtype, k, n):
    # the projection's dequantized weight [n][k], decoded by the C oracle alone
    import oracle as orc
    if dtype == lh.F32:
        return np.asarray(raw, np.float32).reshape(n, k).astype(np.float64)
    return orc.dequant(raw, dtype, k * n).reshape(n, k).astype(np.float64)


def _rms(x, w, eps=1e-5):
    x = np.asarray(x, np.float64)
    return x * np.asarray(w, np.float64) / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


def test_block_forward_zero_branches_is_the_normed_token(tiny):
    # attn_output = 0 and ffn_down = 0: every residual branch adds exactly zero, so the
    # block output is rmsnorm(token) * output_norm whatever the rest of the model does
    W, layers = tiny
    M, C = 3, 5
    feat, tok, kc, vc = synth.dflash_inputs(0x5EED0110, CFG, 2, M, C)
    E, QD = CFG.n_embd, CFG.n_heads * CFG.head_dim
    z = [dict(L, attn_output=np.zeros(QD * E, np.float32), attn_output_dtype=lh.F32,
              ffn_down=np.zeros(CFG.n_ff * E, np.float32), ffn_down_dtype=lh.F32) for L in layers]
    y = dfo.forward_block(feat, tok, W, z, kc, vc, C, CFG)
    np.testing.assert_allclose(y, _rms(tok, W["output_norm"]), rtol=1e-14, atol=0)


def test_block_forward_zero_attn_norm_is_uniform_causal_attention(tiny):
    # attn_norm = 0 zeroes the normed rows, so every query, block key, block value and
    # gate logit is 0: the scores are all equal, the gate is softplus(0) = ln 2, and
    # token t (at position C + M + t) averages the values of the C + M + t + 1
    # positions it may see, of which only the C context values are nonzero:
    #     a_t[h] = ln 2 * sum_{p < C} v_ctx[p][kv(h)] / (C + M + t + 1),
    #     kv(h) = h * n_kv / n_q.
    # With ffn_down = 0 the layer adds only W_o a_t.  One layer, written out directly.
    W, layers = tiny
    M, C = 4, 6
    E, H, KV, HD = CFG.n_embd, CFG.n_heads, CFG.n_kv, CFG.head_dim
    feat, tok, kc, vc = synth.dflash_inputs(0x5EED0111, CFG, 1, M, C)
    L = dict(layers[0], attn_norm=np.zeros(E, np.float32), ffn_down=np.zeros(CFG.n_ff * E, np.float32),
             ffn_down_dtype=lh.F32)
    y = dfo.forward_block(feat, tok, W, [L], kc, vc, C, CFG)
    Wo = _weights_f64(L["attn_output"], L["attn_output_dtype"], H * HD, E)
    vsum = np.asarray(vc[0], np.float64).reshape(C, KV, HD).sum(axis=0)
    want = []
    for t in range(M):
        a = np.concatenate([vsum[h * KV // H] for h in range(H)]) * np.log(2.0) / (C + M + t + 1)
        want.append(_rms(tok[t].astype(np.float64) + Wo @ a, W["output_norm"]))
    np.testing.assert_allclose(y, np.array(want), rtol=1e-12, atol=1e-12 * np.max(np.abs(want)))


def test_block_forward_constant_context_value(tiny):
    # the same closed form with every context value row equal to c: the average over
    # the visible positions is c * C / (C + M + t + 1), a check of the position count
    # that does not depend on which context rows a query sees
    W, layers = tiny
    M, C = 2, 3
    E, H, KV, HD = CFG.n_embd, CFG.n_heads, CFG.n_kv, CFG.head_dim
    feat, tok, kc, _ = synth.dflash_inputs(0x5EED0112, CFG, 1, M, C)
    c = synth.normal(0x5EED0113, KV * HD)
    vc = [np.tile(c, (C, 1))]
    L = dict(layers[0], attn_norm=np.zeros(E, np.float32), ffn_down=np.zeros(CFG.n_ff * E, np.float32),
             ffn_down_dtype=lh.F32)
    y = dfo.forward_block(feat, tok, W, [L], kc, vc, C, CFG)
    Wo = _weights_f64(L["attn_output"], L["attn_output_dtype"], H * HD, E)
    cr = np.asarray(c, np.float64).reshape(KV, HD)
    for t in range(M):
        a = np.concatenate([cr[h * KV // H] for h in range(H)]) * np.log(2.0) * C / (C + M + t + 1)
        np.testing.assert_allclose(y[t], _rms(tok[t].astype(np.float64) + Wo @ a, W["output_norm"]), rtol=1e-12,
                                   atol=1e-12)
