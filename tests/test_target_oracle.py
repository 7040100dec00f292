"""CPU pins of the f64 dense-target oracle (oracle/target_oracle.py).

The composite is checked against what the mathematics fixes, each check chosen so
that a plausible slip fails it: zero residual branches reduce the forward to the
LM head of the normed input (a wrong norm, eps or residual breaks it), attention
over one position returns V (a wrong kv-head mapping or a query leaking in breaks
it), the first cached token equals the uncached forward (a wrong position or cache
append breaks it), RoPE is the identity at position 0 (so the sliding-window table
matters only later), and the capture order follows the reference's rule
(src/target.rs:391-395, 558-560)."""
import numpy as np
import pytest

import dflash_oracle as dfo
import laguna_hip as lh
import oracle as orc
import synth
import target_oracle as tgo

E, H, KV, HD, FF, NL, V = 512, 4, 2, 128, 512, 4, 300


def hparams(**kw):
    return tgo.Hparams(n_embd=E, n_heads=H, n_kv=KV, head_dim=HD, n_ff=FF, n_layers=NL, n_vocab=V, rope_dim=HD,
                       **kw)


@pytest.fixture(scope="module")
def model():
    hp = hparams()
    layers, ex = synth.target_model(0x7A11, hp, gate_layers=[0, 2])
    x = synth.normal(0x7A12, E)
    return hp, layers, ex, x


def run(hp, layers, ex, x, **kw):
    return tgo.forward_token(x, layers, hp, ex["output_norm"], ex["output"], ex["output_dtype"], **kw)


def test_capture_order_follows_the_reference_rule():
    assert tgo.capture_order(4, None) == [0, 1, 2, 3]
    assert tgo.capture_order(4, [3, 1, 3]) == [1, 3]  # ascending, duplicates once
    assert tgo.capture_order(4, [4, 0]) == [0, 4]     # n_layers: the final state, last
    assert tgo.capture_order(4, [7]) == []            # beyond the model: nothing
    assert tgo.capture_order(4, []) == []


def test_captured_states_are_layer_inputs(model):
    hp, layers, ex, x = model
    _, cap_all = run(hp, layers, ex, x)
    assert len(cap_all) == NL
    np.testing.assert_array_equal(cap_all[0], x.astype(np.float64))  # layer 0's input is the token
    _, cap = run(hp, layers, ex, x, layer_indices=[2, 4])
    np.testing.assert_array_equal(cap[0], cap_all[2])
    # the final state (before output_norm) is what one more layer would receive: with
    # one layer removed, the state entering layer 3 is the final state
    hp3 = hparams()
    hp3.n_layers = 3
    _, cap3 = run(hp3, layers[:3], ex, x, layer_indices=[3])
    np.testing.assert_array_equal(cap3[0], cap_all[3])


def test_zero_residual_branches_give_the_lm_head_of_the_normed_input(model):
    # attn_output = 0 and ffn_down = 0: x passes every layer unchanged, so
    # logits = W_out (x * output_norm / sqrt(mean(x^2) + 1e-5))
    hp, layers, ex, x = model
    z = []
    for L in layers:
        L = dict(L)
        L["attn_output"], L["attn_output_dtype"] = np.zeros(L["n_q_heads"] * HD * E, np.float32), lh.F32
        L["ffn_down"], L["ffn_down_dtype"] = np.zeros(FF * E, np.float32), lh.F32
        z.append(L)
    logits, cap = run(hp, z, ex, x, layer_indices=[0, 1, 2, 3, 4])
    x64 = x.astype(np.float64)
    for c in cap:
        np.testing.assert_array_equal(c, x64)
    h = x64 * ex["output_norm"].astype(np.float64) / np.sqrt(np.mean(x64 * x64) + 1e-5)
    W = orc.dequant(ex["output"], ex["output_dtype"], E * V).reshape(V, E).astype(np.float64)
    np.testing.assert_allclose(logits, W @ h, rtol=1e-12, atol=1e-12 * np.abs(W @ h).max())


def test_one_position_attention_ignores_the_queries(model):
    # uncached, each head attends to the token's own key only: softmax over one score
    # is 1 and the head returns its kv head's V, whatever the queries are
    hp, layers, ex, x = model
    base, _ = run(hp, layers, ex, x)
    other = [dict(L, attn_q=synth.q4k_weight(0x7A20 + i, E, L["n_q_heads"] * HD)) for i, L in enumerate(layers)]
    logits, _ = run(hp, other, ex, x)
    np.testing.assert_allclose(logits, base, rtol=1e-12, atol=1e-12 * np.abs(base).max())


def test_attention_of_one_position_is_v_per_group():
    q = synth.normal(1, H * HD).astype(np.float64)
    v = synth.normal(2, KV * HD).astype(np.float64).reshape(1, -1)
    k = synth.normal(3, KV * HD).astype(np.float64).reshape(1, -1)
    a = dfo.attention(q, k, v, [0], H, KV, HD)[0].reshape(H, HD)
    for h in range(H):  # kv head h * KV / H
        np.testing.assert_allclose(a[h], v.reshape(KV, HD)[h * KV // H], rtol=1e-15)


def test_first_cached_token_equals_the_uncached_forward(model):
    hp, layers, ex, x = model
    base, cap0 = run(hp, layers, ex, x, layer_indices=[1, 3])
    cache = tgo.KvCache(NL)
    logits, cap = run(hp, layers, ex, x, layer_indices=[1, 3], cache=cache)
    np.testing.assert_array_equal(logits, base)
    for a, b in zip(cap, cap0):
        np.testing.assert_array_equal(a, b)
    assert cache.len == 1 and all(len(c) == 1 for c in cache.k)


def test_second_cached_token_attends_to_both_positions(model):
    # a two-position cache whose two values are equal returns that value whatever
    # the scores: check by hand against the cache the oracle built
    hp, layers, ex, x = model
    cache = tgo.KvCache(NL)
    run(hp, layers, ex, x, cache=cache)
    run(hp, layers, ex, synth.normal(0x7A30, E), cache=cache)
    assert cache.len == 2
    K = np.stack(cache.k[0])
    vv = np.stack([cache.v[0][0], cache.v[0][0]])
    q = synth.normal(0x7A31, H * HD).astype(np.float64)
    a = dfo.attention(q, K, vv, [1], H, KV, HD)[0].reshape(H, HD)
    for h in range(H):
        np.testing.assert_allclose(a[h], vv[0].reshape(KV, HD)[h * KV // H], rtol=1e-13)


def test_swa_table_is_irrelevant_at_position_0_and_used_after(model):
    hp, layers, ex, x = model
    hs = hparams(swa=True, rope_dim_swa=HD, rope_base_swa=10000.0)
    a, _ = run(hp, layers, ex, x)
    b, _ = run(hs, layers, ex, x)
    np.testing.assert_array_equal(a, b)  # RoPE at position 0 is the identity
    c1, c2 = tgo.KvCache(NL), tgo.KvCache(NL)
    x2 = synth.normal(0x7A40, E)
    for c, h in ((c1, hp), (c2, hs)):
        run(h, layers, ex, x, cache=c)
    la, _ = run(hp, layers, ex, x2, cache=c1)
    lb, _ = run(hs, layers, ex, x2, cache=c2)
    assert np.max(np.abs(la - lb)) > 1e-6 * np.max(np.abs(la))
    # layer 0 is never a sliding-window layer: its cached keys agree
    np.testing.assert_array_equal(c1.k[0][1], c2.k[0][1])
    assert np.max(np.abs(c1.k[1][1] - c2.k[1][1])) > 0


def test_gate_attn_special_values():
    a = np.ones(2 * 4)
    g = np.array([0.0, -50.0])
    y = tgo.gate_attn(a, g, 2, 4).reshape(2, 4)
    np.testing.assert_allclose(y[0], np.log(2.0), rtol=1e-15)
    np.testing.assert_allclose(y[1], np.exp(-50.0), rtol=1e-12)  # log(1 + e^g) ~ e^g for g << 0
    # no threshold: unlike the draft's host softplus (g > 20 ? g : ...), 30 gives log(1 + e^30)
    np.testing.assert_allclose(tgo.gate_attn(np.ones(1), np.array([30.0]), 1, 1), np.log1p(np.exp(30.0)))


def test_no_output_weight_returns_the_normed_final_state(model):
    hp, layers, ex, x = model
    y, cap = tgo.forward_token(x, layers, hp, ex["output_norm"], None, None, layer_indices=[NL])
    np.testing.assert_allclose(y, dfo.rmsnorm(cap[0], ex["output_norm"], 1e-5), rtol=1e-15)


def test_token_embedding_row():
    raw = synth.q8_0_weight(5, E, 10)
    full = orc.dequant(raw, orc.Q8_0, E * 10).reshape(10, E)
    np.testing.assert_array_equal(tgo.token_embedding(raw, orc.Q8_0, E, 7), full[7])
