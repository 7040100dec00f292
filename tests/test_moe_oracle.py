"""CPU pins of the f64 MoE FFN oracle (target_oracle.moe_ffn, following
TargetModel::dispatch_moe_ffn, src/target.rs:607-748).

Each check reduces the composite to something the mathematics fixes, chosen so that
a plausible slip fails it: with one expert selected and its score normalised to 1,
the 32768 / ||h|| rescaling cancels and the layer is that expert's FFN plus the shared
one (a wrong offset, activation or leftover scale breaks it); selection follows
probability + bias in a stable descending order (a reversed sort or a bias left out
breaks it); a non-positive score leaves the rescaled output unscaled, as the
reference does (src/target.rs:710-715); Q4_K experts move with the element offset and
Q8_0 experts do not (src/target.rs:1115-1138).  No reference test or fixture covers
the MoE FFN: beyond these checks its parity is unpinned."""
import numpy as np
import pytest

import oracle as orc
import synth
import target_oracle as tgo

E, FFE, NX, SH = 256, 512, 6, 256  # n_embd, n_ff_exp, n_expert, n_shexp


def weights(seed, expert_dtype=orc.Q4_K):
    def q(dt, s, k, n):
        return (synth.q4k_weight(s, k, n) if dt == orc.Q4_K else synth.q8_0_weight(s, k, n), dt)

    return {
        "ffn_gate_inp": q(orc.Q8_0, seed, E, NX),
        "ffn_gate_exps": q(expert_dtype, seed + 1, E, NX * FFE),
        "ffn_up_exps": q(expert_dtype, seed + 2, E, NX * FFE),
        "ffn_down_exps": q(expert_dtype, seed + 3, FFE, NX * E),
        "ffn_gate_shexp": q(orc.Q4_K, seed + 4, E, SH),
        "ffn_up_shexp": q(orc.Q4_K, seed + 5, E, SH),
        "ffn_down_shexp": q(orc.Q4_K, seed + 6, SH, E),
    }


def expert_ffn(x, w, e):
    x64 = np.asarray(x, np.float32).astype(np.float64)
    off = tgo.expert_offset(e, E, FFE)
    g, _ = tgo.proj_expert(x64, *w["ffn_gate_exps"], E, FFE, off)
    u, _ = tgo.proj_expert(x64, *w["ffn_up_exps"], E, FFE, off)
    d, _ = tgo.proj_expert(g / (1.0 + np.exp(-g)) * u, *w["ffn_down_exps"], FFE, E, off)
    return d


def shared_ffn(x, w):
    x64 = np.asarray(x, np.float32).astype(np.float64)
    g, _ = tgo.proj_expert(x64, *w["ffn_gate_shexp"], E, SH)
    u, _ = tgo.proj_expert(x64, *w["ffn_up_shexp"], E, SH)
    d, _ = tgo.proj_expert(g / (1.0 + np.exp(-g)) * u, *w["ffn_down_shexp"], SH, E)
    return d


def close(a, b):
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-12 * float(np.max(np.abs(b))))


def test_one_normalised_expert_is_its_ffn_plus_the_shared_one():
    w = weights(0x3E00)
    x = synth.normal(0x3E01, E)
    bias = np.zeros(NX, np.float32)
    bias[4] = 5.0  # expert 4 wins whatever the router says
    out, _, chosen, scores = tgo.moe_ffn(x, w, bias, E, NX, 1, FFE, SH, expert_weights_norm=True)
    assert chosen == [4] and scores[0] == pytest.approx(1.0)
    close(out, expert_ffn(x, w, 4) + shared_ffn(x, w))


def test_selection_is_probability_plus_bias_descending_and_stable():
    w = weights(0x3E10)
    x = synth.normal(0x3E11, E)
    bias = np.array([0.0, 3.0, 1.0, 3.0, 2.0, 0.0], np.float32)  # ties 1/3 and 0/5 kept in index order
    logits, _ = tgo.proj_expert(np.asarray(x, np.float64), *w["ffn_gate_inp"], E, NX)
    probs = 1.0 / (1.0 + np.exp(-logits))
    expect = sorted(range(NX), key=lambda i: -(probs[i] + bias[i]))[:3]
    out, _, chosen, scores = tgo.moe_ffn(x, w, bias, E, NX, 3, FFE, SH, expert_weights_scale=2.5)
    assert chosen == expect and set(chosen) <= {1, 2, 3, 4}
    np.testing.assert_allclose(scores, 2.5 * probs[chosen], rtol=1e-15)
    close(out, sum(s * expert_ffn(x, w, e) for e, s in zip(chosen, scores)) + shared_ffn(x, w))


def test_non_positive_score_leaves_the_rescaled_output():
    w = weights(0x3E20)
    x = synth.normal(0x3E21, E)
    bias = np.array([0.0, 0.0, 4.0, 0.0, 0.0, 4.5], np.float32)
    out, _, chosen, scores = tgo.moe_ffn(x, w, bias, E, NX, 2, FFE, SH, expert_weights_scale=-1.0)
    assert chosen == [5, 2] and np.all(scores < 0)
    x64 = np.asarray(x, np.float64)
    ref = shared_ffn(x, w)
    for e in chosen:
        off = tgo.expert_offset(e, E, FFE)
        g, _ = tgo.proj_expert(x64, *w["ffn_gate_exps"], E, FFE, off)
        u, _ = tgo.proj_expert(x64, *w["ffn_up_exps"], E, FFE, off)
        h = g / (1.0 + np.exp(-g)) * u
        ref = ref + tgo.F16_SAFE / np.linalg.norm(h) * expert_ffn(x, w, e)  # linear in h
    close(out, ref)


def test_q4k_experts_move_with_the_offset_and_q8_0_experts_do_not():
    x = synth.normal(0x3E31, E)
    wq = weights(0x3E30)
    a, b = expert_ffn(x, wq, 1), expert_ffn(x, wq, 3)
    assert np.max(np.abs(a - b)) > 1e-3 * np.max(np.abs(a))
    # expert 3 of the stack is the same FFN as a stack holding only expert 3's rows
    one = dict(wq)
    for t, rows in (("ffn_gate_exps", FFE), ("ffn_up_exps", FFE), ("ffn_down_exps", E)):
        raw, dt = wq[t]
        k = E if t != "ffn_down_exps" else FFE
        start = 3 * rows * k // 256 * 144
        one[t] = (np.frombuffer(raw, np.uint8)[start:start + rows * k // 256 * 144], dt)
    close(b, expert_ffn(x, one, 0))
    w8 = weights(0x3E30, orc.Q8_0)
    close(expert_ffn(x, w8, 3), expert_ffn(x, w8, 0))
