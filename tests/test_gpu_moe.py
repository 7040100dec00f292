"""The MoE FFN (lh.dispatch_moe_ffn, mirroring TargetModel::dispatch_moe_ffn,
src/target.rs:607-748) on the GPU against the f64 oracle (target_oracle.moe_ffn).

The experts are picked by bias values two units apart, so the f32 and f64 router
logits cannot order them differently; the tolerance is the products' 1e-4 of the sum
of |terms| reaching each output (the oracle's absdot), the scores within 1e-6."""
import numpy as np
import pytest

import laguna_hip as lh
import oracle as orc
import synth
import target_oracle as tgo
from conftest import parity

pytestmark = pytest.mark.gpu

E, FFE, NX, SH = 512, 768, 8, 512


def weights(seed, expert_dtype, router_dtype=orc.Q8_0):
    def q(dt, s, k, n):
        if dt == orc.F32:
            return (synth.normal(s, k * n, 0.05).astype(np.float32), dt)
        return (synth.q4k_weight(s, k, n) if dt == orc.Q4_K else synth.q8_0_weight(s, k, n), dt)

    return {
        "ffn_gate_inp": q(router_dtype, seed, E, NX),
        "ffn_gate_exps": q(expert_dtype, seed + 1, E, NX * FFE),
        "ffn_up_exps": q(expert_dtype, seed + 2, E, NX * FFE),
        "ffn_down_exps": q(expert_dtype, seed + 3, FFE, NX * E),
        "ffn_gate_shexp": q(orc.Q4_K, seed + 4, E, SH),
        "ffn_up_shexp": q(orc.Q4_K, seed + 5, E, SH),
        "ffn_down_shexp": q(orc.Q4_K, seed + 6, SH, E),
    }


@pytest.mark.parametrize("dtype,used,norm,scale,router", [(orc.Q4_K, 2, True, 1.0, orc.Q8_0),
                                                           (orc.Q4_K, 3, False, 2.5, orc.Q8_0),
                                                           (orc.Q4_K, 2, False, -1.0, orc.Q8_0),
                                                           (orc.Q8_0, 2, True, 1.0, orc.Q8_0),
                                                           (orc.Q4_K, 4, True, 1.0, orc.F32)])
def test_moe_ffn_against_the_oracle(ctx, dtype, used, norm, scale, router):
    # an F32 router (ffn_gate_inp is often stored unquantized) takes the f32 matvec
    seed = 0x3F00 + 16 * used + (dtype == orc.Q8_0)
    print(f"moe ffn dtype={dtype} used={used} norm={norm} scale={scale} router={router}", flush=True)
    w = weights(seed, dtype, router)
    x = synth.normal(seed + 9, E)
    # bias 2 apart (probabilities add less than 1): the order is the bias order
    bias = (synth.uniform(seed + 10, NX) * 0.25 + 2.0 * np.random.default_rng(seed).permutation(NX)).astype(np.float32)
    bufs = {t: (lh.upload_f32(ctx, raw) if dt == orc.F32 else lh.upload_bytes(ctx, raw), dt)
            for t, (raw, dt) in w.items()}
    moe = lh.MoeFfnWeights(lh.upload_f32(ctx, bias), **bufs)
    xb, out = lh.upload_f32(ctx, x), lh.GpuBuffer(ctx, 4 * E)
    chosen, scores = lh.dispatch_moe_ffn(ctx, xb, moe, out, E, NX, used, FFE, SH, expert_weights_norm=norm,
                                         expert_weights_scale=scale)
    y64, a, chosen64, scores64 = tgo.moe_ffn(x, w, bias, E, NX, used, FFE, SH, expert_weights_norm=norm,
                                             expert_weights_scale=scale)
    assert chosen == chosen64
    np.testing.assert_allclose(scores, scores64, rtol=1e-6)
    parity(out.read_f32(E), y64, a, 1e-4)


def test_moe_ffn_rejects_more_experts_than_there_are(ctx):
    w = weights(0x3F80, orc.Q4_K)
    moe = lh.MoeFfnWeights(lh.upload_f32(ctx, np.zeros(NX, np.float32)),
                           **{t: (lh.upload_bytes(ctx, raw), dt) for t, (raw, dt) in w.items()})
    with pytest.raises(lh.LagunaError) as e:
        lh.dispatch_moe_ffn(ctx, lh.upload_f32(ctx, np.zeros(E, np.float32)), moe, lh.GpuBuffer(ctx, 4 * E), E, NX,
                            NX + 1, FFE, SH)
    assert e.value.status == lh.EINVAL
