"""GPU: the dense target forward with hidden capture (lg_target_forward_token,
src/target.rs:298-578) against the f64 oracle, with and without the device K/V
cache and sliding-window RoPE, a target loaded from GGUF, and the verify loop
(src/lib.rs:466-520) end to end with the DFlash draft.

Tolerance: max|err| / max|f64| <= 2e-5 over the logits and each captured state,
on weights of trained magnitude (N(0, 0.02) quantized); the measured errors, which
the tests print, are at most 3.2e-6."""
import numpy as np
import pytest

import dflash_oracle as dfo
import laguna_hip as lh
import synth
import target_oracle as tgo
from gguf_writer import F32, STR, U32, f32_bytes, write_gguf

pytestmark = pytest.mark.gpu

TOL = 2e-5
E, H, KV, HD, FF, NL, V = 512, 4, 2, 128, 1024, 4, 1000


def cfgs(**kw):
    args = dict(n_embd=E, n_heads=H, n_kv=KV, head_dim=HD, n_ff=FF, n_layers=NL, n_vocab=V, rope_dim=HD)
    args.update(kw)
    return lh.TargetConfig(**args), tgo.Hparams(**args)


def rel(y, y64):
    y64 = np.asarray(y64, np.float64)
    return float(np.max(np.abs(np.asarray(y, np.float64) - y64)) / max(np.max(np.abs(y64)), 1e-300))


def build(ctx, seed, cfg, **kw):
    layers, ex = synth.target_model(seed, cfg, **kw)
    model = lh.TargetModel(ctx, cfg, layers, tok_embd=ex["tok_embd"], tok_embd_dtype=ex["tok_embd_dtype"],
                           output_norm=ex["output_norm"], output=ex["output"], output_dtype=ex["output_dtype"])
    return model, layers, ex


def check_step(name, got, want):
    (lg, cap), (lg64, cap64) = got, want
    assert len(cap) == len(cap64), name
    errs = [rel(lg, lg64)] + [rel(c, c64) for c, c64 in zip(cap, cap64)]
    print(f"  {name}: logits {errs[0]:.2e}, captured {['%.2e' % e for e in errs[1:]]}", flush=True)
    assert max(errs) <= TOL, (name, errs)


# mixed weight types: Q8_0 / F32 projections in places, a gate on layers 0 and 2
# only, and layers with 4 and 2 query heads over 2 KV heads
TYPES = {"attn_k": lh.Q8_0, "ffn_up": lh.Q8_0}


def test_forward_token_captures_and_logits(ctx):
    cfg, hp = cfgs()
    print("target forward: 4 layers, capture [1, 2, 4]", flush=True)
    model, layers, ex = build(ctx, 0x7A01, cfg, types=TYPES, gate_layers=[0, 2], n_q_heads=[4, 2, 4, 4])
    x = synth.normal(0x7A02, E)
    for idx in ([1, 2, 4], None, []):
        got = model.forward_token(x, idx)
        want = tgo.forward_token(x, layers, hp, ex["output_norm"], ex["output"], ex["output_dtype"], idx)
        check_step(f"capture {idx}", got, want)
    model.free()


def test_forward_token_f32_gate_and_outputs(ctx):
    # an f32 attention gate and LM head, a Q8_0 down projection (activation kernel + product)
    cfg, hp = cfgs(n_layers=2)
    print("target forward: f32 gate and head, Q8_0 down", flush=True)
    model, layers, ex = build(ctx, 0x7A03, cfg, types={"attn_gate": lh.F32, "ffn_down": lh.Q8_0},
                              output_dtype=lh.F32)
    x = synth.normal(0x7A04, E)
    check_step("f32 gate", model.forward_token(x, [0, 2]),
               tgo.forward_token(x, layers, hp, ex["output_norm"], ex["output"], ex["output_dtype"], [0, 2]))
    model.free()


@pytest.mark.parametrize("swa", [False, True])
def test_forward_token_cached(ctx, swa):
    kw = dict(swa=True, rope_dim_swa=HD, rope_base_swa=10000.0) if swa else {}
    cfg, hp = cfgs(**kw)
    print(f"target cached forward, swa={swa}", flush=True)
    model, layers, ex = build(ctx, 0x7A05, cfg, gate_layers=[1, 3])
    cache, ocache = lh.TargetKvCache(model, 8), tgo.KvCache(NL)
    for t in range(5):
        x = synth.normal(0x7A10 + t, E)
        got = model.forward_token_cached(x, [2], cache)
        want = tgo.forward_token(x, layers, hp, ex["output_norm"], ex["output"], ex["output_dtype"], [2], ocache)
        check_step(f"position {t}", got, want)
        assert cache.len == t + 1
    cache.free()
    model.free()


@pytest.mark.parametrize("cached", [False, True])
def test_forward_token_folded_inputs_and_separate(ctx, cached):
    # Each layer's residual adds and RMSNorms inside its Q4_K input projections (the
    # default: Q, K, V and the gate in one launch, the FFN's gate and up in another, the
    # LM head taking the last add and the output norm) and as their own launches (the
    # switch off): both within TOL of the oracle for the logits and every captured
    # state (each layer's input and the final state), and the normed final hidden of
    # the two within TOL of each other.
    cfg, hp = cfgs()
    print(f"target forward, folded inputs against separate launches, cached={cached}", flush=True)
    model, layers, ex = build(ctx, 0x7A20, cfg, gate_layers=[0, 3], n_q_heads=[4, 2, 4, 4])
    idx = [0, 1, 2, 3, NL]
    steps = 3 if cached else 1
    hidden = {}
    try:
        for folded in (1, 0):
            lh.check(lh.lib().lg_set_fold_norms(folded))
            cache = lh.TargetKvCache(model, steps) if cached else None
            ocache = tgo.KvCache(NL) if cached else None
            hb, cb, lb = lh.GpuBuffer(ctx, 4 * E), lh.GpuBuffer(ctx, 4 * len(idx) * E), lh.GpuBuffer(ctx, 4 * V)
            for t in range(steps):
                x = synth.normal(0x7A21 + t, E)
                xb = lh.upload_f32(ctx, x)
                nc = model.forward_token_device(xb, idx, cb, lb, hidden=hb, cache=cache)
                assert nc == len(idx)
                got = (lb.read_f32(V).copy(), list(cb.read_f32(nc * E).reshape(nc, E).copy()))
                want = tgo.forward_token(x, layers, hp, ex["output_norm"], ex["output"], ex["output_dtype"], idx,
                                         ocache)
                check_step(f"folded={folded} position {t}", got, want)
                hidden[(folded, t)] = hb.read_f32(E).copy()
            if cache is not None:
                assert cache.len == steps
                cache.free()
    finally:
        lh.check(lh.lib().lg_set_fold_norms(1))
    for t in range(steps):
        assert rel(hidden[(1, t)], hidden[(0, t)]) <= TOL


def test_forward_token_folded_inputs_element_fallback(ctx):
    # Norm weights of 1e-30 over a whole 64-element group make that group's normed
    # activations (its maximum included) fall below 2^-60, which the integer-dot digits
    # cannot scale: the layer-input launches (and the LM head, through output_norm) take
    # the per-element loop of the reference's shader, with the residual add and the norm
    # applied per element.  Both paths meet TOL.
    cfg, hp = cfgs(n_layers=2)
    print("target forward, folded inputs on the per-element path", flush=True)
    layers, ex = synth.target_model(0x7A30, cfg)
    for L in layers:
        for nm in ("attn_norm", "ffn_norm"):
            L[nm] = L[nm].copy()
            L[nm][64:128] = 1e-30
    ex["output_norm"] = ex["output_norm"].copy()
    ex["output_norm"][128:192] = 1e-30
    model = lh.TargetModel(ctx, cfg, layers, output_norm=ex["output_norm"], output=ex["output"],
                           output_dtype=ex["output_dtype"])
    x = synth.normal(0x7A31, E)
    want = tgo.forward_token(x, layers, hp, ex["output_norm"], ex["output"], ex["output_dtype"], [0, 1, 2])
    try:
        for folded in (1, 0):
            lh.check(lh.lib().lg_set_fold_norms(folded))
            check_step(f"tiny norm weights, folded={folded}", model.forward_token(x, [0, 1, 2]), want)
    finally:
        lh.check(lh.lib().lg_set_fold_norms(1))
    model.free()


def test_cache_full_is_an_error_and_leaves_len(ctx):
    cfg, _ = cfgs(n_layers=1)
    model, _, _ = build(ctx, 0x7A06, cfg)
    cache = lh.TargetKvCache(model, 2)
    x = synth.normal(0x7A07, E)
    model.forward_token_cached(x, None, cache)
    model.forward_token_cached(x, None, cache)
    with pytest.raises(lh.LagunaError) as e:
        model.forward_token_cached(x, None, cache)
    assert e.value.status == lh.EINVAL and "full" in str(e.value)
    assert cache.len == 2
    cache.free()
    model.free()


def test_no_output_weight_gives_the_normed_hidden(ctx):
    cfg, hp = cfgs(n_layers=2)
    layers, ex = synth.target_model(0x7A08, cfg)
    model = lh.TargetModel(ctx, cfg, layers, output_norm=ex["output_norm"])
    x = synth.normal(0x7A09, E)
    got = model.forward_token(x, [2])
    want = tgo.forward_token(x, layers, hp, ex["output_norm"], None, None, [2])
    check_step("no output weight", got, want)
    model.free()


def test_token_embedding_rows(ctx):
    cfg, _ = cfgs(n_layers=1)
    for dt in (lh.Q8_0, lh.Q4_K, lh.F32):
        model, _, ex = build(ctx, 0x7A0A, cfg, emb_dtype=dt)
        for tok in (0, 17, V - 1):
            want = tgo.token_embedding(ex["tok_embd"], dt, E, tok)
            assert np.array_equal(model.token_embedding(tok), want), (dt, tok)
        with pytest.raises(lh.LagunaError):
            model.token_embedding(V)
        model.free()


def test_gate_attn_glue(ctx):
    n_heads, hd = 8, 128
    a = synth.normal(0x7A0B, n_heads * hd)
    g = np.array([0.0, -3.0, 2.5, 20.5, 40.0, -80.0, 0.125, 7.0], np.float32)
    ab, gb = lh.upload_f32(ctx, a), lh.upload_f32(ctx, g)
    rb = lh.GpuBuffer(ctx, 4 * n_heads * hd)
    lh.dispatch_gate_attn(ctx, ab, gb, rb, n_heads, hd)
    y64 = tgo.gate_attn(a, g, n_heads, hd)
    assert rel(rb.read_f32(n_heads * hd), y64) <= 1e-6
    lh.dispatch_gate_attn(ctx, ab, gb, ab, n_heads, hd)  # in place, as the target calls it
    assert np.array_equal(ab.read_f32(n_heads * hd), rb.read_f32(n_heads * hd))


def _target_gguf(path, cfg, layers, ex, swa=False):
    def t(name, arr, dt, shape):
        return (name, shape, dt, np.asarray(arr).tobytes())

    tensors = [t("token_embd.weight", ex["tok_embd"], ex["tok_embd_dtype"], [E, V]),
               ("output_norm.weight", [E], 0, f32_bytes(ex["output_norm"])),
               t("output.weight", ex["output"], ex["output_dtype"], [E, V])]
    for i, L in enumerate(layers):
        HQ = L["n_q_heads"]
        shapes = {"attn_q": [E, HQ * HD], "attn_k": [E, KV * HD], "attn_v": [E, KV * HD], "attn_gate": [E, HQ],
                  "attn_output": [HQ * HD, E], "ffn_gate": [E, FF], "ffn_up": [E, FF], "ffn_down": [FF, E]}
        for nm in lh.TARGET_NORMS:
            tensors.append((f"blk.{i}.{nm}.weight", [np.asarray(L[nm]).size], 0, f32_bytes(L[nm])))
        for nm in lh.TARGET_PROJ:
            if L[nm] is not None:
                tensors.append(t(f"blk.{i}.{nm}.weight", L[nm], L[nm + "_dtype"], shapes[nm]))
    fields = [("general.architecture", STR, "laguna"), ("laguna.block_count", U32, cfg.n_layers),
              ("laguna.embedding_length", U32, E), ("laguna.feed_forward_length", U32, FF),
              ("laguna.attention.head_count", U32, H), ("laguna.attention.head_count_kv", U32, KV),
              ("laguna.attention.key_length", U32, HD), ("laguna.rope.dimension_count", U32, HD),
              ("laguna.rope.freq_base", F32, 500000.0)]
    if swa:
        fields += [("laguna.rope.dimension_count_swa", U32, HD), ("laguna.rope.freq_base_swa", F32, 10000.0)]
    write_gguf(str(path), fields, tensors)


@pytest.mark.parametrize("swa", [False, True])
def test_target_load_from_gguf(ctx, tmp_path, swa):
    cfg, hp = cfgs(swa=swa, rope_dim_swa=HD if swa else 0)
    layers, ex = synth.target_model(0x7A0C, cfg, types=TYPES, gate_layers=[0, 3], n_q_heads=[4, 2, 4, 2])
    p = tmp_path / "target.gguf"
    _target_gguf(p, cfg, layers, ex, swa)
    print(f"TargetModel.load 4-layer target (swa={swa})", flush=True)
    loaded = lh.TargetModel.load(ctx, str(p))
    assert (loaded.layer_count(), loaded.embedding_length(), loaded.vocab_size()) == (NL, E, V)
    assert loaded.cfg.swa == swa and loaded.cfg.rope_dim_swa == (HD if swa else 0)
    built = lh.TargetModel(ctx, cfg, layers, tok_embd=ex["tok_embd"], tok_embd_dtype=ex["tok_embd_dtype"],
                           output_norm=ex["output_norm"], output=ex["output"], output_dtype=ex["output_dtype"])
    c1, c2, oc = lh.TargetKvCache(loaded, 4), lh.TargetKvCache(built, 4), tgo.KvCache(NL)
    for t in range(3):
        x = loaded.token_embedding(5 + t)
        a = loaded.forward_token_cached(x, [1, 4], c1)
        b = built.forward_token_cached(x, [1, 4], c2)
        assert np.array_equal(a[0], b[0]) and all(np.array_equal(u, v) for u, v in zip(a[1], b[1]))
        check_step(f"loaded, position {t}", a, tgo.forward_token(x, layers, hp, ex["output_norm"], ex["output"],
                                                                 ex["output_dtype"], [1, 4], oc))
    for b in (c1, c2):
        b.free()
    loaded.free()
    built.free()


def test_moe_gguf_is_refused(ctx, tmp_path):
    p = tmp_path / "moe.gguf"
    write_gguf(str(p), [("laguna.block_count", U32, 2), ("laguna.embedding_length", U32, 256),
                        ("laguna.feed_forward_length", U32, 512), ("laguna.attention.head_count", U32, 2),
                        ("laguna.attention.head_count_kv", U32, 1), ("laguna.attention.key_length", U32, 128)],
               [("blk.1.ffn_gate_exps.weight", [256, 512, 2], 0, f32_bytes(np.zeros(256 * 512 * 2)))])
    with pytest.raises(lh.LagunaError) as e:
        lh.TargetModel.load(ctx, str(p))
    assert e.value.status == lh.EUNSUPPORTED


def test_verify_loop_end_to_end(ctx):
    """run_target_dflash_verify with a 4-layer target and a 2-layer draft reading
    target layers [1, 2, 4]: each step's draft and target tokens equal the f64
    oracle's on the same input token wherever the oracle's top-two margin exceeds
    the measured error."""
    cfg, hp = cfgs()
    target, layers, ex = build(ctx, 0x7A0D, cfg, gate_layers=[0, 1])
    dcfg = lh.DFlashConfig(n_embd=E, n_heads=4, n_kv=2, head_dim=HD, rope_dim=HD, n_ff=768, n_aux=3, n_layers=2)
    W, dl = synth.dflash_model(0x7A0E, dcfg, 2, norm_sigma=0.1, trained_scale=True)
    tl = [1, 2, 4]
    draft = lh.DFlashModel(ctx, dcfg, W, dl, target_layers=tl)
    lines = []
    accepted, exact, steps = lh.run_target_dflash_verify(target, draft, 11, 5, log=lines.append)
    print("\n".join(lines), flush=True)
    assert len(accepted) == 5 and exact == sum(s[3] for s in steps)
    kc = [np.zeros((0, dcfg.n_kv * HD), np.float32)] * 2
    decided = 0
    for tok, d, t, ok in steps:
        emb = tgo.token_embedding(ex["tok_embd"], ex["tok_embd_dtype"], E, tok)
        lg64, cap64 = tgo.forward_token(emb, layers, hp, ex["output_norm"], ex["output"], ex["output_dtype"], tl)
        feat = np.concatenate(cap64).reshape(1, -1)
        dh = dfo.forward_block(feat, emb.reshape(1, -1), W, dl, kc, kc, 0, dcfg)[0]
        dlg64 = dfo.proj(dh, ex["output"], ex["output_dtype"], E, V)[0]
        for name, got, lg in (("target", t, lg64), ("draft", d, dlg64)):
            top = np.sort(lg)[-2:]
            if top[1] - top[0] > 10 * TOL * np.max(np.abs(lg)):
                assert got == int(np.argmax(lg)), (name, tok)
                decided += 1
        assert ok == (d == t)
    assert decided >= 6  # most decisions are clear on random weights
    draft.free()
    target.free()
