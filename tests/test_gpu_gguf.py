"""GPU: tensors loaded through the GGUF reader (Model::upload_tensor_quantized,
src/model.rs:174-184) arrive unchanged on the device, feed the projections, and a
draft model loaded from a GGUF file (DFlashModel::load, src/dflash.rs:34-120)
computes the same forward as the one built from the same arrays."""
import numpy as np
import pytest

import dflash_oracle as dfo
import laguna_hip as lh
import oracle as orc
import synth
from conftest import parity
from gguf_writer import ARR, F32, I32, STR, U32, f32_bytes, write_gguf

pytestmark = pytest.mark.gpu


def test_upload_is_byte_exact_across_staging_chunks(ctx, tmp_path):
    # 20 MB spans three 8 MB staging halves; the odd-sized tensor ends mid-chunk
    rng = np.random.default_rng(11)
    big = rng.integers(0, 256, (20 * 2**20 // 34 + 1) * 34, np.uint8)  # whole Q8_0 blocks
    odd = rng.integers(0, 256, 34 * 7, np.uint8)
    p = tmp_path / "w.gguf"
    write_gguf(str(p), [("general.alignment", U32, 64)],
               [("big", [32 * (big.size // 34)], 8, big.tobytes()), ("odd", [224], 8, odd.tobytes())], alignment=64)
    print("gguf upload 20 MB + 238 B", flush=True)
    with lh.GGUFReader(str(p)) as rd:
        for t, raw in zip(rd.tensors, (big, odd)):
            b = rd.upload_tensor_quantized(ctx, t)
            assert np.array_equal(b.download(t.n_bytes()), raw), t.name


def test_projection_on_uploaded_tensor(ctx, tmp_path):
    k, n = 4096, 1024
    raw = synth.q4k_weight(0x5EED0300, k, n)
    x = synth.normal(0x5EED0301, k)
    p = tmp_path / "proj.gguf"
    write_gguf(str(p), [], [("blk.0.ffn_up.weight", [k, n], lh.Q4_K, raw.tobytes())])
    print("gguf Q4_K 4096x1024 projection", flush=True)
    with lh.GGUFReader(str(p)) as rd:
        w = rd.upload_tensor_quantized(ctx, rd.tensor_by_name("blk.0.ffn_up.weight"))
    xb, cb = lh.upload_f32(ctx, x), lh.GpuBuffer(ctx, 4 * n)
    lh.dispatch_proj_quant(ctx, xb, w, cb, k, n, lh.Q4_K)
    y64, a = orc.proj_quant_f64(x, raw, lh.Q4_K, k, n)
    parity(cb.read_f32(n), y64, a, 1e-4)


def _dflash_gguf(path, cfg, W, layers, norm_dtype=0):
    shapes = synth.dflash_shapes(cfg)

    def norm(name, v):
        v = np.asarray(v, np.float32)
        if norm_dtype == 1:  # F16 norms: loaded through the device dequantizer
            return (name, [v.size], 1, v.astype(np.float16).tobytes())
        return (name, [v.size], 0, f32_bytes(v))

    A = cfg.n_aux * cfg.n_embd
    tensors = [norm("enc.aux_norm.weight", W["enc_aux_norm"]), ("fc.weight", [A, cfg.n_embd], W["fc_dtype"],
                                                                 np.asarray(W["fc"]).tobytes()),
               norm("enc.output_norm.weight", W["enc_output_norm"]), norm("output_norm.weight", W["output_norm"])]
    for i, L in enumerate(layers):
        for nm in synth.DFLASH_NORMS:
            tensors.append(norm(f"blk.{i}.{nm}.weight", L[nm]))
        for nm in synth.DFLASH_PROJ:
            kk, nn = shapes[nm]
            tensors.append((f"blk.{i}.{nm}.weight", [kk, nn], L[nm + "_dtype"], np.asarray(L[nm]).tobytes()))
    fields = [("general.architecture", STR, "dflash"), ("dflash.block_count", U32, cfg.n_layers),
              ("dflash.embedding_length", U32, cfg.n_embd), ("dflash.feed_forward_length", U32, cfg.n_ff),
              ("dflash.attention.head_count", U32, cfg.n_heads), ("dflash.attention.head_count_kv", U32, cfg.n_kv),
              ("dflash.attention.key_length", U32, cfg.head_dim), ("dflash.rope.dimension_count", U32, cfg.rope_dim),
              ("dflash.rope.freq_base", F32, cfg.rope_base),
              ("dflash.target_layers", ARR, (I32, list(range(cfg.n_aux))))]
    write_gguf(str(path), fields, tensors)


@pytest.mark.parametrize("norm_dtype", [0, 1])
def test_dflash_model_load(ctx, tmp_path, norm_dtype):
    cfg = lh.DFlashConfig(n_embd=512, n_heads=4, n_kv=2, head_dim=128, rope_dim=128, n_ff=768, n_aux=3, n_layers=2)
    m, ctx_len = 16, 40
    W, layers = synth.dflash_model(0x5EED0310, cfg, cfg.n_layers, norm_sigma=0.1)
    if norm_dtype == 1:  # the file holds f16 norms; compare against their f16 values
        for L in [W] + layers:
            for key in list(L):
                if key.endswith("norm"):
                    L[key] = np.asarray(L[key], np.float16).astype(np.float32)
    feat, tok, kc, vc = synth.dflash_inputs(0x5EED0311, cfg, cfg.n_layers, m, ctx_len)
    p = tmp_path / "draft.gguf"
    _dflash_gguf(p, cfg, W, layers, norm_dtype)
    print(f"DFlashModel.load 2-layer draft (norm dtype {norm_dtype})", flush=True)
    loaded = lh.DFlashModel.load(ctx, str(p))
    assert (loaded.layer_count(), loaded.embedding_length(), loaded.head_count(), loaded.head_count_kv(),
            loaded.head_dim(), loaded.ffn_length(), loaded.n_embd_inp()) == (2, 512, 4, 2, 128, 768, 1536)
    loaded.set_context(kc, vc)
    built = lh.DFlashModel(ctx, cfg, W, layers)
    built.set_context(kc, vc)
    y = loaded.forward_block(feat, tok)
    assert np.array_equal(y, built.forward_block(feat, tok))  # the same bytes on the device
    want = dfo.forward_block(feat, tok, W, layers, kc, vc, ctx_len, cfg)
    e = float(np.max(np.abs(y.astype(np.float64) - want)) / np.max(np.abs(want)))
    assert e <= 1e-3, e
    loaded.free()
    built.free()


def test_dflash_model_load_missing_tensor(ctx, tmp_path):
    p = tmp_path / "partial.gguf"
    write_gguf(str(p), [("dflash.block_count", U32, 1), ("dflash.embedding_length", U32, 256),
                        ("dflash.feed_forward_length", U32, 512), ("dflash.attention.head_count", U32, 2),
                        ("dflash.attention.head_count_kv", U32, 1), ("dflash.attention.key_length", U32, 128)],
               [("enc.aux_norm.weight", [256], 0, f32_bytes(np.ones(256)))])
    with pytest.raises(lh.LagunaError) as e:
        lh.DFlashModel.load(ctx, str(p))
    assert e.value.status == lh.ENOTFOUND and "enc.output_norm.weight" in str(e.value)
