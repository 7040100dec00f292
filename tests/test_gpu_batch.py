"""GPU: small-M (block verify) products against the oracle's f64 accumulation."""
import numpy as np
import pytest

import laguna_hip as lh
import oracle as orc
import synth
from conftest import parity

pytestmark = pytest.mark.gpu

TOL = 1e-4


def bf16_bits(x):
    """Round float32 to bf16 (nearest-even) and return the raw 16-bit codes."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def run_batch(ctx, x, x_dtype, raw, w_dtype, k, n, m):
    xb = lh.upload_bytes(ctx, np.ascontiguousarray(x).view(np.uint8).ravel())
    wb = lh.upload_bytes(ctx, np.ascontiguousarray(raw).view(np.uint8).ravel())
    cb = lh.GpuBuffer(ctx, 4 * m * n)
    lh.dispatch_proj_quant_batch(ctx, xb, x_dtype, wb, cb, k, n, m, w_dtype)
    return cb.read_f32(m * n).reshape(m, n)


@pytest.mark.parametrize("w_dtype,k,n,x_dtype,seed", [
    (lh.Q4_K, 4096, 14336, lh.BF16, 0x5EED0008),
    (lh.Q4_K, 4096, 14336, lh.F32, 0x5EED0008),
    (lh.Q8_0, 4096, 4096, lh.F32, 0x5EED0009),
    (lh.Q8_0, 4096, 4096, lh.BF16, 0x5EED0009),
])
def test_block_verify_configs(ctx, w_dtype, k, n, x_dtype, seed):
    m = 16
    print(f"batch m=16 w={w_dtype} x={x_dtype} k={k} n={n} seed={seed:#x}", flush=True)
    raw = synth.q4k_weight(seed, k, n) if w_dtype == lh.Q4_K else synth.q8_0_weight(seed, k, n)
    x32 = synth.normal(seed + 0x100, m * k).reshape(m, k)
    if x_dtype == lh.BF16:
        xin = bf16_bits(x32)
        xref = (xin.astype(np.uint32) << 16).view(np.float32)
    else:
        xin, xref = x32, x32
    c = run_batch(ctx, xin, x_dtype, raw, w_dtype, k, n, m)
    y64, a = orc.proj_quant_f64(xref, raw, w_dtype, k, n)
    parity(c, y64, a, TOL)


@pytest.mark.parametrize("m", [1, 2, 5, 15, 16, 17, 31, 33, 48, 64])
@pytest.mark.parametrize("w_dtype", [lh.Q4_K, lh.Q8_0])
def test_token_counts(ctx, m, w_dtype):
    k, n = 1024, 100
    print(f"batch m={m} w={w_dtype}", flush=True)
    raw = synth.q4k_weight(200 + m, k, n) if w_dtype == lh.Q4_K else synth.q8_0_weight(200 + m, k, n)
    x = synth.normal(300 + m, m * k).reshape(m, k)
    c = run_batch(ctx, x, lh.F32, raw, w_dtype, k, n, m)
    y64, a = orc.proj_quant_f64(x, raw, w_dtype, k, n)
    parity(c, y64, a, TOL)


def test_m1_matches_matvec(ctx):
    k, n = 4096, 512
    raw = synth.q4k_weight(400, k, n)
    x = synth.normal(401, k)
    print("batch m=1 vs matvec", flush=True)
    c = run_batch(ctx, x[None, :], lh.F32, raw, lh.Q4_K, k, n, 1)[0]
    xb, wb, cb = lh.upload_f32(ctx, x), lh.upload_bytes(ctx, raw), lh.GpuBuffer(ctx, 4 * n)
    lh.dispatch_proj_quant(ctx, xb, wb, cb, k, n, lh.Q4_K)
    y = cb.read_f32(n)
    y64, a = orc.proj_quant_f64(x, raw, orc.Q4_K, k, n)
    parity(c, y64, a, TOL)
    parity(y, y64, a, TOL)


@pytest.mark.parametrize("w_dtype,k,n,m", [(lh.F32, 512, 40, 7), (lh.Q4_K, 96, 8, 3), (lh.Q8_0, 4128, 9, 20)])
def test_generic_path(ctx, w_dtype, k, n, m):
    print(f"batch generic w={w_dtype} k={k} n={n} m={m}", flush=True)
    if w_dtype == lh.F32:
        raw = synth.normal(500, k * n, 0.02)
    elif w_dtype == lh.Q4_K:
        raw = synth.random_q4k(501, -(-(k * n) // 256))
    else:
        raw = synth.q8_0_weight(502, 32, -(-(k * n) // 32))
    x = synth.normal(503, m * k).reshape(m, k)
    c = run_batch(ctx, x, lh.F32, raw, w_dtype, k, n, m)
    y64, a = orc.proj_quant_f64(x, raw, w_dtype, k, n)
    parity(c, y64, a, TOL)


def test_workspace_reuse_across_shapes(ctx):
    # the workspace (fragments, partial sums) grows and is reused: a call's result
    # must not depend on what earlier calls left in it.  (The split of k into
    # slices depends on the token count, so the same token need not round
    # identically at different m; at the same shape it must.)
    k, n = 2048, 64
    raw = synth.q4k_weight(600, k, n)
    x = synth.normal(601, 40 * k).reshape(40, k)
    print("batch workspace reuse", flush=True)
    small = run_batch(ctx, x[:3], lh.F32, raw, lh.Q4_K, k, n, 3)
    big = run_batch(ctx, x, lh.F32, raw, lh.Q4_K, k, n, 40)
    again = run_batch(ctx, x[:3], lh.F32, raw, lh.Q4_K, k, n, 3)
    assert np.array_equal(small, again)
    y64, a = orc.proj_quant_f64(x, raw, lh.Q4_K, k, n)
    parity(big, y64, a, TOL)


@pytest.mark.parametrize("ch,rt", [(1, 1), (1, 4), (2, 1), (2, 2), (2, 4), (4, 1), (4, 2)])
@pytest.mark.parametrize("m", [16, 29])
def test_launch_shapes(ctx, ch, rt, m):
    # Every launch shape (k slice length, rows per wavefront) meets parity and is
    # repeatable; k = 2816 is 11 super-blocks, so the last slice of a 2- or
    # 4-super-block shape runs past the end of k.
    k, n = 2816, 700
    print(f"batch shape ch={ch} rt={rt} m={m}", flush=True)
    raw = synth.q4k_weight(400 + m, k, n)
    x = synth.normal(410 + m, m * k).reshape(m, k)
    lh.check(lh.lib().lg_set_batch_shape(ch, rt))
    try:
        c1 = run_batch(ctx, x, lh.F32, raw, lh.Q4_K, k, n, m)
        c2 = run_batch(ctx, x, lh.F32, raw, lh.Q4_K, k, n, m)
    finally:
        lh.check(lh.lib().lg_set_batch_shape(0, 0))
    assert np.array_equal(c1, c2)
    y64, a = orc.proj_quant_f64(x, raw, lh.Q4_K, k, n)
    parity(c1, y64, a, TOL)


def run_gate_up(ctx, x, raw_g, raw_u, w_dtype, k, n, m):
    xb = lh.upload_f32(ctx, np.ascontiguousarray(x, np.float32).ravel())
    gb, ub = lh.upload_bytes(ctx, np.ascontiguousarray(raw_g).view(np.uint8).ravel()), \
        lh.upload_bytes(ctx, np.ascontiguousarray(raw_u).view(np.uint8).ravel())
    hb, sb = lh.GpuBuffer(ctx, 4 * m * n), lh.GpuBuffer(ctx, 4 * m * n)
    lh.dispatch_silu_gate_up_batch(ctx, xb, gb, ub, hb, sb, k, n, m, w_dtype)
    return hb.read_f32(m * n).reshape(m, n)


def gate_up_parity(h, x, raw_g, raw_u, w_dtype, k, n):
    """h against silu(g) * u from the oracle's f64 products; the bound carries each
    product's sum |W_ij x_j| through the activation (|silu'| < 1.1)."""
    g64, ag = orc.proj_quant_f64(x, raw_g, w_dtype, k, n)
    u64, au = orc.proj_quant_f64(x, raw_u, w_dtype, k, n)
    sg = g64 / (1.0 + np.exp(-g64))
    parity(h, sg * u64, 1.1 * np.abs(u64) * ag + np.abs(sg) * au, TOL)


def weights(w_dtype, seed, k, n):
    if w_dtype == lh.Q4_K:  # k = 96: blocks run across rows (the reference's linear addressing)
        return synth.q4k_weight(seed, k, n) if k % 256 == 0 else synth.random_q4k(seed, -(-(k * n) // 256))
    if w_dtype == lh.Q8_0:
        return synth.q8_0_weight(seed, k, n)
    return synth.normal(seed, k * n, 0.02)


@pytest.mark.parametrize("w_dtype,k,n,m", [
    (lh.Q4_K, 4096, 1536, 16), (lh.Q4_K, 4096, 1536, 1), (lh.Q4_K, 2816, 700, 29), (lh.Q4_K, 1024, 300, 40),
    (lh.Q8_0, 1024, 700, 16), (lh.Q8_0, 4096, 512, 33),
    (lh.F32, 512, 40, 7), (lh.Q4_K, 96, 8, 3),  # outside the matrix-core path
])
def test_silu_gate_up(ctx, w_dtype, k, n, m):
    # The FFN's gate and up products with the activation (src/dflash.rs:963-965)
    print(f"gate/up pair w={w_dtype} k={k} n={n} m={m}", flush=True)
    raw_g, raw_u = weights(w_dtype, 500 + m, k, n), weights(w_dtype, 600 + m, k, n)
    x = synth.normal(700 + m, m * k).reshape(m, k)
    h = run_gate_up(ctx, x, raw_g, raw_u, w_dtype, k, n, m)
    assert np.array_equal(h, run_gate_up(ctx, x, raw_g, raw_u, w_dtype, k, n, m))
    gate_up_parity(h, x, raw_g, raw_u, w_dtype, k, n)


@pytest.mark.parametrize("ch,rt", [(1, 1), (1, 4), (2, 2), (2, 4), (4, 2)])
def test_silu_gate_up_launch_shapes(ctx, ch, rt):
    k, n, m = 2816, 700, 29
    print(f"gate/up pair shape ch={ch} rt={rt}", flush=True)
    raw_g, raw_u = synth.q4k_weight(800, k, n), synth.q4k_weight(801, k, n)
    x = synth.normal(802, m * k).reshape(m, k)
    lh.check(lh.lib().lg_set_batch_shape(ch, rt))
    try:
        h = run_gate_up(ctx, x, raw_g, raw_u, lh.Q4_K, k, n, m)
    finally:
        lh.check(lh.lib().lg_set_batch_shape(0, 0))
    gate_up_parity(h, x, raw_g, raw_u, lh.Q4_K, k, n)


def tile_q4k(raw, k, n):
    """The LG_Q4_K_T16 layout restated in numpy: tile (t, b) = 16 row headers, then
    quant bytes [group g][piece p][row r]; rows past n are zero blocks."""
    nb, nt = k // 256, -(-n // 16)
    blocks = np.zeros((nt * 16, nb, 144), np.uint8)
    blocks[:n] = np.frombuffer(np.ascontiguousarray(raw).tobytes(), np.uint8).reshape(n, nb, 144)
    blocks = blocks.reshape(nt, 16, nb, 144).transpose(0, 2, 1, 3)  # [t][b][r][144]
    hdr = blocks[..., :16].reshape(nt, nb, 256)
    q = blocks[..., 16:].reshape(nt, nb, 16, 4, 4, 8).transpose(0, 1, 3, 4, 2, 5).reshape(nt, nb, 2048)
    return np.concatenate([hdr, q], axis=2).ravel()


def tile_q80(raw, k, n):
    """The LG_Q8_0_T16 layout restated in numpy: tile (t, c) = the 16 rows' 8 f16
    scales (row-major), then quants [block j][piece p][row r], biased to unsigned
    (q + 128 = q XOR 0x80); rows past n are zero bytes."""
    nc, nt = k // 256, -(-n // 16)
    blocks = np.zeros((nt * 16, nc, 8, 34), np.uint8)
    blocks[:n] = np.frombuffer(np.ascontiguousarray(raw).tobytes(), np.uint8).reshape(n, nc, 8, 34)
    blocks[:n, :, :, 2:] ^= 0x80
    blocks = blocks.reshape(nt, 16, nc, 8, 34).transpose(0, 2, 1, 3, 4)  # [t][c][r][j][34]
    sc = blocks[..., :2].reshape(nt, nc, 256)
    q = blocks[..., 2:].reshape(nt, nc, 16, 8, 4, 8).transpose(0, 1, 3, 4, 2, 5).reshape(nt, nc, 4096)
    return np.concatenate([sc, q], axis=2).ravel()


@pytest.mark.parametrize("k,n", [(4096, 512), (2048, 37), (256, 3)])
def test_repack_tiled_q80_layout(ctx, k, n):
    print(f"repack Q8_0 k={k} n={n}", flush=True)
    raw = synth.q8_0_weight(930 + n, k, n)
    tb = lh.repack_tiled(ctx, lh.upload_bytes(ctx, raw), lh.Q8_0, k, n)
    assert tb.size == lh.lib().lg_tiled_bytes(lh.Q8_0, k, n) == -(-n // 16) * (k // 256) * 4352
    assert np.array_equal(tb.download(), tile_q80(raw, k, n))


@pytest.mark.parametrize("k,n,m,ch", [(4096, 4096, 16, 0), (2048, 37, 29, 0), (4096, 700, 5, 2), (1024, 300, 40, 1)])
def test_tiled_q80_products_equal_raw(ctx, k, n, m, ch):
    print(f"tiled Q8_0 product k={k} n={n} m={m} ch={ch}", flush=True)
    raw = synth.q8_0_weight(940 + n, k, n)
    x = synth.normal(941 + m, m * k).reshape(m, k)
    wb = lh.upload_bytes(ctx, raw)
    tb = lh.repack_tiled(ctx, wb, lh.Q8_0, k, n)
    lh.check(lh.lib().lg_set_batch_shape(ch, 0))
    try:
        c_raw = run_batch(ctx, x, lh.F32, raw, lh.Q8_0, k, n, m)
        xb, c_t = lh.upload_f32(ctx, x.ravel()), lh.GpuBuffer(ctx, 4 * m * n)
        lh.dispatch_proj_quant_batch(ctx, xb, lh.F32, tb, c_t, k, n, m, lh.Q8_0_T16)
    finally:
        lh.check(lh.lib().lg_set_batch_shape(0, 0))
    ct = c_t.read_f32(m * n).reshape(m, n)
    assert np.array_equal(ct, c_raw)
    y64, a = orc.proj_quant_f64(x, raw, lh.Q8_0, k, n)
    parity(ct, y64, a, TOL)


@pytest.mark.parametrize("k,n", [(4096, 1536), (2816, 700), (256, 5), (1024, 33)])
def test_repack_tiled_layout(ctx, k, n):
    print(f"repack Q4_K k={k} n={n}", flush=True)
    raw = synth.q4k_weight(900 + n, k, n)
    wb = lh.upload_bytes(ctx, raw)
    tb = lh.repack_tiled(ctx, wb, lh.Q4_K, k, n)
    assert tb.size == lh.lib().lg_tiled_bytes(lh.Q4_K, k, n) == -(-n // 16) * (k // 256) * 2304
    assert np.array_equal(tb.download(), tile_q4k(raw, k, n))


@pytest.mark.parametrize("k,n,m,x_dtype", [
    (4096, 1536, 16, lh.F32), (4096, 1536, 16, lh.BF16), (2816, 700, 29, lh.F32), (1024, 33, 1, lh.F32),
    (4096, 14336, 16, lh.F32), (256, 5, 40, lh.F32),
])
def test_tiled_products_equal_raw(ctx, k, n, m, x_dtype):
    # the same kernels over tiles: results equal the raw layout's bit for bit
    print(f"tiled product k={k} n={n} m={m} x={x_dtype}", flush=True)
    raw = synth.q4k_weight(950 + n, k, n)
    x32 = synth.normal(960 + m, m * k).reshape(m, k)
    xin = bf16_bits(x32) if x_dtype == lh.BF16 else x32
    xref = (xin.astype(np.uint32) << 16).view(np.float32) if x_dtype == lh.BF16 else x32
    wb = lh.upload_bytes(ctx, raw)
    tb = lh.repack_tiled(ctx, wb, lh.Q4_K, k, n)
    xb = lh.upload_bytes(ctx, np.ascontiguousarray(xin).view(np.uint8).ravel())
    c_raw, c_t = lh.GpuBuffer(ctx, 4 * m * n), lh.GpuBuffer(ctx, 4 * m * n)
    lh.dispatch_proj_quant_batch(ctx, xb, x_dtype, wb, c_raw, k, n, m, lh.Q4_K)
    lh.dispatch_proj_quant_batch(ctx, xb, x_dtype, tb, c_t, k, n, m, lh.Q4_K_T16)
    ct = c_t.read_f32(m * n)
    assert np.array_equal(ct, c_raw.read_f32(m * n))
    y64, a = orc.proj_quant_f64(xref, raw, lh.Q4_K, k, n)
    parity(ct.reshape(m, n), y64, a, TOL)


@pytest.mark.parametrize("ch,rt", [(1, 1), (2, 4), (4, 2)])
def test_tiled_launch_shapes_and_pair(ctx, ch, rt):
    k, n, m = 2816, 700, 29
    print(f"tiled shapes ch={ch} rt={rt}", flush=True)
    rg, ru = synth.q4k_weight(970, k, n), synth.q4k_weight(971, k, n)
    x = synth.normal(972, m * k).reshape(m, k)
    gb, ub = lh.upload_bytes(ctx, rg), lh.upload_bytes(ctx, ru)
    tg, tu = lh.repack_tiled(ctx, gb, lh.Q4_K, k, n), lh.repack_tiled(ctx, ub, lh.Q4_K, k, n)
    xb = lh.upload_f32(ctx, x.ravel())
    h1, h2, sc = (lh.GpuBuffer(ctx, 4 * m * n) for _ in range(3))
    lh.check(lh.lib().lg_set_batch_shape(ch, rt))
    try:
        lh.dispatch_silu_gate_up_batch(ctx, xb, gb, ub, h1, sc, k, n, m, lh.Q4_K)
        lh.dispatch_silu_gate_up_batch(ctx, xb, tg, tu, h2, sc, k, n, m, lh.Q4_K_T16)
    finally:
        lh.check(lh.lib().lg_set_batch_shape(0, 0))
    h = h2.read_f32(m * n)
    assert np.array_equal(h, h1.read_f32(m * n))
    gate_up_parity(h.reshape(m, n), x, rg, ru, lh.Q4_K, k, n)


def test_tiled_rejects_bad_input(ctx):
    raw = synth.q4k_weight(980, 512, 16)
    wb = lh.upload_bytes(ctx, raw)
    with pytest.raises(lh.LagunaError):
        lh.check(lh.lib().lg_repack_tiled(wb.ptr, lh.F32, 512, 16, wb.ptr, ctx.stream))
    with pytest.raises(lh.LagunaError):  # k not a multiple of 256
        lh.check(lh.lib().lg_repack_tiled(wb.ptr, lh.Q8_0, 96, 16, wb.ptr, ctx.stream))
    assert lh.lib().lg_tiled_bytes(lh.Q4_K, 500, 16) == 0
    assert lh.lib().lg_tiled_bytes(lh.F32, 512, 16) == 0
