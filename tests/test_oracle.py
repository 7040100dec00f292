"""CPU checks that pin the oracle: the reference's own known answers, closed forms
that isolate each index/packing rule, and the independent numpy restatement
stored in tests/golden/golden.npz."""
import os
import sys

import numpy as np
import pytest

import oracle as orc
import synth

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import make_golden  # noqa: E402  (the independent numpy restatement)

pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")


# ---------------------------------------------------------------- f16 decoder

def test_half_reference_unit_tests():
    # src/dflash.rs:1334-1344 (test_dequant_bf16, which decodes binary16)
    assert orc.half_to_f32(0x3C00) == 1.0
    assert orc.half_to_f32(0x3E00) == 1.5


def test_half_matches_ieee_except_subnormals(golden):
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    # Through an array (the "BF16" branch applies the half decoder per element): a
    # scalar ctypes float return would quiet signalling-NaN payloads on the way.
    ours = orc.dequant_to_f32(codes.view(np.uint8), orc.BF16, 65536).view(np.uint32)
    assert np.array_equal(ours, golden["half_bits"])
    exp = (codes >> 10) & 31
    normal = (exp != 0) & (exp != 31)
    ieee = codes.view(np.float16).astype(np.float32).view(np.uint32)
    assert np.array_equal(ours[normal], ieee[normal])           # every normal code is IEEE
    zero = (codes & 0x7FFF) == 0
    assert np.array_equal(ours[zero], ieee[zero])               # +-0
    inf = (exp == 31) & ((codes & 0x3FF) == 0)
    assert np.all(np.isinf(ours[inf].view(np.float32)))


def test_half_subnormal_quirk_closed_form():
    # exponent 0, mantissa m != 0 -> 2^-14 * (1 + m/1024), not 2^-24 * m
    assert orc.half_to_f32(0x0001) == np.float32(2.0 ** -14 * (1 + 1 / 1024))
    assert orc.half_to_f32(0x03FF) == np.float32(2.0 ** -14 * (1 + 1023 / 1024))
    assert orc.half_to_f32(0x8001) == -np.float32(2.0 ** -14 * (1 + 1 / 1024))
    assert abs(orc.half_to_f32(0x0001) - 6.109476e-05) < 1e-11


# ---------------------------------------------------------------- dequant_to_f32

def test_dequant_q8_0_reference_unit_test():
    # src/dflash.rs:1347-1356: d = 0x3C00 (1.0), q = 1 -> 1.0
    data = np.zeros(34, np.uint8)
    data[0:2] = np.array([0x3C00], np.uint16).view(np.uint8)
    data[2:] = 1
    out = orc.dequant_to_f32(data, orc.Q8_0, 32)
    assert abs(out[0] - 1.0) < 1e-3 and np.all(out == 1.0)


def test_dequant_f32_and_unsupported_reference_unit_tests():
    # src/dflash.rs:1359-1373
    vals = (np.arange(16, dtype=np.float32) * np.float32(0.001))
    out = orc.dequant_to_f32(vals.view(np.uint8), orc.F32, 16)
    assert abs(out[5] - 0.005) < 1e-6 and np.array_equal(out, vals)
    out = orc.dequant_to_f32(np.zeros(32, np.uint8), 4, 16)  # Q5_0: unsupported
    assert out.shape == (16,) and np.all(out == 0.0)


def test_dequant_q8_0_closed_forms():
    for d_code, d in [(0x3C00, 1.0), (0x0400, 2.0 ** -14), (0x7BFF, 65504.0)]:
        blk = np.zeros(34, np.uint8)
        blk[0:2] = np.array([d_code], np.uint16).view(np.uint8)
        q = np.array([-128, -1, 0, 1, 127] + [0] * 27, np.int8)
        blk[2:] = q.view(np.uint8)
        out = orc.dequant_to_f32(blk, orc.Q8_0, 32)
        assert np.array_equal(out, (q.astype(np.float64) * d).astype(np.float32))


def test_dequant_q8_0_golden(golden):
    out = orc.dequant_to_f32(golden["q8_raw"], orc.Q8_0, int(golden["q8_n"]))
    assert np.array_equal(out.view(np.uint32), golden["q8_deq"].view(np.uint32))


def test_dequant_q8_0_truncated_data_leaves_zeros():
    raw = synth.q8_0_weight(7, 64, 2)          # 4 blocks
    out = orc.dequant_to_f32(raw[: 3 * 34 + 10], orc.Q8_0, 128)
    full = orc.dequant_to_f32(raw, orc.Q8_0, 128)
    assert np.array_equal(out[:96], full[:96]) and np.all(out[96:] == 0)


def test_legacy_q4k_closed_form(golden):
    out = orc.dequant_to_f32(golden["legacy_blk"], orc.Q4_K, 256)
    assert np.array_equal(out, golden["legacy_out"])


def test_half_branches_f16_vs_bf16():
    codes = np.array([0x3C00, 0x0001, 0x8000, 0x7C00, 0xFC00, 0x7E01], np.uint16)
    f16 = orc.dequant_to_f32(codes.view(np.uint8), orc.F16, codes.size)
    bf = orc.dequant_to_f32(codes.view(np.uint8), orc.BF16, codes.size)
    assert f16[0] == 1.0 and bf[0] == 1.0
    assert f16[1] == np.float32(2.0 ** -24)                          # F16 branch: IEEE subnormal
    assert bf[1] == np.float32(2.0 ** -14 * (1 + 1 / 1024))          # "BF16" branch: quirk
    assert np.signbit(f16[2]) and f16[2] == 0
    assert np.isposinf(f16[3]) and np.isneginf(f16[4])
    assert f16[5:].view(np.uint32)[0] == 0x7FC00000                    # canonical NaN
    assert bf[5:].view(np.uint32)[0] == 0x7F800000 | (0x201 << 13)     # payload kept


# ---------------------------------------------------------------- ggml Q4_K decode

def _q4_block(d=0x3C00, dmin=0x0000, scales=None, qs=None):
    blk = np.zeros(144, np.uint8)
    blk[0:4] = np.array([d, dmin], np.uint16).view(np.uint8)
    if scales is not None:
        blk[4:16] = scales
    if qs is not None:
        blk[16:] = qs
    return blk


def test_q4k_nibble_order_closed_form():
    # d = 1, dmin = 0, every scale 1 -> value = q; low nibbles are elements 0-31 of
    # each 64-group, high nibbles 32-63.
    sc = np.zeros(12, np.uint8)
    sc[0:4] = 1                    # sc[0..3] = 1
    sc[8:12] = 1                   # sc[4..7] low nibble = 1 (m[4..7] = 0)
    qs = (np.arange(128) % 16 | ((15 - np.arange(128) % 16) << 4)).astype(np.uint8)
    out = orc.dequant_q4k(_q4_block(scales=sc, qs=qs), 256)
    for g in range(4):
        i = np.arange(32)
        b = qs[32 * g + i]
        assert np.array_equal(out[64 * g + i], (b & 15).astype(np.float32))
        assert np.array_equal(out[64 * g + 32 + i], (b >> 4).astype(np.float32))


def test_q4k_min_closed_form():
    # sc = 0, m = 1, dmin = 1 -> -1 everywhere
    sc = np.zeros(12, np.uint8)
    sc[4:8] = 1
    sc[8:12] = 0x10
    out = orc.dequant_q4k(_q4_block(dmin=0x3C00, scales=sc, qs=np.full(128, 0x5A, np.uint8)), 256)
    assert np.all(out == -1.0)


@pytest.mark.parametrize("j", range(8))
def test_q4k_scale_packing_isolated(j):
    # Set exactly the bits that feed sub-block j's scale (value 37 = 0b100101) and
    # min (value 22 = 0b010110); every other sub-block must decode sc = m = 0.
    sc = np.zeros(12, np.uint8)
    S, Mv = 37, 22
    if j < 4:
        sc[j] = S
        sc[j + 4] = Mv
    else:
        sc[j + 4] = (S & 15) | ((Mv & 15) << 4)
        sc[j - 4] = (S >> 4) << 6
        sc[j] = (Mv >> 4) << 6
    qs = np.full(128, 0x11, np.uint8)  # q = 1 everywhere
    out = orc.dequant_q4k(_q4_block(d=0x3C00, dmin=0x3C00, scales=sc, qs=qs), 256).reshape(8, 32)
    for jj in range(8):
        expect = (S - Mv) if jj == j else 0.0
        assert np.all(out[jj] == expect), (j, jj, out[jj][:4])


def test_q4k_golden(golden):
    out = orc.dequant_q4k(golden["q4_raw"], int(golden["q4_n"]))
    assert np.array_equal(out.view(np.uint32), golden["q4_deq"].view(np.uint32))


def test_q4k_single_rounding():
    # (d*sc)*q and dmin*m are exact in f32; only the subtraction rounds, so the
    # value equals the f64 result rounded once to f32.
    raw = synth.q4k_weight(11, 256, 64)
    out = orc.dequant_q4k(raw, 256 * 64)
    blocks = raw.reshape(-1, 144)
    d = blocks[:, 0:2].copy().view(np.float16)[:, 0].astype(np.float64)
    dmin = blocks[:, 2:4].copy().view(np.float16)[:, 0].astype(np.float64)
    sc, mn = make_golden.q4k_unpack_scales(blocks[:, 4:16])
    qs = blocks[:, 16:].reshape(-1, 4, 32)
    q = np.stack([qs & 15, qs >> 4], axis=2).reshape(-1, 8, 32).astype(np.float64)
    exact = d[:, None, None] * sc[:, :, None] * q - (dmin[:, None] * mn)[:, :, None]
    assert np.array_equal(out, exact.astype(np.float32).ravel())


# ---------------------------------------------------------------- matvec orders

def test_proj_f32_reference_layout_known_answer(golden):
    # src/lib.rs:120-165: c[j] = sum_i a[i] * b[j*8+i], |err| < 1e-4
    c = orc.proj_f32(golden["mm_a"], golden["mm_b"], 8, 3)
    assert np.all(np.abs(c - golden["mm_expected"]) < 1e-4)
    c2 = orc.proj_f32(golden["mm_a"], golden["mm_b"].reshape(3, 8).T.copy(), 8, 3, row_major=1)
    assert np.array_equal(c, c2)


def test_proj_one_hot_gives_columns():
    k, n = 512, 8
    raw4 = synth.q4k_weight(21, k, n)
    W = orc.dequant_q4k(raw4, k * n).reshape(n, k)
    for j in [0, 31, 32, 63, 64, 255, 256, 511]:
        x = np.zeros(k, np.float32)
        x[j] = 1.0
        assert np.array_equal(orc.proj_q4k(x, raw4, k, n), W[:, j])
    raw8 = synth.q8_0_weight(22, k, n)
    W8 = orc.dequant_to_f32(raw8, orc.Q8_0, k * n).reshape(n, k)
    x = np.zeros(k, np.float32)
    x[100] = 1.0
    assert np.array_equal(orc.proj_q8_0(x, raw8, k, n), W8[:, 100])


def test_proj_golden_f64(golden):
    k, n = int(golden["mv4_k"]), int(golden["mv4_n"])
    raw = golden["q4_raw"][: n * k // 256 * 144]
    y, a = orc.proj_quant_f64(golden["mv4_x"], raw, orc.Q4_K, k, n)
    assert np.allclose(y, golden["mv4_y"], rtol=0, atol=1e-9 * np.max(golden["mv4_abs"]))
    assert np.allclose(a, golden["mv4_abs"], rtol=1e-12)
    k, n = int(golden["mv8_k"]), int(golden["mv8_n"])
    raw = golden["q8_raw"][: n * k // 32 * 34]
    y, a = orc.proj_quant_f64(golden["mv8_x"], raw, orc.Q8_0, k, n)
    assert np.allclose(y, golden["mv8_y"], rtol=0, atol=1e-9 * np.max(golden["mv8_abs"]))


def test_proj_f32_orders_within_tolerance_of_f64():
    k, n = 4096, 64
    raw = synth.q4k_weight(31, k, n)
    x = synth.normal(32, k)
    y32 = orc.proj_q4k(x, raw, k, n)
    y64, a = orc.proj_quant_f64(x, raw, orc.Q4_K, k, n)
    assert np.max(np.abs(y32 - y64) / a) < 1e-5
    raw8 = synth.q8_0_weight(33, k, n)
    y32 = orc.proj_q8_0(x, raw8, k, n)
    y64, a = orc.proj_quant_f64(x, raw8, orc.Q8_0, k, n)
    assert np.max(np.abs(y32 - y64) / a) < 1e-5


def test_proj_linearity_and_expert_offset():
    k, n = 256, 6
    raw = synth.q4k_weight(41, k, 2 * n)
    x1, x2 = synth.normal(42, k), synth.normal(43, k)
    y1, _ = orc.proj_quant_f64(x1, raw, orc.Q4_K, k, n)
    y2, _ = orc.proj_quant_f64(x2, raw, orc.Q4_K, k, n)
    y12, _ = orc.proj_quant_f64(x1 + x2, raw, orc.Q4_K, k, n)
    assert np.allclose(y12, y1 + y2, rtol=1e-6, atol=1e-6)
    # expert_offset = n*k selects the second half of the tensor
    yo = orc.proj_q4k(x1, raw, k, n, expert_offset=n * k)
    yb = orc.proj_q4k(x1, raw[n * k // 256 * 144:], k, n)
    assert np.array_equal(yo, yb)


def test_proj_mt_matches_serial():
    k, n = 4096, 32
    raw = synth.q4k_weight(51, k, n)
    x = synth.normal(52, k)
    assert np.array_equal(orc.proj_q4k(x, raw, k, n), orc.proj_q4k(x, raw, k, n, threads=4))


# ---------------------------------------------------------------- activation

def test_silu_closed_forms():
    g = np.array([0.0, 30.0, -30.0, 1.0, -1.0, 2.5], np.float32)
    up = np.ones_like(g)
    h = orc.silu_mul_f32(g, up)
    h64 = orc.silu_mul_f64(g, up)
    assert h[0] == 0.0 and abs(h[1] - 30.0) < 1e-5 and abs(h[2]) < 1e-10
    # silu(x) - silu(-x) = x
    assert abs((h64[3] - h64[4]) - 1.0) < 1e-15
    assert np.allclose(h, h64, rtol=1e-6, atol=1e-30)


def test_argmax_nan_free_is_last_occurrence_of_max():
    # max_by keeps the last of equal maxima (src/lib.rs:456-464); numpy's argmax
    # over the reversed row finds that index independently
    rng = np.random.default_rng(5)
    for n in (1, 2, 3, 17, 1000, 151936):
        for ties in (False, True):
            v = (rng.integers(-4, 5, n) if ties else rng.standard_normal(n)).astype(np.float32)
            assert orc.argmax(v) == n - 1 - int(np.argmax(v[::-1])), (n, ties)


def test_argmax_closed_forms():
    f = np.float32
    nan, inf = f(np.nan), f(np.inf)
    assert orc.argmax(np.zeros(0, f)) == 0                    # unwrap_or(0)
    assert orc.argmax(np.full(7, 3.0, f)) == 6                # all equal: the last
    assert orc.argmax(np.array([0.0, -0.0], f)) == 1          # -0 == +0: the later
    assert orc.argmax(np.array([-0.0, 0.0, -0.0], f)) == 2
    assert orc.argmax(np.array([1.0, inf, 2.0, inf, 3.0], f)) == 3
    assert orc.argmax(np.array([-inf, -inf], f)) == 1
    # a NaN is taken as Equal: it becomes the best and the next element replaces it
    assert orc.argmax(np.array([5.0, nan, 1.0, 2.0], f)) == 3
    assert orc.argmax(np.array([5.0, 1.0, nan], f)) == 2      # last element NaN
    assert orc.argmax(np.array([nan, 1.0, 0.5], f)) == 1      # NaN first
    assert orc.argmax(np.array([nan, nan, nan], f)) == 2
    assert orc.argmax(np.array([3.0, nan, 9.0, nan, 4.0, 4.0, 1.0], f)) == 5  # after the last NaN only


def test_multithreaded_legs_equal_serial():
    """The benchmark's multi-threaded CPU legs compute the same values as the serial
    restatements: Q8_0 dequant_to_f32 (including a tensor cut short, where the serial
    loop stops at the first short block) and the proj.comp-order f32 matvec."""
    raw = synth.q8_0_weight(0x5EED0101, 1024, 64)
    n = 1024 * 64
    for data in (raw, raw[: 34 * 1000 + 20]):
        a = orc.dequant_to_f32(data, orc.Q8_0, n)
        b = orc.dequant_q8_0_mt(data, n, 4)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    w = synth.normal(0x5EED0102, 512 * 96)
    x = synth.normal(0x5EED0103, 512)
    for rm in (0, 1):
        a = orc.proj_f32(x, w, 512, 96, row_major=rm)
        b = orc.proj_f32(x, w, 512, 96, row_major=rm, threads=4)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
