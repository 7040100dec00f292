"""GPU: lg_dequant_to_f32 against the oracle, bit for bit."""
import numpy as np
import pytest

import laguna_hip as lh
import oracle as orc
import synth

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    """Bit-identical, except that NaN equals NaN (payload rules differ between
    the CPU and the GPU once a NaN goes through arithmetic)."""
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return np.array_equal(a.view(np.uint32)[~nan], b.view(np.uint32)[~nan]) and np.array_equal(np.isnan(a), np.isnan(b))


def test_q4k_full_config_tensor(ctx):
    print("dequant Q4_K 4096x14336 seed 0x5EED0003", flush=True)
    raw = synth.q4k_weight(0x5EED0003, 4096, 14336)
    n = 4096 * 14336
    got = lh.dequant_to_f32(ctx, raw, lh.Q4_K, n)
    assert np.array_equal(got.view(np.uint32), orc.dequant_q4k(raw, n).view(np.uint32))


def test_q8_0_full_config_tensor(ctx):
    print("dequant Q8_0 4096x4096 seed 0x5EED0001", flush=True)
    raw = synth.q8_0_weight(0x5EED0001, 4096, 4096)
    n = 4096 * 4096
    got = lh.dequant_to_f32(ctx, raw, lh.Q8_0, n)
    assert np.array_equal(got.view(np.uint32), orc.dequant_to_f32(raw, orc.Q8_0, n).view(np.uint32))


def test_golden_blocks_with_special_scales(ctx, golden):
    # subnormal-quirk d/dmin, +-0, max f16, all-63 scales, ragged n
    for dtype, raw, n in [(lh.Q4_K, golden["q4_raw"], int(golden["q4_n"])),
                          (lh.Q8_0, golden["q8_raw"], int(golden["q8_n"]))]:
        print("dequant golden", dtype, n, flush=True)
        got = lh.dequant_to_f32(ctx, raw, dtype, n)
        want = golden["q4_deq"] if dtype == lh.Q4_K else golden["q8_deq"]
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("dtype", [lh.Q4_K, lh.Q8_0])
def test_truncated_data_and_ragged_tail(ctx, dtype):
    raw = synth.q4k_weight(3, 256, 8) if dtype == lh.Q4_K else synth.q8_0_weight(3, 32, 16)
    bs = 144 if dtype == lh.Q4_K else 34
    for n, keep in [(2048, raw.size), (2000, raw.size), (2048, 5 * bs + 7), (100, raw.size), (1, raw.size)]:
        print("dequant truncated", dtype, n, keep, flush=True)
        got = lh.dequant_to_f32(ctx, raw[:keep], dtype, n)
        want = (orc.dequant_q4k(raw[:keep], n) if dtype == lh.Q4_K else orc.dequant_to_f32(raw[:keep], orc.Q8_0, n))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q4k_unaligned_base(ctx):
    # a tensor that does not start on a 16-byte boundary takes the byte-addressed kernel
    raw = synth.q4k_weight(9, 256, 40)
    buf = lh.GpuBuffer(ctx, raw.size + 16)
    buf.upload(raw, offset=3)
    out = lh.GpuBuffer(ctx, 4 * raw.size // 144 * 256)
    n = raw.size // 144 * 256
    print("dequant Q4_K unaligned base", flush=True)
    lh.dequant_to_f32_device(ctx, buf.ptr + 3, raw.size, lh.Q4_K, n, out)
    assert np.array_equal(out.read_f32(n).view(np.uint32), orc.dequant_q4k(raw, n).view(np.uint32))


def test_nonfinite_scales(ctx):
    raw = synth.q4k_weight(4, 256, 4).reshape(-1, 144).copy()
    raw[0, 0:2] = np.array([0x7C00], np.uint16).view(np.uint8)   # d = +inf
    raw[1, 2:4] = np.array([0x7E00], np.uint16).view(np.uint8)   # dmin = NaN
    raw[2, 0:2] = np.array([0xFC01], np.uint16).view(np.uint8)   # d = signalling NaN
    raw = raw.ravel()
    print("dequant Q4_K non-finite scales", flush=True)
    got = lh.dequant_to_f32(ctx, raw, lh.Q4_K, 1024)
    assert same_bits(got, orc.dequant_q4k(raw, 1024))


@pytest.mark.parametrize("dtype", [lh.F32, lh.F16, lh.BF16])
def test_elementwise_branches(ctx, dtype):
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    data = codes.view(np.uint8) if dtype != lh.F32 else synth.normal(5, 4096).view(np.uint8)
    n = data.size // (4 if dtype == lh.F32 else 2) + 3  # 3 past the data: zeros
    print("dequant elementwise", dtype, flush=True)
    got = lh.dequant_to_f32(ctx, data, dtype, n)
    assert np.array_equal(got.view(np.uint32), orc.dequant_to_f32(data, dtype, n).view(np.uint32))


def test_unsupported_type_gives_zeros(ctx):
    # src/dflash.rs:463 (and its unit test :1368-1373)
    print("dequant unsupported", flush=True)
    got = lh.dequant_to_f32(ctx, np.full(64, 0x55, np.uint8), 4, 16)
    assert got.shape == (16,) and np.all(got == 0)
