"""GPU: the quantized projections at a vocab-sized output (the target's LM head,
project_normalized_hidden, src/target.rs:580-605: dispatch_proj_quant with
n = vocab), for one token and for a 16-token verify block, against the oracle's f64
accumulation."""
import numpy as np
import pytest

import laguna_hip as lh
import oracle as orc
import synth
from conftest import parity

pytestmark = pytest.mark.gpu

K, VOCAB = 4096, 151936


@pytest.fixture(scope="module")
def head(ctx):
    raw = synth.q4k_weight(0x5EED0320, K, VOCAB)  # 350 MB of Q4_K blocks
    return raw, lh.upload_bytes(ctx, raw)


def test_lm_head_one_token(ctx, head):
    raw, wb = head
    print(f"lm head Q4_K {K}->{VOCAB} M=1", flush=True)
    x = synth.normal(0x5EED0321, K)
    cb = lh.GpuBuffer(ctx, 4 * VOCAB)
    lh.dispatch_proj_quant(ctx, lh.upload_f32(ctx, x), wb, cb, K, VOCAB, lh.Q4_K)
    y64, a = orc.proj_quant_f64(x, raw, lh.Q4_K, K, VOCAB)
    parity(cb.read_f32(VOCAB), y64, a, 1e-4)


@pytest.mark.parametrize("x_dtype", [lh.F32, lh.BF16])
def test_lm_head_verify_block(ctx, head, x_dtype):
    # 16 tokens through the small-M kernel, every row against the f64 reference
    raw, wb = head
    m = 16
    print(f"lm head Q4_K {K}->{VOCAB} M={m} x={'f32' if x_dtype == lh.F32 else 'bf16'}", flush=True)
    x = synth.normal(0x5EED0322, m * K).reshape(m, K)
    if x_dtype == lh.BF16:
        u = x.view(np.uint32).astype(np.uint64)
        xin = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        x = (xin.astype(np.uint32) << 16).view(np.float32)
    else:
        xin = x
    xb = lh.upload_bytes(ctx, np.ascontiguousarray(xin).view(np.uint8).ravel())
    cb = lh.GpuBuffer(ctx, 4 * m * VOCAB)
    lh.dispatch_proj_quant_batch(ctx, xb, x_dtype, wb, cb, K, VOCAB, m, lh.Q4_K)
    c = cb.read_f32(m * VOCAB).reshape(m, VOCAB)
    y64, a = orc.proj_quant_f64(np.ascontiguousarray(x), raw, lh.Q4_K, K, VOCAB)
    parity(c, y64, a, 1e-4)


@pytest.mark.parametrize("m,n", [(20, VOCAB), (16, VOCAB - 2), (32, VOCAB)])
def test_lm_head_block_finishing_launch(ctx, head, m, n):
    # Vocab-sized blocks are split over k into more than 4,096 workgroups, so their
    # slices only store partial sums and a second launch adds them: 20 and 32 rows
    # are two token tiles (the second partial at m = 20), n = VOCAB - 2 is not a
    # multiple of 4 (element-wise loads and stores).  Every row against f64, and two
    # calls bit for bit.
    raw, wb = head
    print(f"lm head Q4_K {K}->{n} M={m} (finishing launch)", flush=True)
    x = synth.normal(0x5EED0323 + m, m * K).reshape(m, K)
    xb = lh.upload_f32(ctx, x.ravel())
    cb = lh.GpuBuffer(ctx, 4 * m * n)
    lh.dispatch_proj_quant_batch(ctx, xb, lh.F32, wb, cb, K, n, m, lh.Q4_K)
    c = cb.read_f32(m * n).reshape(m, n)
    lh.dispatch_proj_quant_batch(ctx, xb, lh.F32, wb, cb, K, n, m, lh.Q4_K)
    assert np.array_equal(cb.read_f32(m * n).reshape(m, n).view(np.uint32), c.view(np.uint32))
    y64, a = orc.proj_quant_f64(x, raw[: n * (raw.size // VOCAB)], lh.Q4_K, K, n)  # the first n rows
    parity(c, y64, a, 1e-4)
