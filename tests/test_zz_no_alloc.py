"""GPU: the allocation-free small-M product (lg_dispatch_proj_quant_batch_static)
against lg_dispatch_proj_quant_batch, bit for bit, on two calls in a row (the
second smaller), and its size limit.  Called through the C ABI."""
import numpy as np
import pytest

import laguna_hip as lh
import oracle as orc
import synth
from conftest import parity

pytestmark = pytest.mark.gpu


def run(ctx, fn, xb, x_dtype, wb, k, n, m, w_dtype):
    cb = lh.GpuBuffer(ctx, 4 * m * n)
    cb.fill(0xFF)
    lh.check(getattr(lh.lib(), fn)(xb.ptr, x_dtype, wb.ptr, cb.ptr, k, n, m, w_dtype, ctx.stream))
    out = cb.read_f32(m * n).reshape(m, n).copy()
    cb.free()
    return out


def test_static_scratch_equals_workspace_entry_point(ctx):
    # the larger call first, then a smaller one that finds the scratch as the first left it
    for w_dtype, k, n, m, seed in [(lh.Q4_K, 4096, 14336, 16, 0x5EED0008), (lh.Q8_0, 4096, 1024, 5, 0x5EED0009)]:
        print(f"static scratch: w={w_dtype} k={k} n={n} m={m}", flush=True)
        raw = synth.q4k_weight(seed, k, n) if w_dtype == lh.Q4_K else synth.q8_0_weight(seed, k, n)
        x = synth.normal(seed + 0x100, m * k)
        wb, xb = lh.upload_bytes(ctx, raw), lh.upload_f32(ctx, x)
        want = run(ctx, "lg_dispatch_proj_quant_batch", xb, lh.F32, wb, k, n, m, w_dtype)
        got = run(ctx, "lg_dispatch_proj_quant_batch_static", xb, lh.F32, wb, k, n, m, w_dtype)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        y64, a = orc.proj_quant_f64(x.reshape(m, k), raw, w_dtype, k, n)
        parity(got, y64, a)
        wb.free()
        xb.free()


def test_static_scratch_rejects_oversize(ctx):
    # a vocab-sized Q8_0 product at m = 16 is split over 16 k slices: about 155 MB of
    # partial sums, past the 16 MiB scratch
    k, n, m = 4096, 151936, 16
    st = lh.lib().lg_dispatch_proj_quant_batch_static(None, lh.F32, None, None, k, n, m, lh.Q8_0, None)
    assert st == lh.EINVAL and b"scratch" in lh.lib().lg_last_error()
