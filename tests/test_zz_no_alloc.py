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
    # one 256-element chunk per k slice (a launch-shape override) at m = 32: 16 slices of
    # 32 x 14336 partial sums (about 29 MB), past the 16 MiB scratch
    k, n, m = 4096, 14336, 32
    lh.check(lh.lib().lg_set_batch_shape(1, 0))
    try:
        need = lh.lib().lg_proj_quant_batch_ws_bytes(k, n, m, lh.Q4_K)
        assert need > lh.STATIC_SCRATCH_BYTES
        st = lh.lib().lg_dispatch_proj_quant_batch_static(None, lh.F32, None, None, k, n, m, lh.Q4_K, None)
        assert st == lh.EINVAL and b"scratch" in lh.lib().lg_last_error()
    finally:
        lh.check(lh.lib().lg_set_batch_shape(0, 0))


def test_static_scratch_several_tile_pairs(ctx):
    # m = 40: three token tiles in two launches that reuse the counters and partial sums
    k, n, m = 2048, 700, 40
    print(f"static scratch: m={m} k={k} n={n}", flush=True)
    raw = synth.q4k_weight(0x5EED0021, k, n)
    x = synth.normal(0x5EED0022, m * k)
    wb, xb = lh.upload_bytes(ctx, raw), lh.upload_f32(ctx, x)
    want = run(ctx, "lg_dispatch_proj_quant_batch", xb, lh.F32, wb, k, n, m, lh.Q4_K)
    got = run(ctx, "lg_dispatch_proj_quant_batch_static", xb, lh.F32, wb, k, n, m, lh.Q4_K)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    y64, a = orc.proj_quant_f64(x.reshape(m, k), raw, lh.Q4_K, k, n)
    parity(got, y64, a)
    wb.free()
    xb.free()


def test_static_scratch_limit(ctx):
    # with one chunk per k slice (a launch-shape override), the largest k (n = 1024,
    # m = 32) whose partial sums fit the scratch runs and equals the workspace entry
    # point; the next multiple of 256 is refused
    n, m = 1024, 32
    L = lh.lib()
    lh.check(L.lg_set_batch_shape(1, 0))
    try:
        k = 256
        while L.lg_proj_quant_batch_ws_bytes(k + 256, n, m, lh.Q4_K) <= lh.STATIC_SCRATCH_BYTES:
            k += 256
        print(f"static scratch limit: k={k} fits, k={k + 256} does not", flush=True)
        raw = synth.q4k_weight(0x5EED0023, k + 256, n)
        x = synth.normal(0x5EED0024, m * (k + 256))
        wb = lh.upload_bytes(ctx, raw)
        xb = lh.upload_f32(ctx, x)
        cb = lh.GpuBuffer(ctx, 4 * m * n)
        st = L.lg_dispatch_proj_quant_batch_static(xb.ptr, lh.F32, wb.ptr, cb.ptr, k + 256, n, m, lh.Q4_K,
                                                   ctx.stream)
        assert st == lh.EINVAL and b"scratch" in L.lg_last_error()
        cb.free()
        raw = synth.q4k_weight(0x5EED0023, k, n)
        wb.free()
        wb = lh.upload_bytes(ctx, raw)
        xs = x[: m * k]
        xb.free()
        xb = lh.upload_f32(ctx, xs)
        want = run(ctx, "lg_dispatch_proj_quant_batch", xb, lh.F32, wb, k, n, m, lh.Q4_K)
        got = run(ctx, "lg_dispatch_proj_quant_batch_static", xb, lh.F32, wb, k, n, m, lh.Q4_K)
    finally:
        lh.check(L.lg_set_batch_shape(0, 0))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    y64, a = orc.proj_quant_f64(xs.reshape(m, k), raw, lh.Q4_K, k, n)
    parity(got, y64, a)
    wb.free()
    xb.free()


def test_static_scratch_graph_replays(ctx):
    # a static call captured into a HIP graph on its own stream, replayed three times
    # with eager calls of another shape on the same scratch between the replays: every
    # replay equals the eager result
    import ctypes

    h = ctypes.CDLL("libamdhip64.so")
    vp, pvp = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)
    h.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
    h.hipStreamEndCapture.argtypes = [vp, pvp]
    h.hipGraphInstantiate.argtypes = [pvp, vp, vp, vp, ctypes.c_size_t]
    h.hipGraphLaunch.argtypes = [vp, vp]
    h.hipGraphExecDestroy.argtypes = [vp]
    h.hipGraphDestroy.argtypes = [vp]
    L = lh.lib()
    k, n, m = 4096, 1536, 16
    raw = synth.q4k_weight(0x5EED0025, k, n)
    x = synth.normal(0x5EED0026, m * k)
    wb, xb = lh.upload_bytes(ctx, raw), lh.upload_f32(ctx, x)
    want = run(ctx, "lg_dispatch_proj_quant_batch", xb, lh.F32, wb, k, n, m, lh.Q4_K)
    raw2 = synth.q8_0_weight(0x5EED0027, 2048, 700)
    x2 = synth.normal(0x5EED0028, 5 * 2048)
    wb2, xb2 = lh.upload_bytes(ctx, raw2), lh.upload_f32(ctx, x2)
    want2 = run(ctx, "lg_dispatch_proj_quant_batch", xb2, lh.F32, wb2, 2048, 700, 5, lh.Q8_0)
    st = lh.Stream()
    cb = lh.GpuBuffer(ctx, 4 * m * n)
    g, ge = ctypes.c_void_p(), ctypes.c_void_p()
    print("static scratch: capture", flush=True)
    assert h.hipStreamBeginCapture(st.ptr, 1) == 0
    try:
        rc = L.lg_dispatch_proj_quant_batch_static(xb.ptr, lh.F32, wb.ptr, cb.ptr, k, n, m, lh.Q4_K, st.ptr)
    finally:
        assert h.hipStreamEndCapture(st.ptr, ctypes.byref(g)) == 0
    lh.check(rc)
    assert h.hipGraphInstantiate(ctypes.byref(ge), g, None, None, 0) == 0
    try:
        for rep in range(3):
            print(f"static scratch: replay {rep}", flush=True)
            cb.fill(0xFF)
            ctx.sync()
            assert h.hipGraphLaunch(ge, st.ptr) == 0
            st.sync()
            got = cb.read_f32(m * n).reshape(m, n)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
            got2 = run(ctx, "lg_dispatch_proj_quant_batch_static", xb2, lh.F32, wb2, 2048, 700, 5, lh.Q8_0)
            assert np.array_equal(got2.view(np.uint32), want2.view(np.uint32))
    finally:
        h.hipGraphExecDestroy(ge)
        h.hipGraphDestroy(g)
        st.destroy()
    for b in (wb, xb, wb2, xb2, cb):
        b.free()
