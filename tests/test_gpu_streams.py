"""GPU: the split-k products keep their partial sums and arrival counters per
stream.  Two products on two streams at the same time must both be right, and
a graph captured from a stream must replay the eager result."""
import ctypes

import numpy as np
import pytest

import laguna_hip as lh
import oracle as orc
import synth
from conftest import parity

pytestmark = pytest.mark.gpu

_HIP = None


def hip():
    global _HIP
    if _HIP is None:
        h = ctypes.CDLL("libamdhip64.so")
        h.hipStreamBeginCapture.argtypes = [ctypes.c_void_p, ctypes.c_int]
        h.hipStreamEndCapture.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
        h.hipGraphInstantiate.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p, ctypes.c_void_p,
                                          ctypes.c_void_p, ctypes.c_size_t]
        h.hipGraphLaunch.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        h.hipGraphExecDestroy.argtypes = [ctypes.c_void_p]
        h.hipGraphDestroy.argtypes = [ctypes.c_void_p]
        _HIP = h
    return _HIP


CAPTURE_THREAD_LOCAL = 1


def product(ctx, x, w, c, k, n, m, w_dtype, stream):
    return lh.lib().lg_dispatch_proj_quant_batch(x.ptr, lh.F32, w.ptr, c.ptr, k, n, m, w_dtype, stream)


def test_two_streams_at_once(ctx):
    """A Q4_K and a Q8_0 block product issued on two streams without a wait between
    them: each equals the same product run alone, bit for bit, and the f64 oracle."""
    m = 16
    cases = [(lh.Q4_K, 4096, 14336, 0x5EED0008), (lh.Q8_0, 4096, 4096, 0x5EED0009)]
    print("two streams: Q4_K 4096x14336 and Q8_0 4096x4096, m=16", flush=True)
    bufs = []
    for dt, k, n, seed in cases:
        raw = synth.q4k_weight(seed, k, n) if dt == lh.Q4_K else synth.q8_0_weight(seed, k, n)
        x = synth.normal(seed + 0x100, m * k)
        bufs.append((dt, k, n, raw, x, lh.upload_bytes(ctx, raw), lh.upload_f32(ctx, x), lh.GpuBuffer(ctx, 4 * m * n)))
    alone = []
    for dt, k, n, raw, x, wb, xb, cb in bufs:
        lh.check(product(ctx, xb, wb, cb, k, n, m, dt, None))
        alone.append(cb.read_f32(m * n).copy())
    s0, s1 = lh.Stream(), lh.Stream()
    for rep in range(3):
        for (dt, k, n, raw, x, wb, xb, cb), s in zip(bufs, (s0, s1)):
            cb.fill(0xFF)
        ctx.sync()
        for (dt, k, n, raw, x, wb, xb, cb), s in zip(bufs, (s0, s1)):
            lh.check(product(ctx, xb, wb, cb, k, n, m, dt, s.ptr))
        s0.sync()
        s1.sync()
        for (dt, k, n, raw, x, wb, xb, cb), ref in zip(bufs, alone):
            got = cb.read_f32(m * n)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"dtype {dt} rep {rep}"
    for (dt, k, n, raw, x, wb, xb, cb), ref in zip(bufs, alone):
        y64, a = orc.proj_quant_f64(x.reshape(m, k), raw, dt, k, n)
        parity(ref.reshape(m, n), y64, a)
    s0.destroy()
    s1.destroy()


def test_capture_needs_a_sized_workspace_then_replays(ctx):
    k, n, m, dt, seed = 4096, 4096, 16, lh.Q4_K, 0x5EED0103
    print(f"capture: Q4_K {k}x{n} m={m}", flush=True)
    raw = synth.q4k_weight(seed, k, n)
    x = synth.normal(seed + 1, m * k)
    wb, xb, cb = lh.upload_bytes(ctx, raw), lh.upload_f32(ctx, x), lh.GpuBuffer(ctx, 4 * m * n)
    ref = lh.GpuBuffer(ctx, 4 * m * n)
    lh.check(product(ctx, xb, wb, ref, k, n, m, dt, None))
    want = ref.read_f32(m * n).copy()
    s = lh.Stream()
    h = hip()
    graph = ctypes.c_void_p()
    # a fresh stream has no workspace: growing it under capture is refused
    assert h.hipStreamBeginCapture(s.ptr, CAPTURE_THREAD_LOCAL) == 0
    st = product(ctx, xb, wb, cb, k, n, m, dt, s.ptr)
    assert h.hipStreamEndCapture(s.ptr, ctypes.byref(graph)) == 0
    assert st == lh.EINVAL and b"captured" in lh.lib().lg_last_error()
    if graph.value:
        h.hipGraphDestroy(graph)
    # one eager call sizes it; the captured call then replays the eager result
    lh.check(product(ctx, xb, wb, cb, k, n, m, dt, s.ptr))
    s.sync()
    assert h.hipStreamBeginCapture(s.ptr, CAPTURE_THREAD_LOCAL) == 0
    st = product(ctx, xb, wb, cb, k, n, m, dt, s.ptr)
    assert h.hipStreamEndCapture(s.ptr, ctypes.byref(graph)) == 0
    lh.check(st)
    ge = ctypes.c_void_p()
    assert h.hipGraphInstantiate(ctypes.byref(ge), graph, None, None, 0) == 0
    for rep in range(3):
        cb.fill(0xFF)
        ctx.sync()
        assert h.hipGraphLaunch(ge, s.ptr) == 0
        s.sync()
        got = cb.read_f32(m * n)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"replay {rep}"
        lh.check(product(ctx, xb, wb, ref, k, n, m, dt, None))  # eager work between replays
        ctx.sync()
    h.hipGraphExecDestroy(ge)
    h.hipGraphDestroy(graph)
    s.destroy()
