"""ctypes view of the CPU oracle (liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Only the tests, the smoke check and the benchmark's CPU-baseline leg use this
module, and only as the checker.  Each wrapper names the reference lines its C
function restates (see oracle.h for how each one is pinned).
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

F32, F16, Q8_0, Q4_K, BF16 = 0, 1, 8, 12, 30

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_u8p = ctypes.POINTER(ctypes.c_uint8)


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"oracle not built: {path} (run `make -C oracle`)")
        L = ctypes.CDLL(path)
        L.orc_half_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_half_to_f32.restype = ctypes.c_float
        L.orc_dequant_to_f32.argtypes = [_u8p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_size_t, _f32p]
        L.orc_q4k_value.argtypes = [_u8p, ctypes.c_uint64]
        L.orc_q4k_value.restype = ctypes.c_float
        L.orc_q8_0_value.argtypes = [_u8p, ctypes.c_uint64]
        L.orc_q8_0_value.restype = ctypes.c_float
        L.orc_dequant_q4k.argtypes = [_u8p, ctypes.c_size_t, ctypes.c_size_t, _f32p]
        L.orc_proj_f32.argtypes = [_f32p, _f32p, _f32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
        L.orc_proj_f32_mt.argtypes = [_f32p, _f32p, _f32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                      ctypes.c_int]
        L.orc_dequant_q8_0_mt.argtypes = [_u8p, ctypes.c_size_t, ctypes.c_size_t, _f32p, ctypes.c_int]
        L.orc_proj_q8_0.argtypes = [_f32p, _u8p, _f32p, ctypes.c_uint32, ctypes.c_uint32]
        L.orc_proj_q4k.argtypes = [_f32p, _u8p, _f32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]
        L.orc_proj_q4k_mt.argtypes = [_f32p, _u8p, _f32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int]
        L.orc_proj_q8_0_mt.argtypes = [_f32p, _u8p, _f32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int]
        L.orc_proj_quant_f64.argtypes = [_f32p, ctypes.c_uint32, _u8p, ctypes.c_uint32, ctypes.c_uint32,
                                         ctypes.c_uint32, ctypes.c_uint64, _f64p, _f64p]
        L.orc_proj_quant_f64x.argtypes = [_f64p, _u8p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                          _f64p, _f64p]
        L.orc_silu_mul_f32.argtypes = [_f32p, _f32p, _f32p, ctypes.c_uint32]
        L.orc_silu_mul_f64.argtypes = [_f32p, _f32p, _f64p, ctypes.c_uint32]
        L.orc_argmax_f32.argtypes = [_f32p, ctypes.c_size_t]
        L.orc_argmax_f32.restype = ctypes.c_size_t
        _LIB = L
    return _LIB


def _p(a, t):
    return a.ctypes.data_as(t)


def _u8(b):
    return np.ascontiguousarray(np.frombuffer(b, np.uint8) if isinstance(b, (bytes, bytearray)) else b, np.uint8)


def half_to_f32(h):
    """src/dflash.rs:314-329"""
    return lib().orc_half_to_f32(int(h))


def dequant_to_f32(data, dtype, n):
    """src/dflash.rs:331-465 (its Q4_K branch is the legacy non-ggml decode)."""
    d = _u8(data)
    out = np.empty(n, np.float32)
    lib().orc_dequant_to_f32(_p(d, _u8p), d.size, dtype, n, _p(out, _f32p))
    return out


def dequant_q4k(data, n):
    """ggml Q4_K decode of kernels/proj_q4k.comp:46-87 over a whole tensor."""
    d = _u8(data)
    out = np.empty(n, np.float32)
    lib().orc_dequant_q4k(_p(d, _u8p), d.size, n, _p(out, _f32p))
    return out


def dequant(data, dtype, n):
    """The decode each quantized projection applies: ggml Q4_K (proj_q4k.comp)
    or Q8_0 (dequant_to_f32 / proj_q8_0.comp, identical)."""
    if dtype == Q4_K:
        return dequant_q4k(data, n)
    return dequant_to_f32(data, dtype, n)


def proj_f32(x, w, k, n, row_major=0, threads=1):
    """kernels/proj.comp:23-33"""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    c = np.empty(n, np.float32)
    if threads > 1:
        lib().orc_proj_f32_mt(_p(x, _f32p), _p(w, _f32p), _p(c, _f32p), k, n, row_major, threads)
    else:
        lib().orc_proj_f32(_p(x, _f32p), _p(w, _f32p), _p(c, _f32p), k, n, row_major)
    return c


def dequant_q8_0_mt(data, n, threads):
    """The Q8_0 arm of dequant_to_f32 (src/dflash.rs:379-397) on `threads` threads."""
    d = _u8(data)
    out = np.empty(n, np.float32)
    lib().orc_dequant_q8_0_mt(_p(d, _u8p), d.size, n, _p(out, _f32p), threads)
    return out


def proj_q8_0(x, w, k, n, threads=1):
    """kernels/proj_q8_0.comp:47-66"""
    x = np.ascontiguousarray(x, np.float32)
    w = _u8(w)
    c = np.empty(n, np.float32)
    if threads > 1:
        lib().orc_proj_q8_0_mt(_p(x, _f32p), _p(w, _u8p), _p(c, _f32p), k, n, threads)
    else:
        lib().orc_proj_q8_0(_p(x, _f32p), _p(w, _u8p), _p(c, _f32p), k, n)
    return c


def proj_q4k(x, w, k, n, expert_offset=0, threads=1):
    """kernels/proj_q4k.comp:60-92"""
    x = np.ascontiguousarray(x, np.float32)
    w = _u8(w)
    c = np.empty(n, np.float32)
    if threads > 1:
        assert expert_offset == 0
        lib().orc_proj_q4k_mt(_p(x, _f32p), _p(w, _u8p), _p(c, _f32p), k, n, threads)
    else:
        lib().orc_proj_q4k(_p(x, _f32p), _p(w, _u8p), _p(c, _f32p), k, n, expert_offset)
    return c


def proj_quant_f64(x, w, dtype, k, n, elem_offset=0):
    """f64 accumulation of the exact dequantized weights; x is [m, k] or [k].
    Returns (y, absdot) shaped [m, n] (or [n])."""
    x = np.ascontiguousarray(x, np.float32)
    squeeze = x.ndim == 1
    x2 = x.reshape(-1, k)
    m = x2.shape[0]
    w = _u8(w) if dtype != F32 else np.ascontiguousarray(w, np.float32).view(np.uint8).ravel()
    y = np.empty((m, n), np.float64)
    a = np.empty((m, n), np.float64)
    lib().orc_proj_quant_f64(_p(x2, _f32p), m, _p(w, _u8p), dtype, k, n, elem_offset, _p(y, _f64p), _p(a, _f64p))
    if squeeze:
        return y[0], a[0]
    return y, a


def proj_quant_f64x(x64, w, dtype, k, n):
    """f64 accumulation for a float64 activation vector."""
    x64 = np.ascontiguousarray(x64, np.float64)
    w = _u8(w)
    y = np.empty(n, np.float64)
    a = np.empty(n, np.float64)
    lib().orc_proj_quant_f64x(_p(x64, _f64p), _p(w, _u8p), dtype, k, n, _p(y, _f64p), _p(a, _f64p))
    return y, a


def silu_mul_f32(g, up):
    """kernels/activation.comp:21-28"""
    g = np.ascontiguousarray(g, np.float32)
    up = np.ascontiguousarray(up, np.float32)
    h = np.empty(g.size, np.float32)
    lib().orc_silu_mul_f32(_p(g, _f32p), _p(up, _f32p), _p(h, _f32p), g.size)
    return h


def silu_mul_f64(g, up):
    g = np.ascontiguousarray(g, np.float32)
    up = np.ascontiguousarray(up, np.float32)
    h = np.empty(g.size, np.float64)
    lib().orc_silu_mul_f64(_p(g, _f32p), _p(up, _f32p), _p(h, _f64p), g.size)
    return h


def argmax(logits):
    """src/lib.rs:456-464 (the reference's argmax over one row of logits)"""
    v = np.ascontiguousarray(logits, np.float32).ravel()
    return int(lib().orc_argmax_f32(_p(v, _f32p), v.size))
