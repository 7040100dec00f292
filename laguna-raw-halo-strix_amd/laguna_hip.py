"""Python host mirror of laguna-raw's projection API over liblaguna_hip.so (ctypes).

The reference host (Rust) drives Vulkan through GpuBuffer (src/vulkan.rs:341-452)
and the dispatch_* helpers of src/target.rs and src/dflash.rs.  This module keeps
those names and argument orders:

    GpuBuffer.new(ctx, size) / .upload(bytes) / .read_f32(n)   src/vulkan.rs:350-452
    dispatch_proj_quant(ctx, x, w, c, k, n, dtype)              src/target.rs:1086-1099
    dispatch_proj_quant_expert(ctx, x, w, c, k, n, dtype, off)  src/target.rs:1101-1162
    dispatch_proj(ctx, x, w, c, k, n)                           src/dflash.rs:1009-1019
    dispatch_proj_row(ctx, x, w, c, k, n, row_major)            src/dflash.rs:1021-1051
    dispatch_proj_read(ctx, x, w, k, n) -> np.ndarray           src/dflash.rs:1054-1090
    dispatch_activation(ctx, gate, up, h, n)                    src/dflash.rs:1305-1327
    dequant_to_f32(data, dtype, n_elements) -> np.ndarray       src/dflash.rs:331-465

plus the build's additions (fused SiLU down-projection, small-M block product).
The reference panics on failure; here every failing call raises LagunaError
with the library's message.  There is no CPU fallback: if the shared library
is missing, importing works but the first call raises.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblaguna_hip.so")

F32, F16, Q8_0, Q4_K, BF16 = 0, 1, 8, 12, 30
OK, EINVAL, EHIP, ENOMEM, EUNSUPPORTED, EIO, ENODEV = range(7)

# C-ABI symbols declared in include/laguna_hip.h, with ctypes signatures.
_vp, _u32, _u64, _i = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int
SIGNATURES = {
    "lg_last_error": (ctypes.c_char_p, []),
    "lg_version": (ctypes.c_char_p, []),
    "lg_device_count": (_i, [ctypes.POINTER(_i)]),
    "lg_init": (_i, [_i]),
    "lg_set_blocking": (_i, [_i]),
    "lg_buf_alloc": (_i, [ctypes.POINTER(_vp), _u64]),
    "lg_buf_free": (_i, [_vp]),
    "lg_buf_upload": (_i, [_vp, _vp, _u64, _vp]),
    "lg_buf_download": (_i, [_vp, _vp, _u64, _vp]),
    "lg_buf_memset": (_i, [_vp, _i, _u64, _vp]),
    "lg_buf_copy": (_i, [_vp, _vp, _u64, _vp]),
    "lg_stream_create": (_i, [ctypes.POINTER(_vp)]),
    "lg_stream_destroy": (_i, [_vp]),
    "lg_sync": (_i, [_vp]),
    "lg_dequant_to_f32": (_i, [_vp, _u64, _i, _u64, _vp, _vp]),
    "lg_dispatch_proj_quant": (_i, [_vp, _vp, _vp, _u32, _u32, _i, _vp]),
    "lg_dispatch_proj_quant_expert": (_i, [_vp, _vp, _vp, _u32, _u32, _i, _u32, _vp]),
    "lg_dispatch_proj": (_i, [_vp, _vp, _vp, _u32, _u32, _vp]),
    "lg_dispatch_proj_row": (_i, [_vp, _vp, _vp, _u32, _u32, _u32, _vp]),
    "lg_dispatch_proj_read": (_i, [_vp, _vp, _u32, _u32, _vp, _vp]),
    "lg_dispatch_activation": (_i, [_vp, _vp, _vp, _u32, _vp]),
    "lg_dispatch_silu_mul_proj_quant": (_i, [_vp, _vp, _vp, _vp, _u32, _u32, _i, _vp]),
    "lg_dispatch_proj_quant_batch": (_i, [_vp, _i, _vp, _vp, _u32, _u32, _u32, _i, _vp]),
}
# Tuning hooks exported beside the ABI (not part of the drop-in surface).
EXTRA = {
    "lg_set_m1_grid_cap": (_i, [_u32]),
}


class LagunaError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"[status {status}] {msg}")
        self.status = status


_LIB = None


def lib():
    """Load liblaguna_hip.so (raises if it has not been built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise LagunaError(ENODEV, f"{LIB_PATH} is not built; run __graft_entry__.build() or make")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in {**SIGNATURES, **EXTRA}.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def check(status):
    if status != OK:
        raise LagunaError(status, lib().lg_last_error().decode())
    return status


def _ptr(a):
    if a is None:
        return None
    if isinstance(a, GpuBuffer):
        return a.ptr
    if isinstance(a, int):
        return a
    if isinstance(a, np.ndarray):
        return a.ctypes.data
    raise TypeError(type(a))


def device_count():
    n = ctypes.c_int(0)
    check(lib().lg_device_count(ctypes.byref(n)))
    return n.value


class VulkanContext:
    """Per-process device context (VulkanContext::init takes pdevices[0]; so does this)."""

    def __init__(self, device=0, blocking=False):
        check(lib().lg_init(device))
        check(lib().lg_set_blocking(1 if blocking else 0))
        self.device = device
        self.stream = None  # the null stream

    @classmethod
    def init(cls, device=0):
        return cls(device)

    def sync(self):
        check(lib().lg_sync(self.stream))


class GpuBuffer:
    """Device buffer in HBM (the reference's GpuBuffer is host-visible memory)."""

    def __init__(self, ctx, size):
        self.ctx = ctx
        self.size = int(size)
        p = ctypes.c_void_p()
        check(lib().lg_buf_alloc(ctypes.byref(p), self.size))
        self.ptr = p.value

    @classmethod
    def new(cls, ctx, size):
        return cls(ctx, size)

    def upload(self, data, offset=0):
        a = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray)) else data)
        check(lib().lg_buf_upload(self.ptr + offset, a.ctypes.data, a.nbytes, self.ctx.stream))

    def download(self, nbytes=None, offset=0):
        nbytes = self.size - offset if nbytes is None else nbytes
        out = np.empty(nbytes, np.uint8)
        check(lib().lg_buf_download(out.ctypes.data, self.ptr + offset, nbytes, self.ctx.stream))
        return out

    def read_f32(self, n, offset=0):
        return self.download(4 * n, offset).view(np.float32)

    def copy_from(self, other, nbytes=None):
        nbytes = min(self.size, other.size) if nbytes is None else nbytes
        check(lib().lg_buf_copy(self.ptr, other.ptr, nbytes, self.ctx.stream))

    def fill(self, value=0):
        check(lib().lg_buf_memset(self.ptr, value, self.size, self.ctx.stream))

    def free(self):
        if self.ptr:
            lib().lg_buf_free(self.ptr)
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def upload_f32(ctx, data):
    """src/dflash.rs:upload_f32 — new buffer holding the f32 array."""
    a = np.ascontiguousarray(data, np.float32)
    b = GpuBuffer(ctx, max(4, a.nbytes))
    b.upload(a)
    return b


def upload_bytes(ctx, data):
    """Model::upload_tensor_quantized (src/model.rs:174-184): raw bytes, unchanged."""
    a = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray)) else data)
    b = GpuBuffer(ctx, max(16, a.nbytes))
    b.upload(a.view(np.uint8).ravel())
    return b


def dispatch_proj_quant(ctx, x, w, c, k, n, dtype):
    check(lib().lg_dispatch_proj_quant(_ptr(x), _ptr(w), _ptr(c), k, n, dtype, ctx.stream))


def dispatch_proj_quant_expert(ctx, x, w, c, k, n, dtype, expert_offset):
    check(lib().lg_dispatch_proj_quant_expert(_ptr(x), _ptr(w), _ptr(c), k, n, dtype, expert_offset, ctx.stream))


def dispatch_proj(ctx, x, w, c, k, n):
    check(lib().lg_dispatch_proj(_ptr(x), _ptr(w), _ptr(c), k, n, ctx.stream))


def dispatch_proj_row(ctx, x, w, c, k, n, row_major):
    check(lib().lg_dispatch_proj_row(_ptr(x), _ptr(w), _ptr(c), k, n, row_major, ctx.stream))


def dispatch_proj_read(ctx, x, w, k, n):
    out = np.empty(n, np.float32)
    check(lib().lg_dispatch_proj_read(_ptr(x), _ptr(w), k, n, out.ctypes.data, ctx.stream))
    return out


def dispatch_activation(ctx, gate, up, h, n):
    check(lib().lg_dispatch_activation(_ptr(gate), _ptr(up), _ptr(h), n, ctx.stream))


def dispatch_silu_mul_proj_quant(ctx, gate, up, w, c, k, n, dtype):
    check(lib().lg_dispatch_silu_mul_proj_quant(_ptr(gate), _ptr(up), _ptr(w), _ptr(c), k, n, dtype, ctx.stream))


def dispatch_proj_quant_batch(ctx, x, x_dtype, w, c, k, n, m, w_dtype):
    check(lib().lg_dispatch_proj_quant_batch(_ptr(x), x_dtype, _ptr(w), _ptr(c), k, n, m, w_dtype, ctx.stream))


def dequant_to_f32_device(ctx, data_buf, data_len, dtype, n_elements, out_buf):
    check(lib().lg_dequant_to_f32(_ptr(data_buf), data_len, dtype, n_elements, _ptr(out_buf), ctx.stream))


def dequant_to_f32(ctx, data, dtype, n_elements):
    """dequant_to_f32 (src/dflash.rs:331-465) run on the device; returns a host array."""
    a = np.ascontiguousarray(np.frombuffer(data, np.uint8) if isinstance(data, (bytes, bytearray)) else data).view(np.uint8).ravel()
    src = GpuBuffer(ctx, max(16, a.nbytes))
    if a.nbytes:
        src.upload(a)
    out = GpuBuffer(ctx, max(4, 4 * n_elements))
    dequant_to_f32_device(ctx, src, a.nbytes, dtype, n_elements, out)
    r = out.read_f32(n_elements)
    src.free()
    out.free()
    return r
