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
Q8_0_T16, Q4_K_T16 = 1008, 1012  # Q8_0 / Q4_K repacked into 16-row tiles by repack_tiled (not GGUF types)
TILED = {Q4_K: Q4_K_T16, Q8_0: Q8_0_T16}
OK, EINVAL, EHIP, ENOMEM, EUNSUPPORTED, EIO, ENODEV, ENOTFOUND = range(8)
STATIC_SCRATCH_BYTES = (16 << 20) + 65536  # the allocation-free product's device array

# C-ABI symbols declared in include/laguna_hip.h, with ctypes signatures.
_vp, _u32, _u64, _i, _f = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int, ctypes.c_float
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
    "lg_dispatch_proj_quant_batch_static": (_i, [_vp, _i, _vp, _vp, _u32, _u32, _u32, _i, _vp]),
    "lg_proj_quant_batch_ws_bytes": (_u64, [_u32, _u32, _u32, _i]),
    "lg_dispatch_silu_gate_up_batch": (_i, [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _i, _vp]),
    "lg_dispatch_argmax": (_i, [_vp, _u32, _u32, _u64, _vp, _vp]),
    "lg_tiled_bytes": (_u64, [_i, _u32, _u32]),
    "lg_repack_tiled": (_i, [_vp, _i, _u32, _u32, _vp, _vp]),
    "lg_dispatch_rmsnorm": (_i, [_vp, _vp, _vp, _u32, _u32, _f, _vp]),
    "lg_dispatch_enc_aux_norm": (_i, [_vp, _vp, _vp, _u32, _u32, _u32, _vp]),
    "lg_dispatch_qk_norm_rope": (_i, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _f, _vp]),
    "lg_dispatch_mha_attn": (_i, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _i, _vp]),
    "lg_dispatch_gate_mul": (_i, [_vp, _vp, _vp, _u32, _u32, _u32, _vp]),
    "lg_dispatch_softplus_gate_mul": (_i, [_vp, _vp, _vp, _u32, _u32, _u32, _vp]),
    "lg_dispatch_add": (_i, [_vp, _vp, _vp, _u32, _vp]),
    "lg_dispatch_gate_attn": (_i, [_vp, _vp, _vp, _u32, _u32, _vp]),
    "lg_target_forward_token": (_i, [_vp, _vp, _vp, _u32, _vp, ctypes.POINTER(_u32), _vp, _vp, _vp, _vp]),
    "lg_target_capture_count": (_i, [_u32, _vp, _u32, ctypes.POINTER(_u32)]),
    "lg_dflash_encode": (_i, [_vp, _vp, _u32, _vp, _vp]),
    "lg_dflash_forward_block": (_i, [_vp, _vp, _vp, _u32, _u32, _vp, _vp]),
    "lg_dflash_graph_create": (_i, [_vp, _vp, _vp, _u32, _u32, _vp, _vp, ctypes.POINTER(_vp)]),
    "lg_dflash_graph_launch": (_i, [_vp, _vp]),
    "lg_dflash_graph_destroy": (_i, [_vp]),
    "lg_gguf_type_info": (_i, [_i, ctypes.POINTER(_u32), ctypes.POINTER(_u32), ctypes.POINTER(_i),
                               ctypes.POINTER(_i)]),
    "lg_gguf_open": (_i, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "lg_gguf_close": (_i, [_vp]),
    "lg_gguf_header": (_i, [_vp, ctypes.POINTER(_u32), ctypes.POINTER(_u64), ctypes.POINTER(_u64),
                            ctypes.POINTER(_u64)]),
    "lg_gguf_metadata": (_i, [_vp, _vp]),
    "lg_gguf_tensor_info": (_i, [_vp, _u64, _vp]),
    "lg_gguf_find_tensor": (_i, [_vp, ctypes.c_char_p, ctypes.POINTER(_u64)]),
    "lg_gguf_read_tensor": (_i, [_vp, _u64, _vp, _u64]),
    "lg_gguf_upload_tensor": (_i, [_vp, _u64, _vp, _u64, _vp]),
    "lg_gguf_field_count": (_i, [_vp, ctypes.POINTER(_u64)]),
    "lg_gguf_field": (_i, [_vp, _u64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_i), ctypes.POINTER(_u64),
                           ctypes.POINTER(_i)]),
    "lg_gguf_get_u64": (_i, [_vp, _u64, _u64, ctypes.POINTER(_u64)]),
    "lg_gguf_get_i64": (_i, [_vp, _u64, _u64, ctypes.POINTER(ctypes.c_int64)]),
    "lg_gguf_get_f32": (_i, [_vp, _u64, _u64, ctypes.POINTER(_f)]),
    "lg_gguf_get_f64": (_i, [_vp, _u64, _u64, ctypes.POINTER(ctypes.c_double)]),
    "lg_gguf_get_bool": (_i, [_vp, _u64, _u64, ctypes.POINTER(_i)]),
    "lg_gguf_get_str": (_i, [_vp, _u64, _u64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_u64)]),
    "lg_gguf_find_field": (_i, [_vp, ctypes.c_char_p, ctypes.POINTER(_u64)]),
    # launch-shape tuning hooks (no counterpart in the reference)
    "lg_set_m1_grid_cap": (_i, [_u32]),
    "lg_set_m1_split": (_i, [_u32]),
    "lg_set_m1_kernel": (_i, [_u32]),
    "lg_set_fold_norms": (_i, [_u32]),
    "lg_set_batch_shape": (_i, [_u32, _u32]),
    # ceiling kernels for measurement (no counterpart in the reference)
    "lg_bench_empty": (_i, [_u32, _vp]),
    "lg_bench_read": (_i, [_vp, _u64, _vp]),
    "lg_bench_read_shape": (_i, [_vp, _u64, _u32, _u32, _u32, _u32, _vp]),
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
        for name, (res, args) in SIGNATURES.items():
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


def dispatch_silu_gate_up_batch(ctx, x, w_gate, w_up, h, u_scratch, k, n, m, w_dtype):
    """h = silu(x W_gate^T) * (x W_up^T) for m rows of f32 x (src/dflash.rs:963-965)."""
    check(lib().lg_dispatch_silu_gate_up_batch(_ptr(x), _ptr(w_gate), _ptr(w_up), _ptr(h), _ptr(u_scratch), k, n, m,
                                               w_dtype, ctx.stream))


def repack_tiled(ctx, w, dtype, k, n):
    """The k x n Q4_K or Q8_0 tensor in `w` (raw GGUF blocks on the device) repacked
    into a new buffer of 16-row tiles (type TILED[dtype]), for the small-M products."""
    out = GpuBuffer(ctx, lib().lg_tiled_bytes(dtype, k, n))
    check(lib().lg_repack_tiled(_ptr(w), dtype, k, n, _ptr(out), ctx.stream))
    return out


def dispatch_argmax(ctx, logits, n, rows=1, ld=None, out=None):
    """argmax (src/lib.rs:456-464) of each of `rows` rows of n logits on the device
    (row r at float offset r * ld).  Returns the indices as int64 (and leaves them
    in `out`, a GpuBuffer of 4 * rows bytes, when given)."""
    ld = n if ld is None else ld
    ob = out if out is not None else GpuBuffer(ctx, 4 * max(rows, 1))
    try:
        check(lib().lg_dispatch_argmax(_ptr(logits), n, rows, ld, _ptr(ob), ctx.stream))
        return np.frombuffer(ob.download(4 * rows), np.uint32).astype(np.int64)
    finally:
        if out is None:
            ob.free()


def verify_step(ctx, draft_logits, target_logits, n_vocab):
    """The decision of one run_target_dflash_verify step (src/lib.rs:497-503), taken
    on the device logits of the draft (after project_normalized_hidden) and of the
    target: both argmaxes, accepted when they agree, and the next token is the
    draft's when accepted and the target's otherwise.
    Returns (next_token, accepted, draft_token, target_token)."""
    d = int(dispatch_argmax(ctx, draft_logits, n_vocab)[0])
    t = int(dispatch_argmax(ctx, target_logits, n_vocab)[0])
    return (d if d == t else t), d == t, d, t


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


# ---- streams ------------------------------------------------------------------------


class Stream:
    """A created (non-null) HIP stream: HIP graph capture needs one."""

    def __init__(self):
        p = ctypes.c_void_p()
        check(lib().lg_stream_create(ctypes.byref(p)))
        self.ptr = p.value

    def sync(self):
        check(lib().lg_sync(self.ptr))

    def destroy(self):
        if self.ptr:
            lib().lg_stream_destroy(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


def _stream(ctx, stream):
    return stream.ptr if isinstance(stream, Stream) else (ctx.stream if stream is None else stream)


# ---- DFlash glue (src/dflash.rs dispatch_* helpers; one row each, as the reference) ----

RMS_EPS = 1e-5   # src/dflash.rs:987
QK_EPS = 1e-6    # src/dflash.rs:1105


def dispatch_rmsnorm(ctx, w, x, out, n, rows=1, eps=RMS_EPS):
    """dispatch_rmsnorm(ctx, shader, w, x, out, n) (src/dflash.rs:979-1007)."""
    check(lib().lg_dispatch_rmsnorm(_ptr(w), _ptr(x), _ptr(out), n, rows, eps, ctx.stream))


def dispatch_enc_aux_norm(ctx, x, aux_norm_w, out, n_feat, n_aux, n_total):
    """dispatch_enc_aux_norm (src/dflash.rs:1200-1233); n_total = n_aux * n_feat per token
    (eps 1e-5, as the reference)."""
    check(lib().lg_dispatch_enc_aux_norm(_ptr(x), _ptr(aux_norm_w), _ptr(out), n_feat, n_aux, n_total, ctx.stream))


def dispatch_qk_norm_rope(ctx, x, norm_w, freq, out, n_heads, head_dim, rope_dim, pos, rows=1, eps=QK_EPS):
    """dispatch_qk_norm_rope (src/dflash.rs:1093-1129)."""
    check(lib().lg_dispatch_qk_norm_rope(_ptr(x), _ptr(norm_w), _ptr(freq), _ptr(out), n_heads, head_dim, rope_dim,
                                         pos, rows, eps, ctx.stream))


def dispatch_mha_attn_seq(ctx, q_normed, k_seq, v_seq, out, n_q_heads, n_kv_heads, head_dim, seq_len, q_pos,
                          rows=1, causal=1):
    """dispatch_mha_attn_seq (src/dflash.rs:1160-1199); the reference always passes causal = 1."""
    check(lib().lg_dispatch_mha_attn(_ptr(q_normed), _ptr(k_seq), _ptr(v_seq), _ptr(out), n_q_heads, n_kv_heads,
                                     head_dim, seq_len, q_pos, rows, causal, ctx.stream))


def dispatch_gate_mul(ctx, attn_out, v_rep, gate, n_hd, n_heads, head_dim):
    """dispatch_gate_mul(ctx, shader, attn_out, v_rep, gate, n_hd, n_heads, head_dim)
    (src/dflash.rs:1236-1266): attn_out[i] = v_rep[i] * gate[i / head_dim], i < n_hd."""
    check(lib().lg_dispatch_gate_mul(_ptr(attn_out), _ptr(v_rep), _ptr(gate), n_hd, n_heads, head_dim, ctx.stream))


def dispatch_softplus_gate_mul(ctx, attn_out, v_rep, gate, n_hd, n_heads, head_dim):
    """src/dflash.rs:956-959 on the device: gate -> softplus (threshold 20), then gate_mul."""
    check(lib().lg_dispatch_softplus_gate_mul(_ptr(attn_out), _ptr(v_rep), _ptr(gate), n_hd, n_heads, head_dim,
                                              ctx.stream))


def dispatch_gate_attn(ctx, attn_out, gate, result, n_heads, head_dim):
    """dispatch_gate_attn (src/target.rs:992-1020): result = attn_out * log(1 + exp(gate[head]))."""
    check(lib().lg_dispatch_gate_attn(_ptr(attn_out), _ptr(gate), _ptr(result), n_heads, head_dim, ctx.stream))


def dispatch_add(ctx, a, b, out, n):
    """dispatch_add (src/dflash.rs:1281-1303)."""
    check(lib().lg_dispatch_add(_ptr(a), _ptr(b), _ptr(out), n, ctx.stream))


MOE_TENSORS = ("ffn_gate_inp", "ffn_gate_exps", "ffn_up_exps", "ffn_down_exps", "ffn_gate_shexp", "ffn_up_shexp",
               "ffn_down_shexp")
F16_SAFE = np.float32(32768.0)             # src/target.rs:699
MOE_NORM_MIN = np.float32(6.103515625e-5)  # src/target.rs:666


class MoeFfnWeights:
    """The MoE FFN tensors of a TargetLayer (src/target.rs:181-235): each name of
    MOE_TENSORS is a (GpuBuffer, dtype) pair of raw blocks (the experts' gate, up and
    down weights stacked expert after expert), exp_probs_b a GpuBuffer of n_expert f32."""

    def __init__(self, exp_probs_b, **tensors):
        missing = [t for t in MOE_TENSORS if t not in tensors]
        if missing:
            raise LagunaError(EINVAL, f"MoeFfnWeights: missing {missing}")
        self.exp_probs_b = exp_probs_b
        for t in MOE_TENSORS:
            setattr(self, t, tensors[t])


def dispatch_moe_ffn(ctx, norm_x, moe, ffn_out, n_embd, n_expert, n_expert_used, n_ff_exp, n_shexp,
                     expert_weights_norm=False, expert_weights_scale=1.0):
    """TargetModel::dispatch_moe_ffn (src/target.rs:607-748), driven from the host as
    there: the router's logits come back to the host, which picks the experts (sigmoid
    probabilities plus exp_probs_b, a stable descending sort, the first n_expert_used) and
    their scores, and launches each expert's gate and up projections at the expert's
    element offset (a u32, as there; Q8_0 and F32 weights ignore it), the activation, the
    down projection of the hidden rescaled to an L2 norm of 32768 on the host, that
    scale undone times the score on the host when the score is > 0, and the adds; then
    the shared expert.  ffn_out receives the sum.  Returns (selected experts, scores)."""
    if not 0 < n_expert_used <= n_expert:
        raise LagunaError(EINVAL, f"dispatch_moe_ffn: {n_expert_used} of {n_expert} experts")
    one = np.float32(1.0)
    scratch = []

    def buf(n):
        b = GpuBuffer(ctx, 4 * n)
        scratch.append(b)
        return b

    try:
        scores_buf = buf(n_expert)
        dispatch_proj_quant(ctx, norm_x, moe.ffn_gate_inp[0], scores_buf, n_embd, n_expert, moe.ffn_gate_inp[1])
        logits = scores_buf.read_f32(n_expert)
        probs = (one / (one + np.exp(-logits))).astype(np.float32)
        sel = (probs + moe.exp_probs_b.read_f32(n_expert)).astype(np.float32)
        chosen = [int(i) for i in np.argsort(-sel, kind="stable")[:n_expert_used]]
        scores = probs[chosen].astype(np.float32)
        if expert_weights_norm:
            total = np.float32(0.0)
            for v in scores:  # Iterator::sum, in order
                total = np.float32(total + v)
            scores = (scores / max(total, MOE_NORM_MIN)).astype(np.float32)
        if expert_weights_scale != 0.0 and expert_weights_scale != 1.0:
            scores = (scores * np.float32(expert_weights_scale)).astype(np.float32)

        moe_out, expert, gate, up, hidden = buf(n_embd), buf(n_embd), buf(n_ff_exp), buf(n_ff_exp), buf(n_ff_exp)
        moe_out.upload(np.zeros(n_embd, np.float32))
        for e, sc in zip(chosen, scores):
            off = (e * n_embd * n_ff_exp) & 0xFFFFFFFF
            dispatch_proj_quant_expert(ctx, norm_x, moe.ffn_gate_exps[0], gate, n_embd, n_ff_exp,
                                       moe.ffn_gate_exps[1], off)
            dispatch_proj_quant_expert(ctx, norm_x, moe.ffn_up_exps[0], up, n_embd, n_ff_exp, moe.ffn_up_exps[1], off)
            dispatch_activation(ctx, gate, up, hidden, n_ff_exp)
            h = hidden.read_f32(n_ff_exp)
            sq = np.add.accumulate(h * h, dtype=np.float32)[-1]  # in order, as Iterator::sum
            col_l2 = np.float32(min(max(np.float32(np.sqrt(sq)), np.float32(1e-8)), np.float32(1e30)))
            hidden.upload(((h * F16_SAFE) / col_l2).astype(np.float32))
            dispatch_proj_quant_expert(ctx, hidden, moe.ffn_down_exps[0], expert, n_ff_exp, n_embd,
                                       moe.ffn_down_exps[1], off)
            if sc > 0.0:
                o = expert.read_f32(n_embd)
                expert.upload((o * np.float32((col_l2 / F16_SAFE) * sc)).astype(np.float32))
            dispatch_add(ctx, moe_out, expert, moe_out, n_embd)

        sg, su, sh, so = buf(n_shexp), buf(n_shexp), buf(n_shexp), buf(n_embd)
        dispatch_proj_quant(ctx, norm_x, moe.ffn_gate_shexp[0], sg, n_embd, n_shexp, moe.ffn_gate_shexp[1])
        dispatch_proj_quant(ctx, norm_x, moe.ffn_up_shexp[0], su, n_embd, n_shexp, moe.ffn_up_shexp[1])
        dispatch_activation(ctx, sg, su, sh, n_shexp)
        dispatch_proj_quant(ctx, sh, moe.ffn_down_shexp[0], so, n_shexp, n_embd, moe.ffn_down_shexp[1])
        dispatch_add(ctx, moe_out, so, ffn_out, n_embd)
        return chosen, scores
    finally:
        ctx.sync()  # the launches above still read the scratch buffers
        for b in scratch:
            b.free()


def rope_freq(rope_dim, base=500000.0):
    """The f32 table of src/dflash.rs:898-904: 1 / base^(2i / rope_dim)."""
    i = np.arange(rope_dim // 2, dtype=np.float32)
    return (np.float32(1.0) / np.power(np.float32(base), (np.float32(2.0) * i) / np.float32(rope_dim))).astype(
        np.float32)


# ---- DFlash draft model ----------------------------------------------------------------


class DFlashConfig:
    """Hyperparameters of DFlashModel (src/dflash.rs:121-155 accessors).  Defaults are
    the 6-layer draft: hidden 4096, 32 Q / 8 KV heads of 128, FFN 14336, 3 aux layers."""

    def __init__(self, n_embd=4096, n_heads=32, n_kv=8, head_dim=128, rope_dim=128, n_ff=14336, n_aux=3,
                 n_layers=6, rope_base=500000.0, rms_eps=RMS_EPS, qk_eps=QK_EPS):
        self.n_embd, self.n_heads, self.n_kv, self.head_dim = n_embd, n_heads, n_kv, head_dim
        self.rope_dim, self.n_ff, self.n_aux, self.n_layers = rope_dim, n_ff, n_aux, n_layers
        self.rope_base, self.rms_eps, self.qk_eps = rope_base, rms_eps, qk_eps


class _Hparams(ctypes.Structure):
    _fields_ = [(n, _u32) for n in ("n_embd", "n_heads", "n_kv_heads", "head_dim", "rope_dim", "n_ff", "n_aux",
                                    "n_layers")] + [("rope_base", _f), ("rms_eps", _f), ("qk_eps", _f)]


DFLASH_NORMS = ("attn_norm", "attn_q_norm", "attn_k_norm", "ffn_norm")
DFLASH_PROJ = ("attn_q", "attn_k", "attn_v", "attn_gate", "attn_output", "ffn_gate", "ffn_up", "ffn_down")


class _Layer(ctypes.Structure):
    _fields_ = ([(n, _vp) for n in DFLASH_NORMS] + [(n, _vp) for n in DFLASH_PROJ]
                + [(n + "_type", _i) for n in DFLASH_PROJ] + [("k_ctx", _vp), ("v_ctx", _vp)])


class _Model(ctypes.Structure):
    _fields_ = [("hp", _Hparams), ("enc_aux_norm", _vp), ("fc", _vp), ("fc_type", _i), ("enc_output_norm", _vp),
                ("output_norm", _vp), ("layers", ctypes.POINTER(_Layer))]


class DFlashModel:
    """DFlashModel (src/dflash.rs:22-31) over device tensors.

    `enc` holds enc_aux_norm, fc (+ fc_dtype), enc_output_norm and optionally
    output_norm; `layers` one dict per decoder layer with the f32 norms of
    DFLASH_NORMS and, for each projection p of DFLASH_PROJ, the raw GGUF bytes
    p and their type p + "_dtype" (tensor names of src/dflash.rs:68-79).  The
    bytes are uploaded unchanged (Model::upload_tensor_quantized); with `tiled`
    (the default) Q4_K and Q8_0 projections are then repacked on the device into
    16-row tiles, which the forward's small-M products read as contiguous 2304-byte tiles
    (the results are the same bit for bit)."""

    def __init__(self, ctx, cfg, enc, layers, tiled=True, target_layers=None):
        self.ctx, self.cfg = ctx, cfg
        self._tl = list(target_layers or [])
        self._bufs = []
        self.layers = []
        up = self._up
        E, QD, KVD = cfg.n_embd, cfg.n_heads * cfg.head_dim, cfg.n_kv * cfg.head_dim
        shapes = {"attn_q": (E, QD), "attn_k": (E, KVD), "attn_v": (E, KVD), "attn_gate": (E, cfg.n_heads),
                  "attn_output": (QD, E), "ffn_gate": (E, cfg.n_ff), "ffn_up": (E, cfg.n_ff), "ffn_down": (cfg.n_ff, E)}

        def proj_w(a, dtype, k, n):
            b = up(a)
            if not tiled or int(dtype) not in TILED or k % 256:
                return b, int(dtype)
            t = repack_tiled(ctx, b, int(dtype), k, n)
            self._bufs.append(t)
            self._bufs.remove(b)
            ctx.sync()  # the repack has read the raw blocks
            b.free()
            return t, TILED[int(dtype)]

        fc_buf, fc_type = proj_w(enc["fc"], enc["fc_dtype"], cfg.n_aux * E, E)
        self._enc = {"enc_aux_norm": up(enc["enc_aux_norm"], np.float32), "fc": fc_buf,
                     "enc_output_norm": up(enc["enc_output_norm"], np.float32),
                     "output_norm": up(enc["output_norm"], np.float32) if enc.get("output_norm") is not None else None}
        self._layer_desc = (_Layer * len(layers))()
        for i, L in enumerate(layers):
            d = self._layer_desc[i]
            for n in DFLASH_NORMS:
                setattr(d, n, up(L[n], np.float32).ptr)
            for n in DFLASH_PROJ:
                b, t = proj_w(L[n], L[n + "_dtype"], *shapes[n])
                setattr(d, n, b.ptr)
                setattr(d, n + "_type", t)
        self._desc = _Model()
        h = self._desc.hp
        h.n_embd, h.n_heads, h.n_kv_heads, h.head_dim = cfg.n_embd, cfg.n_heads, cfg.n_kv, cfg.head_dim
        h.rope_dim, h.n_ff, h.n_aux, h.n_layers = cfg.rope_dim, cfg.n_ff, cfg.n_aux, len(layers)
        h.rope_base, h.rms_eps, h.qk_eps = cfg.rope_base, cfg.rms_eps, cfg.qk_eps
        self._desc.enc_aux_norm = self._enc["enc_aux_norm"].ptr
        self._desc.fc = self._enc["fc"].ptr
        self._desc.fc_type = fc_type
        self._desc.enc_output_norm = self._enc["enc_output_norm"].ptr
        self._desc.output_norm = self._enc["output_norm"].ptr if self._enc["output_norm"] else None
        self._desc.layers = self._layer_desc
        self.ctx_len = 0

    def _up(self, a, dtype=None):
        if isinstance(a, GpuBuffer):  # already on the device (e.g. uploaded from a GGUF file)
            self._bufs.append(a)
            return a
        a = np.ascontiguousarray(a if dtype is None else np.asarray(a, dtype))
        b = upload_bytes(self.ctx, a.view(np.uint8).ravel())
        self._bufs.append(b)
        return b

    @classmethod
    def load(cls, ctx, gguf_path, tiled=True):
        """DFlashModel::load (src/dflash.rs:34-120) with Model::from_reader's
        hyperparameters (src/model.rs:29-129).  Projections are uploaded as their raw
        GGUF blocks (Q4_K, Q8_0 and F32 run as stored; other types are dequantized to
        f32 on the device), norms as f32.  Unlike the reference, which keeps a
        missing tensor as None and panics when the forward needs it, a missing
        tensor raises here."""
        with GGUFReader(gguf_path) as rd:
            md = rd.metadata
            need = {"block_count": md.block_count, "embedding_length": md.embedding_length,
                    "feed_forward_length": md.feed_forward_length, "head_count": md.attention_head_count,
                    "head_count_kv": md.attention_head_count_kv, "key_length": md.attention_key_length}
            missing = [k for k, v in need.items() if not v]
            if missing:
                raise LagunaError(EIO, f"{gguf_path}: no {', '.join(missing)} in the metadata")
            cfg = DFlashConfig(n_embd=md.embedding_length, n_heads=md.attention_head_count,
                               n_kv=md.attention_head_count_kv, head_dim=md.attention_key_length,
                               rope_dim=md.rope_dimension_count or 0, n_ff=md.feed_forward_length,
                               n_aux=len(md.target_layers or []), n_layers=md.block_count,
                               rope_base=md.rope_freq_base if md.rope_freq_base is not None else 500000.0)

            def tensor(name, as_f32=False):
                t = rd.tensor_by_name(name)
                if t is None:
                    raise LagunaError(ENOTFOUND, f"{gguf_path}: no tensor {name!r}")
                raw = rd.upload_tensor_quantized(ctx, t)
                if t.dtype == F32 or (not as_f32 and t.dtype in (Q4_K, Q8_0)):
                    return raw, t.dtype
                out = GpuBuffer(ctx, 4 * t.n_elements())  # dequant_to_f32 on the device
                dequant_to_f32_device(ctx, raw, t.n_bytes(), t.dtype, t.n_elements(), out)
                return out, F32

            enc = {"enc_aux_norm": tensor("enc.aux_norm.weight", True)[0],
                   "enc_output_norm": tensor("enc.output_norm.weight", True)[0],
                   "output_norm": tensor("output_norm.weight", True)[0] if rd.tensor_by_name("output_norm.weight")
                   else None}
            enc["fc"], enc["fc_dtype"] = tensor("fc.weight")
            layers = []
            for i in range(cfg.n_layers):
                L = {}
                for n in DFLASH_NORMS:
                    L[n] = tensor(f"blk.{i}.{n}.weight", True)[0]
                for n in DFLASH_PROJ:
                    L[n], L[n + "_dtype"] = tensor(f"blk.{i}.{n}.weight")
                layers.append(L)
        ctx.sync()
        return cls(ctx, cfg, enc, layers, tiled, target_layers=md.target_layers or [])

    # accessors of src/dflash.rs:121-155
    def layer_count(self):
        return self._desc.hp.n_layers

    def embedding_length(self):
        return self.cfg.n_embd

    def ffn_length(self):
        return self.cfg.n_ff

    def head_count(self):
        return self.cfg.n_heads

    def head_count_kv(self):
        return self.cfg.n_kv

    def rope_dim(self):
        return self.cfg.rope_dim

    def head_dim(self):
        return self.cfg.head_dim

    def n_embd_inp(self):
        return self.cfg.n_aux * self.cfg.n_embd

    def target_layers(self):
        """The target layers whose hidden states feed the encoder (metadata
        target_layers, src/dflash.rs:149-151)."""
        return list(self._tl)

    def set_context(self, k_ctx, v_ctx):
        """Per-layer cached context keys (normed, roped) and values, [ctx_len][n_kv*head_dim] f32."""
        assert len(k_ctx) == len(v_ctx) == self.layer_count()
        n = np.asarray(k_ctx[0]).shape[0]
        for i in range(self.layer_count()):
            assert np.asarray(k_ctx[i]).shape[0] == np.asarray(v_ctx[i]).shape[0] == n
            self._layer_desc[i].k_ctx = self._up(k_ctx[i], np.float32).ptr if n else None
            self._layer_desc[i].v_ctx = self._up(v_ctx[i], np.float32).ptr if n else None
        self.ctx_len = n

    @property
    def desc(self):
        return ctypes.byref(self._desc)

    def encode(self, target_features):
        """DFlashModel::encode (src/dflash.rs:157-234) for one or more feature rows."""
        f = np.ascontiguousarray(target_features, np.float32).reshape(-1, self.n_embd_inp())
        m = f.shape[0]
        fb = upload_f32(self.ctx, f)
        ob = GpuBuffer(self.ctx, 4 * m * self.cfg.n_embd)
        check(lib().lg_dflash_encode(self.desc, fb.ptr, m, ob.ptr, self.ctx.stream))
        return ob.read_f32(m * self.cfg.n_embd).reshape(m, -1)

    def forward_block_device(self, feat, tok, m, out, ctx_len=None, stream=None):
        ctx_len = self.ctx_len if ctx_len is None else ctx_len
        check(lib().lg_dflash_forward_block(self.desc, _ptr(feat), _ptr(tok), m, ctx_len, _ptr(out),
                                            _stream(self.ctx, stream)))

    def forward_block(self, target_features, token_input, ctx_len=None):
        """m tokens over the cached context; returns the final hidden [m][n_embd]."""
        t = np.ascontiguousarray(token_input, np.float32).reshape(-1, self.cfg.n_embd)
        m = t.shape[0]
        f = np.ascontiguousarray(target_features, np.float32).reshape(m, self.n_embd_inp())
        fb, tb = upload_f32(self.ctx, f), upload_f32(self.ctx, t)
        ob = GpuBuffer(self.ctx, 4 * m * self.cfg.n_embd)
        self.forward_block_device(fb, tb, m, ob, ctx_len)
        return ob.read_f32(m * self.cfg.n_embd).reshape(m, -1)

    def forward_injected_decode_hidden(self, target_features, token_input):
        """src/dflash.rs:877-976: one token, no cached context."""
        return self.forward_block(target_features, token_input, ctx_len=0)[0]

    def capture(self, feat, tok, m, out, stream, ctx_len=None):
        """The block forward captured into a HIP graph on `stream` (a Stream)."""
        return DFlashGraph(self, feat, tok, m, out, stream, self.ctx_len if ctx_len is None else ctx_len)

    def free(self):
        for b in self._bufs:
            b.free()
        self._bufs = []


class DFlashGraph:
    def __init__(self, model, feat, tok, m, out, stream, ctx_len):
        self.model, self.stream = model, stream  # keep the tensors alive
        g = ctypes.c_void_p()
        check(lib().lg_dflash_graph_create(model.desc, _ptr(feat), _ptr(tok), m, ctx_len, _ptr(out), stream.ptr,
                                           ctypes.byref(g)))
        self.ptr = g.value

    def launch(self):
        check(lib().lg_dflash_graph_launch(self.ptr, self.stream.ptr))

    def destroy(self):
        if self.ptr:
            lib().lg_dflash_graph_destroy(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


# ---------------------------------------------------------------------------------------
# Dense target model (src/target.rs TargetModel) and the verify loop (src/lib.rs:466-520)

TARGET_NORMS = ("attn_norm", "attn_q_norm", "attn_k_norm", "ffn_norm")
TARGET_PROJ = ("attn_q", "attn_k", "attn_v", "attn_gate", "attn_output", "ffn_gate", "ffn_up", "ffn_down")


class TargetConfig:
    """Dense target hyperparameters (Model::from_reader, src/model.rs:29-129, and the
    forward's RoPE set-up, src/target.rs:321-376)."""

    def __init__(self, n_embd, n_heads, n_kv, head_dim, n_ff, n_layers, n_vocab, rope_dim, rope_dim_swa=0,
                 swa=False, rope_base=500000.0, rope_base_swa=10000.0, rms_eps=RMS_EPS, qk_eps=QK_EPS):
        self.n_embd, self.n_heads, self.n_kv, self.head_dim = n_embd, n_heads, n_kv, head_dim
        self.n_ff, self.n_layers, self.n_vocab = n_ff, n_layers, n_vocab
        self.rope_dim, self.rope_dim_swa, self.swa = rope_dim, rope_dim_swa, bool(swa)
        self.rope_base, self.rope_base_swa, self.rms_eps, self.qk_eps = rope_base, rope_base_swa, rms_eps, qk_eps


class _TgtHparams(ctypes.Structure):
    _fields_ = [(n, _u32) for n in ("n_embd", "n_heads", "n_kv_heads", "head_dim", "n_ff", "n_layers", "n_vocab",
                                    "rope_dim", "rope_dim_swa")] + \
               [("swa", _i), ("rope_base", _f), ("rope_base_swa", _f), ("rms_eps", _f), ("qk_eps", _f)]


class _TgtLayer(ctypes.Structure):
    _fields_ = ([(n, _vp) for n in TARGET_NORMS] + [(n, _vp) for n in TARGET_PROJ]
                + [(n + "_type", _i) for n in TARGET_PROJ] + [("n_q_heads", _u32)])


class _TgtModel(ctypes.Structure):
    _fields_ = [("hp", _TgtHparams), ("layers", ctypes.POINTER(_TgtLayer)), ("output_norm", _vp), ("output", _vp),
                ("output_type", _i)]


class _TgtKv(ctypes.Structure):
    _fields_ = [("k", _vp), ("v", _vp), ("capacity", _u32), ("len", _u32)]


class TargetKvCache:
    """TargetKvCache (src/target.rs:74-101) in device memory: per layer, `capacity`
    positions of normed, roped keys and raw values."""

    def __init__(self, target, capacity):
        cfg = target.cfg
        n = cfg.n_layers * capacity * cfg.n_kv * cfg.head_dim * 4
        self.k, self.v = GpuBuffer(target.ctx, max(n, 4)), GpuBuffer(target.ctx, max(n, 4))
        self._c = _TgtKv(self.k.ptr, self.v.ptr, capacity, 0)

    @property
    def len(self):
        return self._c.len

    @property
    def capacity(self):
        return self._c.capacity

    def clear(self):
        """src/target.rs:92-100 (the stored values are overwritten as tokens arrive)."""
        self._c.len = 0

    def free(self):
        self.k.free()
        self.v.free()


class TargetModel:
    """TargetModel (src/target.rs:103-605) over device tensors, dense layers.

    `layers`: one dict per layer with the f32 norms of TARGET_NORMS and, for each
    projection p of TARGET_PROJ, its raw GGUF bytes p and type p + "_dtype"
    (attn_gate may be absent or None: no gate); "n_q_heads" defaults to
    cfg.n_heads.  `tok_embd` (+ tok_embd_dtype) is the token embedding tensor,
    `output` (+ output_dtype) the LM head [n_vocab][n_embd], `output_norm` its
    norm.  Weights are uploaded as their raw GGUF bytes (load_weight,
    src/target.rs:114-127)."""

    def __init__(self, ctx, cfg, layers, tok_embd=None, tok_embd_dtype=F32, output_norm=None, output=None,
                 output_dtype=None, target_layers=None):
        self.ctx, self.cfg = ctx, cfg
        self._bufs = []
        self._tl = list(target_layers or [])
        up = self._up
        self._layer_desc = (_TgtLayer * len(layers))()
        for i, L in enumerate(layers):
            d = self._layer_desc[i]
            for n in TARGET_NORMS:
                setattr(d, n, up(L[n], np.float32).ptr)
            for n in TARGET_PROJ:
                if L.get(n) is None:
                    assert n == "attn_gate", f"layer {i}: no {n}"
                    continue
                setattr(d, n, up(L[n]).ptr)
                setattr(d, n + "_type", int(L[n + "_dtype"]))
            d.n_q_heads = int(L.get("n_q_heads", cfg.n_heads))
        self._desc = _TgtModel()
        h = self._desc.hp
        h.n_embd, h.n_heads, h.n_kv_heads, h.head_dim = cfg.n_embd, cfg.n_heads, cfg.n_kv, cfg.head_dim
        h.n_ff, h.n_layers, h.n_vocab = cfg.n_ff, len(layers), cfg.n_vocab
        h.rope_dim, h.rope_dim_swa, h.swa = cfg.rope_dim, cfg.rope_dim_swa, int(cfg.swa)
        h.rope_base, h.rope_base_swa, h.rms_eps, h.qk_eps = cfg.rope_base, cfg.rope_base_swa, cfg.rms_eps, cfg.qk_eps
        self._desc.layers = self._layer_desc
        self._desc.output_norm = up(output_norm, np.float32).ptr if output_norm is not None else None
        if output is not None:
            self._desc.output = up(output).ptr
            self._desc.output_type = int(output_dtype)
        self._emb = up(tok_embd) if tok_embd is not None else None
        self._emb_dtype = int(tok_embd_dtype)

    def _up(self, a, dtype=None):
        if isinstance(a, GpuBuffer):  # already on the device (e.g. uploaded from a GGUF file)
            self._bufs.append(a)
            return a
        a = np.ascontiguousarray(a if dtype is None else np.asarray(a, dtype))
        b = upload_bytes(self.ctx, a.view(np.uint8).ravel())
        self._bufs.append(b)
        return b

    @classmethod
    def load(cls, ctx, gguf_path):
        """TargetModel::load (src/target.rs:129-261) for a dense model, with
        Model::from_reader's hyperparameters (src/model.rs:29-129).  Projections stay
        raw GGUF blocks (Q4_K, Q8_0, F32; other types are dequantized to f32 on the
        device, as load_weight's F32 arm does on the host); norms are f32.  MoE
        models (ffn_gate_exps tensors) are refused; a missing tensor raises."""
        with GGUFReader(gguf_path) as rd:
            md = rd.metadata
            if any("ffn_gate_exps" in t.name for t in rd.tensors):
                raise LagunaError(EUNSUPPORTED, f"{gguf_path}: MoE layers are not supported by the one-call device "
                                                "forward (dispatch_moe_ffn runs a MoE FFN from the host)")
            need = {"block_count": md.block_count, "embedding_length": md.embedding_length,
                    "feed_forward_length": md.feed_forward_length, "head_count": md.attention_head_count,
                    "head_count_kv": md.attention_head_count_kv, "key_length": md.attention_key_length}
            missing = [k for k, v in need.items() if not v]
            if missing:
                raise LagunaError(EIO, f"{gguf_path}: no {', '.join(missing)} in the metadata")

            def meta(*keys):  # the key aliases of GGUFReader's metadata parser (src/gguf.rs:570-604)
                for key in keys:
                    if rd.find_field(key) is not None:
                        return rd.field(key)
                return None

            rope_dim_swa = int(meta("laguna.rope.dimension_count_swa", "dflash.rope.dimension_count_swa",
                                    "rope.dimension_count_swa") or 0)
            window = meta("laguna.attention.sliding_window", "dflash.attention.sliding_window")
            base_swa = meta("laguna.rope.freq_base_swa", "dflash.rope.freq_base_swa", "rope.freq_base_swa")
            E, HD = md.embedding_length, md.attention_key_length

            def tensor(name, as_f32=False, required=True):
                t = rd.tensor_by_name(name)
                if t is None:
                    if required:
                        raise LagunaError(ENOTFOUND, f"{gguf_path}: no tensor {name!r}")
                    return None, None, None
                raw = rd.upload_tensor_quantized(ctx, t)
                if t.dtype == F32 or (not as_f32 and t.dtype in (Q4_K, Q8_0)):
                    return raw, t.dtype, t
                out = GpuBuffer(ctx, 4 * t.n_elements())  # dequant_to_f32 on the device
                dequant_to_f32_device(ctx, raw, t.n_bytes(), t.dtype, t.n_elements(), out)
                raw.free()
                return out, F32, t

            layers = []
            for i in range(md.block_count):
                L = {}
                for n in TARGET_NORMS:
                    L[n] = tensor(f"blk.{i}.{n}.weight", True)[0]
                for n in TARGET_PROJ:
                    b, dt, t = tensor(f"blk.{i}.{n}.weight", required=n != "attn_gate")
                    L[n], L[n + "_dtype"] = b, dt
                    if n == "attn_q":  # src/target.rs:236-246
                        L["n_q_heads"] = t.shape[1] // HD if len(t.shape) >= 2 else md.attention_head_count
                layers.append(L)
            emb, emb_dt, emb_t = tensor("token_embd.weight", required=False)
            if emb_t is not None and emb_dt != emb_t.dtype:  # keep the embedding raw: rows decode on demand
                emb.free()
                emb, emb_dt = rd.upload_tensor_quantized(ctx, emb_t), emb_t.dtype
            out_norm = tensor("output_norm.weight", True, required=False)[0]
            out, out_dt, _ = tensor("output.weight", required=False)
            n_vocab = emb_t.n_elements() // E if emb_t is not None else (md.vocab_size or 0)
            cfg = TargetConfig(n_embd=E, n_heads=md.attention_head_count, n_kv=md.attention_head_count_kv,
                               head_dim=HD, n_ff=md.feed_forward_length, n_layers=md.block_count, n_vocab=n_vocab,
                               rope_dim=md.rope_dimension_count or 0, rope_dim_swa=rope_dim_swa,
                               swa=rope_dim_swa > 0 or int(window or 0) > 0,
                               rope_base=md.rope_freq_base if md.rope_freq_base is not None else 500000.0,
                               rope_base_swa=float(base_swa) if base_swa is not None else 10000.0)
            tl = md.target_layers or []
            model = cls(ctx, cfg, layers, tok_embd=emb, tok_embd_dtype=emb_dt if emb_dt is not None else F32,
                        output_norm=out_norm, output=out, output_dtype=out_dt, target_layers=tl)
            model._emb_tensor = emb_t
        ctx.sync()
        return model

    # accessors of src/target.rs:263-296
    def layer_count(self):
        return self._desc.hp.n_layers

    def embedding_length(self):
        return self.cfg.n_embd

    def vocab_size(self):
        return self.cfg.n_vocab

    def target_layers(self):
        return list(self._tl)

    @property
    def desc(self):
        return ctypes.byref(self._desc)

    def capture_count(self, layer_indices):
        lst = None if layer_indices is None else np.ascontiguousarray(layer_indices, np.uint32)
        c = _u32()
        check(lib().lg_target_capture_count(self.layer_count(), _ptr(lst), 0 if lst is None else lst.size,
                                            ctypes.byref(c)))
        return c.value

    def forward_token_device(self, inp, layer_indices, captured, logits, hidden=None, cache=None, stream=None):
        """The forward on device buffers; returns the number of captured states."""
        lst = None if layer_indices is None else np.ascontiguousarray(layer_indices, np.uint32)
        nc = _u32()
        check(lib().lg_target_forward_token(self.desc, _ptr(inp), _ptr(lst), 0 if lst is None else lst.size,
                                            _ptr(captured), ctypes.byref(nc), _ptr(logits), _ptr(hidden),
                                            ctypes.byref(cache._c) if cache is not None else None,
                                            _stream(self.ctx, stream)))
        return nc.value

    def _forward(self, inp, layer_indices, cache):
        E = self.cfg.n_embd
        nc = self.capture_count(layer_indices)
        xb = upload_f32(self.ctx, np.asarray(inp, np.float32).reshape(E))
        cb = GpuBuffer(self.ctx, 4 * max(nc, 1) * E)
        n_out = self.cfg.n_vocab if self._desc.output else E
        lb = GpuBuffer(self.ctx, 4 * n_out)
        self.forward_token_device(xb, layer_indices, cb, lb, cache=cache)
        cap = cb.read_f32(nc * E).reshape(nc, E) if nc else np.zeros((0, E), np.float32)
        return lb.read_f32(n_out).copy(), [c.copy() for c in cap]

    def forward_token(self, inp, layer_indices=None):
        """src/target.rs:298-300: (logits, captured hidden states)."""
        return self._forward(inp, layer_indices, None)

    def forward_token_cached(self, inp, layer_indices, cache):
        """src/target.rs:305-312 over a TargetKvCache."""
        return self._forward(inp, layer_indices, cache)

    def project_normalized_hidden_device(self, hidden, logits):
        check(lib().lg_dispatch_proj_quant(_ptr(hidden), self._desc.output, _ptr(logits), self.cfg.n_embd,
                                           self.cfg.n_vocab, self._desc.output_type, self.ctx.stream))

    def project_normalized_hidden(self, hidden):
        """src/target.rs:580-605: the LM head applied to a normed hidden state."""
        if not self._desc.output:
            raise LagunaError(EINVAL, "project_normalized_hidden: the model has no output weight")
        hb = upload_f32(self.ctx, np.asarray(hidden, np.float32).reshape(self.cfg.n_embd))
        lb = GpuBuffer(self.ctx, 4 * self.cfg.n_vocab)
        self.project_normalized_hidden_device(hb, lb)
        return lb.read_f32(self.cfg.n_vocab).copy()

    def token_embedding_device(self, token, out):
        """target_token_embedding (src/lib.rs:431-454) into a device buffer: row
        `token` of token_embd, decoded on the device (Q4_K as ggml blocks)."""
        E = self.cfg.n_embd
        if self._emb is None:
            raise LagunaError(EINVAL, "token_embedding: the model has no token_embd tensor")
        if not 0 <= token < self.cfg.n_vocab:
            raise LagunaError(EINVAL, f"token_id {token} >= vocab_size {self.cfg.n_vocab}")
        bb, be, _, _ = gguf_type_info(self._emb_dtype)
        if (token * E) % be == 0 and E % be == 0:  # the row is whole blocks: decode only it
            off, nbytes = token * E // be * bb, E // be * bb
            dequant_to_f32_device(self.ctx, self._emb.ptr + off, nbytes, self._emb_dtype, E, out)
            return
        full = GpuBuffer(self.ctx, 4 * (token + 1) * E)
        dequant_to_f32_device(self.ctx, self._emb, self._emb.size, self._emb_dtype, (token + 1) * E, full)
        check(lib().lg_buf_copy(_ptr(out), full.ptr + 4 * token * E, 4 * E, self.ctx.stream))
        self.ctx.sync()
        full.free()

    def token_embedding(self, token):
        ob = GpuBuffer(self.ctx, 4 * self.cfg.n_embd)
        self.token_embedding_device(token, ob)
        return ob.read_f32(self.cfg.n_embd).copy()

    def free(self):
        for b in self._bufs:
            b.free()
        self._bufs = []


class VerifyLoop:
    """run_target_dflash_verify (src/lib.rs:466-520) with every step on the device:
    token embedding, the target forward capturing the draft's target layers (as the
    draft's features, [n_aux][n_embd] in layer order), the draft forward of that
    token (forward_injected_decode_hidden), the LM head on the draft's hidden state,
    and both argmaxes; only the two token ids come back to the host."""

    def __init__(self, target, draft, target_layers=None):
        self.target, self.draft = target, draft
        self.layers = [int(v) for v in (target_layers if target_layers is not None else draft.target_layers())]
        E, ctx = target.cfg.n_embd, target.ctx
        nc = target.capture_count(self.layers)
        if nc * E != draft.n_embd_inp():
            raise LagunaError(EINVAL, f"the draft takes {draft.n_embd_inp()} features; the target captures "
                                      f"{nc} states of {E} for layers {self.layers}")
        V = target.cfg.n_vocab
        self.emb, self.feat, self.hidden = GpuBuffer(ctx, 4 * E), GpuBuffer(ctx, 4 * nc * E), GpuBuffer(ctx, 4 * E)
        self.logits = GpuBuffer(ctx, 4 * 2 * V)  # row 0: target, row 1: draft
        self.tok = GpuBuffer(ctx, 8)

    def step(self, token):
        """One step: (next_token, accepted, draft_token, target_token)."""
        t, ctx, V = self.target, self.target.ctx, self.target.cfg.n_vocab
        t.token_embedding_device(token, self.emb)
        t.forward_token_device(self.emb, self.layers, self.feat, self.logits)
        self.draft.forward_block_device(self.feat, self.emb, 1, self.hidden, ctx_len=0)
        t.project_normalized_hidden_device(self.hidden, self.logits.ptr + 4 * V)
        tgt, drf = (int(v) for v in dispatch_argmax(ctx, self.logits, V, rows=2, out=self.tok))
        accept = drf == tgt
        return (drf if accept else tgt), accept, drf, tgt

    def free(self):
        for b in (self.emb, self.feat, self.hidden, self.logits, self.tok):
            b.free()


def run_target_dflash_verify(target, draft, start_token, n_steps, target_layers=None, log=None):
    """src/lib.rs:466-520: returns (accepted tokens, exact accepts, per-step
    (input, draft, target, accept)); `log` (e.g. print) receives the reference's lines."""
    loop = VerifyLoop(target, draft, target_layers)
    token, accepted, exact, steps = start_token, [], 0, []
    try:
        for step in range(n_steps):
            nxt, ok, d, t = loop.step(token)
            exact += int(ok)
            accepted.append(nxt)
            steps.append((token, d, t, ok))
            if log:
                log(f"step {step}: input={token} draft={d} target={t} {'ACCEPT' if ok else 'REJECT'} -> accepted={nxt}")
            token = nxt
    finally:
        loop.free()
    if log:
        log(f"accepted tokens: {accepted}")
        log(f"exact draft accept rate: {exact}/{n_steps}")
    return accepted, exact, steps


# ---------------------------------------------------------------------------------------
# GGUF v3 reader (GGUFReader / TensorInfo / GGUFMetadata, src/gguf.rs:172-514)

GGUF_MAX_DIMS = 8
WHOLE = 2**64 - 1  # "the field itself" for the typed metadata reads


class _GgufTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("n_dims", _u32), ("shape", _u64 * GGUF_MAX_DIMS), ("dtype", _i),
                ("data_offset", _u64), ("n_elements", _u64), ("n_bytes", _u64)]


class _GgufMeta(ctypes.Structure):
    _fields_ = [("present", _u32), ("architecture", ctypes.c_char * 64), ("general_name", ctypes.c_char * 256),
                ("decoder_arch", ctypes.c_char * 64)] + \
               [(n, _u64) for n in ("file_type", "alignment", "block_count", "context_length", "embedding_length",
                                    "feed_forward_length", "head_count", "head_count_kv", "key_length",
                                    "value_length", "rope_dimension_count", "expert_count", "expert_used_count",
                                    "vocab_size")] + \
               [("rms_epsilon", _f), ("rope_freq_base", _f), ("expert_weights_norm", _i),
                ("n_target_layers", _u32), ("target_layers", ctypes.c_int64 * 64)]


# LG_GGUF_HAS_* bits, in declaration order
_META_FIELDS = ["architecture", "general_name", "file_type", "alignment", "block_count", "context_length",
                "embedding_length", "feed_forward_length", "head_count", "head_count_kv", "key_length",
                "value_length", "rms_epsilon", "rope_freq_base", "rope_dimension_count", "expert_count",
                "expert_used_count", "vocab_size", "target_layers", "decoder_arch", "expert_weights_norm"]
# GGUFMetadata's field names for the ones the C struct names differently
_META_NAMES = {"head_count": "attention_head_count", "head_count_kv": "attention_head_count_kv",
               "key_length": "attention_key_length", "value_length": "attention_value_length",
               "rms_epsilon": "attention_layer_norm_rms_epsilon"}


def gguf_type_info(dtype):
    """(block_size, block_elements, is_supported, is_quantized) of a GGUF type id
    (TensorType, src/gguf.rs:91-170)."""
    bb, be, sup, q = _u32(), _u32(), _i(), _i()
    check(lib().lg_gguf_type_info(dtype, ctypes.byref(bb), ctypes.byref(be), ctypes.byref(sup), ctypes.byref(q)))
    return bb.value, be.value, bool(sup.value), bool(q.value)


class TensorInfo:
    """src/gguf.rs:172-201."""

    def __init__(self, index, name, shape, dtype, data_offset, n_elements, n_bytes):
        self.index, self.name, self.shape, self.dtype = index, name, shape, dtype
        self.data_offset, self._n_elements, self._n_bytes = data_offset, n_elements, n_bytes

    def n_elements(self):
        return self._n_elements

    def n_bytes(self):
        return self._n_bytes

    def __repr__(self):
        return f"TensorInfo({self.name!r}, shape={self.shape}, dtype={self.dtype}, offset={self.data_offset})"


class GGUFMetadata:
    """The populated fields (None when absent) plus raw_fields: [(key, value)] in file order."""

    def __init__(self, m, raw_fields):
        for bit, f in enumerate(_META_FIELDS):
            name = _META_NAMES.get(f, f)
            if not m.present & (1 << bit):
                setattr(self, name, None)
            elif f in ("architecture", "general_name", "decoder_arch"):
                setattr(self, name, getattr(m, f).decode())
            elif f == "target_layers":
                setattr(self, name, [int(m.target_layers[i]) for i in range(m.n_target_layers)])
            elif f == "expert_weights_norm":
                setattr(self, name, bool(m.expert_weights_norm))
            else:
                setattr(self, name, getattr(m, f))
        self.raw_fields = raw_fields


class GGUFReader:
    """GGUFReader (src/gguf.rs:311-433) over the C reader.  Values of raw_fields are
    Python ints, floats, bools, strs or lists of them."""

    def __init__(self, path):
        h = _vp()
        check(lib().lg_gguf_open(os.fsencode(path), ctypes.byref(h)))
        self._h = h
        v, tc, fc, off = _u32(), _u64(), _u64(), _u64()
        check(lib().lg_gguf_header(h, ctypes.byref(v), ctypes.byref(tc), ctypes.byref(fc), ctypes.byref(off)))
        self.version, self.tensor_count, self.field_count = v.value, tc.value, fc.value
        self.tensor_data_offset = off.value
        self.tensors = []
        for i in range(self.tensor_count):
            t = _GgufTensor()
            check(lib().lg_gguf_tensor_info(h, i, ctypes.byref(t)))
            self.tensors.append(TensorInfo(i, t.name.decode(), [t.shape[d] for d in range(t.n_dims)], t.dtype,
                                           t.data_offset, t.n_elements, t.n_bytes))
        m = _GgufMeta()
        check(lib().lg_gguf_metadata(h, ctypes.byref(m)))
        self.metadata = GGUFMetadata(m, [(k, self.field_at(i)) for i, k in enumerate(self._keys())])

    @classmethod
    def open(cls, path):
        return cls(path)

    def _keys(self):
        n = _u64()
        check(lib().lg_gguf_field_count(self._h, ctypes.byref(n)))
        keys = []
        for i in range(n.value):
            k = ctypes.c_char_p()
            check(lib().lg_gguf_field(self._h, i, ctypes.byref(k), None, None, None))
            keys.append(k.value.decode())
        return keys

    def find_field(self, key):
        """Index of the first metadata field named `key`, or None."""
        idx = _u64()
        st = lib().lg_gguf_find_field(self._h, key.encode(), ctypes.byref(idx))
        if st == ENOTFOUND:
            return None
        check(st)
        return idx.value

    def field(self, key):
        """The value of the first metadata field named `key` (LagunaError if absent)."""
        idx = self.find_field(key)
        if idx is None:
            raise LagunaError(ENOTFOUND, f"no metadata key {key!r}")
        return self.field_at(idx)

    def field_at(self, index):
        """The value of the index-th metadata field."""
        t, n, et = _i(), _u64(), _i()
        check(lib().lg_gguf_field(self._h, index, None, ctypes.byref(t), ctypes.byref(n), ctypes.byref(et)))
        if t.value == 9:
            if et.value == 9:
                return None  # arrays of arrays are not mirrored
            return [self._scalar(index, et.value, j) for j in range(n.value)]
        return self._scalar(index, t.value, WHOLE)

    def _scalar(self, index, typ, elem):
        h = self._h
        if typ == 8:
            out, n = ctypes.c_char_p(), _u64()
            check(lib().lg_gguf_get_str(h, index, elem, ctypes.byref(out), ctypes.byref(n)))
            return ctypes.string_at(out, n.value).decode("utf-8", "replace")
        if typ in (6, 12):
            out = ctypes.c_double()
            check(lib().lg_gguf_get_f64(h, index, elem, ctypes.byref(out)))
            return out.value
        if typ == 7:
            out = _i()
            check(lib().lg_gguf_get_bool(h, index, elem, ctypes.byref(out)))
            return bool(out.value)
        out = ctypes.c_int64()
        check(lib().lg_gguf_get_i64(h, index, elem, ctypes.byref(out)))
        return out.value if typ in (1, 3, 5, 11) else out.value & (2**64 - 1)

    def tensor_by_name(self, name):
        """src/gguf.rs:407-409: the first tensor of that name, or None."""
        idx = _u64()
        st = lib().lg_gguf_find_tensor(self._h, name.encode(), ctypes.byref(idx))
        if st == ENOTFOUND:
            return None
        check(st)
        return self.tensors[idx.value]

    def tensors_with_dtype(self, dtype):
        return [t for t in self.tensors if t.dtype == dtype]

    def read_tensor_data(self, tensor):
        """src/gguf.rs:415-421: the tensor's n_bytes raw bytes."""
        buf = np.empty(tensor.n_bytes(), np.uint8)
        check(lib().lg_gguf_read_tensor(self._h, tensor.index, buf.ctypes.data, buf.size))
        return buf

    def upload_tensor_quantized(self, ctx, tensor, stream=None):
        """Model::upload_tensor_quantized (src/model.rs:174-184): the raw bytes in a new device buffer."""
        b = GpuBuffer(ctx, max(tensor.n_bytes(), 1))
        check(lib().lg_gguf_upload_tensor(self._h, tensor.index, b.ptr, tensor.n_bytes(), stream))
        return b

    def layer_count(self):
        return self.metadata.block_count

    def embedding_length(self):
        return self.metadata.embedding_length

    def close(self):
        if self._h:
            check(lib().lg_gguf_close(self._h))
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
