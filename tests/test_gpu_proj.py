"""GPU: M=1 projections against the oracle's f64 accumulation (tolerance 1e-4 on
max|err|/sum|W x| and on ||err||_inf/||y||_inf), plus the reference's own
layout known answer and the edge cases of the dispatch functions."""
import numpy as np
import pytest

import laguna_hip as lh
import oracle as orc
import synth
from conftest import parity

pytestmark = pytest.mark.gpu

TOL = 1e-4


def weight(dtype, seed, k, n):
    if dtype == lh.Q4_K:
        return synth.q4k_weight(seed, k, n)
    if dtype == lh.Q8_0:
        return synth.q8_0_weight(seed, k, n)
    return synth.normal(seed, k * n, 0.02)


def run_proj(ctx, dtype, raw, x, k, n, expert_offset=None):
    wb = lh.upload_bytes(ctx, raw.view(np.uint8))
    xb = lh.upload_f32(ctx, x)
    cb = lh.GpuBuffer(ctx, 4 * n)
    if expert_offset is None:
        lh.dispatch_proj_quant(ctx, xb, wb, cb, k, n, dtype)
    else:
        lh.dispatch_proj_quant_expert(ctx, xb, wb, cb, k, n, dtype, expert_offset)
    return cb.read_f32(n)


@pytest.mark.parametrize("dtype,k,n,seed", [
    (lh.Q4_K, 4096, 14336, 0x5EED0003),   # gate/up projection, headline shape
    (lh.Q4_K, 14336, 4096, 0x5EED0005),   # down projection
    (lh.Q4_K, 12288, 4096, 0x5EED000B),   # encoder fc (3 x 4096 in)
    (lh.Q4_K, 4096, 4096, 0x5EED000F),    # attn_q: one 8-wavefront workgroup per CU, two rows a wave
    (lh.Q4_K, 4096, 1024, 0x5EED000C),    # attn_k / attn_v
    (lh.Q4_K, 4096, 32, 0x5EED000D),      # attn_gate
    (lh.Q8_0, 4096, 4096, 0x5EED0001),    # o_proj
    (lh.Q8_0, 14336, 4096, 0x5EED000E),
    (lh.Q8_0, 12288, 256, 0x5EED000F),
    (lh.Q8_0, 8192, 300, 0x5EED0010),
])
def test_config_shapes(ctx, dtype, k, n, seed):
    print(f"proj dtype={dtype} k={k} n={n} seed={seed:#x}", flush=True)
    raw = weight(dtype, seed, k, n)
    x = synth.normal(seed + 1, k)
    y = run_proj(ctx, dtype, raw, x, k, n)
    y64, a = orc.proj_quant_f64(x, raw, dtype, k, n)
    parity(y, y64, a, TOL)


def assert_same_non_finite(y, y64):
    y = np.asarray(y, np.float64)
    assert np.array_equal(np.isnan(y), np.isnan(y64)), "NaN pattern differs"
    assert np.array_equal(np.isinf(y), np.isinf(y64)), "inf pattern differs"
    inf = np.isinf(y64)
    assert np.array_equal(np.sign(y[inf]), np.sign(y64[inf]))


@pytest.mark.parametrize("dtype,k,n", [(lh.Q4_K, 4096, 300), (lh.Q4_K, 1024, 37), (lh.Q4_K, 12288, 40),
                                       (lh.Q4_K, 20480, 40), (lh.Q8_0, 4096, 300), (lh.Q8_0, 1024, 37),
                                       (lh.Q8_0, 14336, 40)])
def test_activations_outside_the_digit_range(ctx, dtype, k, n):
    # Q4_K up to k = 16384 and Q8_0 up to 4096 convert x to byte digits (per
    # 64-element group up to 4096, per super-block beyond); values they cannot scale
    # (non-finite, >= 2^21, nonzero below 2^-60) send the call to the reference's
    # per-element loop, whose results the f64 accumulation matches.  Beyond those k
    # (Q4_K 20480, Q8_0 14336) the f32 vector kernels take every finite value as it is
    # and a lane holding inf or NaN sums its terms element by element.
    raw = weight(dtype, 300 + k, k, n)
    x = synth.normal(301 + k, k)
    for idx, val in [(5, np.inf), (k - 3, -np.inf), (k // 3, np.nan)]:
        print(f"proj dtype={dtype} k={k} x[{idx}]={val}", flush=True)
        xs = x.copy()
        xs[idx] = val
        y64, _ = orc.proj_quant_f64(xs, raw, dtype, k, n)
        assert_same_non_finite(run_proj(ctx, dtype, raw, xs, k, n), y64)
    cases = {
        "huge": lambda v: np.where(np.arange(k) == 77, np.float32(3e6), v),       # one value >= 2^21
        "tiny": lambda v: (v * 1e-20).astype(np.float32),                           # all below 2^-60
        "wide": lambda v: np.where(np.arange(k) % 64 == 9, np.float32(30.0), v * np.float32(1e-3)),
        "zero_groups": lambda v: np.where((np.arange(k) // 64) % 3 == 1, np.float32(0.0), v),
        "mixed_scales": lambda v: (v * np.exp2(np.arange(k) // 64 % 40 - 30.0)).astype(np.float32),
    }
    for name, f in cases.items():
        print(f"proj dtype={dtype} k={k} {name} activations", flush=True)
        xs = f(x).astype(np.float32)
        y64, a = orc.proj_quant_f64(xs, raw, dtype, k, n)
        parity(run_proj(ctx, dtype, raw, xs, k, n), y64, a, TOL)


def test_q4k_exponent0_scales(ctx):
    # d and dmin codes with exponent 0 and a non-zero mantissa, which the reference
    # decodes as 2^-14 * (1 + m/1024) (src/dflash.rs:314-329), on the k <= 4096 path
    k, n = 4096, 256
    print("proj q4k exponent-0 f16 scales", flush=True)
    raw = synth.q4k_weight(310, k, n).reshape(-1, 144).copy()
    h = np.frombuffer(raw[:, 0:4].tobytes(), np.uint16).reshape(-1, 2).copy()
    sel = np.arange(raw.shape[0])
    h[sel % 7 == 0, 0] = 0x0001 + (sel[sel % 7 == 0] % 0x3FF).astype(np.uint16)
    h[sel % 5 == 0, 1] = 0x8000 | (0x0100 + (sel[sel % 5 == 0] % 0x2FF)).astype(np.uint16)
    raw[:, 0:4] = h.view(np.uint8).reshape(-1, 4)
    raw = raw.ravel()
    x = synth.normal(311, k)
    y64, a = orc.proj_quant_f64(x, raw, orc.Q4_K, k, n)
    parity(run_proj(ctx, lh.Q4_K, raw, x, k, n), y64, a, TOL)


@pytest.mark.parametrize("dtype", [lh.Q4_K, lh.Q8_0])
@pytest.mark.parametrize("k,n", [(256, 1), (256, 7), (512, 33), (768, 5), (1024, 64), (2048, 9),
                                 (2304, 11), (3072, 13), (4352, 3), (6144, 17), (16384, 5),
                                 (16640, 7), (20480, 64), (32768, 33)])  # past 16384: passes over k
def test_small_and_odd_shapes(ctx, dtype, k, n):
    seed = 1000 + k + n
    print(f"proj small dtype={dtype} k={k} n={n}", flush=True)
    raw = weight(dtype, seed, k, n)
    x = synth.normal(seed + 1, k)
    y = run_proj(ctx, dtype, raw, x, k, n)
    y64, a = orc.proj_quant_f64(x, raw, dtype, k, n)
    parity(y, y64, a, TOL)


@pytest.mark.parametrize("dtype,k,n", [(lh.Q4_K, 96, 8), (lh.Q4_K, 288, 8), (lh.Q4_K, 20000, 64),
                                       (lh.Q8_0, 96, 5), (lh.Q8_0, 4128, 7), (lh.Q8_0, 32, 1)])
def test_generic_path_shapes(ctx, dtype, k, n):
    # k not a multiple of 256 (or above 16384): reference linear addressing,
    # rows that start inside a block
    print(f"proj generic dtype={dtype} k={k} n={n}", flush=True)
    bs = 256 if dtype == lh.Q4_K else 32
    nblk = -(-(k * n) // bs)
    raw = synth.random_q4k(77, nblk) if dtype == lh.Q4_K else synth.q8_0_weight(77, bs, nblk)
    x = synth.normal(78, k)
    y = run_proj(ctx, dtype, raw, x, k, n)
    y64, a = orc.proj_quant_f64(x, raw, dtype, k, n)
    parity(y, y64, a, TOL)


@pytest.mark.parametrize("offset", [4096 * 64, 256 * 3, 100])
def test_expert_offset_q4k(ctx, offset):
    # kernels/proj_q4k.comp:67: lin = expert_offset + i*k + j (aligned -> fast path,
    # unaligned -> element-wise path)
    k, n = 4096, 64
    raw = synth.q4k_weight(91, k, 2 * n)
    x = synth.normal(92, k)
    print(f"proj expert offset {offset}", flush=True)
    y = run_proj(ctx, lh.Q4_K, raw, x, k, n, expert_offset=offset)
    y64, a = orc.proj_quant_f64(x, raw, orc.Q4_K, k, n, elem_offset=offset)
    parity(y, y64, a, TOL)


def test_expert_offset_ignored_for_q8_0(ctx):
    # src/target.rs:1118-1138: the Q8_0 arm binds no offset
    k, n = 1024, 16
    raw = synth.q8_0_weight(93, k, 2 * n)
    x = synth.normal(94, k)
    print("proj q8_0 expert offset ignored", flush=True)
    y_off = run_proj(ctx, lh.Q8_0, raw, x, k, n, expert_offset=k * n)
    y0 = run_proj(ctx, lh.Q8_0, raw, x, k, n)
    assert np.array_equal(y_off, y0)


def test_reference_layout_known_answer(ctx, golden):
    # src/lib.rs:120-165 (proj.comp, k=8, n=3), |err| < 1e-4
    print("proj f32 known answer 8x3", flush=True)
    a, b = golden["mm_a"], golden["mm_b"]
    y = run_proj(ctx, lh.F32, b, a, 8, 3)
    assert np.all(np.abs(y - golden["mm_expected"]) < 1e-4)
    xb, wb, cb = lh.upload_f32(ctx, a), lh.upload_f32(ctx, b.reshape(3, 8).T.copy()), lh.GpuBuffer(ctx, 12)
    lh.dispatch_proj_row(ctx, xb, wb, cb, 8, 3, 1)
    assert np.all(np.abs(cb.read_f32(3) - golden["mm_expected"]) < 1e-4)
    out = lh.dispatch_proj_read(ctx, xb, lh.upload_f32(ctx, b), 8, 3)
    assert np.all(np.abs(out - golden["mm_expected"]) < 1e-4)


@pytest.mark.parametrize("k,n", [(4096, 1024), (1000, 17), (3, 5)])
def test_f32_weights(ctx, k, n):
    print(f"proj f32 k={k} n={n}", flush=True)
    w = synth.normal(95, k * n, 0.02)
    x = synth.normal(96, k)
    y = run_proj(ctx, lh.F32, w, x, k, n)
    y64, a = orc.proj_quant_f64(x, w, orc.F32, k, n)
    parity(y, y64, a, TOL)


def test_fused_silu_down_projection(ctx):
    # config: Q4_K 14336 -> 4096 with x = silu(gate) * up computed in the kernel
    k, n = 14336, 4096
    print("fused silu down-proj 14336->4096 seeds 0x5EED0005/6/7", flush=True)
    raw = synth.q4k_weight(0x5EED0005, k, n)
    gate, up = synth.normal(0x5EED0006, k), synth.normal(0x5EED0007, k)
    wb, gb, ub, cb = lh.upload_bytes(ctx, raw), lh.upload_f32(ctx, gate), lh.upload_f32(ctx, up), lh.GpuBuffer(ctx, 4 * n)
    lh.dispatch_silu_mul_proj_quant(ctx, gb, ub, wb, cb, k, n, lh.Q4_K)
    h64 = orc.silu_mul_f64(gate, up)
    y64, a = orc.proj_quant_f64x(h64, raw, orc.Q4_K, k, n)
    parity(cb.read_f32(n), y64, a, TOL)


@pytest.mark.parametrize("dtype,k,n", [(lh.Q4_K, 4096, 100), (lh.Q8_0, 4096, 50), (lh.Q4_K, 1024, 8),
                                       (lh.Q4_K, 288, 4)])
def test_fused_silu_other_shapes(ctx, dtype, k, n):
    print(f"fused silu dtype={dtype} k={k} n={n}", flush=True)
    bs = 256 if dtype == lh.Q4_K else 32
    nblk = -(-(k * n) // bs)
    raw = synth.random_q4k(97, nblk) if dtype == lh.Q4_K else synth.q8_0_weight(97, bs, nblk)
    gate, up = synth.normal(98, k), synth.normal(99, k)
    wb, gb, ub, cb = lh.upload_bytes(ctx, raw), lh.upload_f32(ctx, gate), lh.upload_f32(ctx, up), lh.GpuBuffer(ctx, 4 * n)
    lh.dispatch_silu_mul_proj_quant(ctx, gb, ub, wb, cb, k, n, dtype)
    y64, a = orc.proj_quant_f64x(orc.silu_mul_f64(gate, up), raw, dtype, k, n)
    parity(cb.read_f32(n), y64, a, TOL)


def fused_run(ctx, raw, gate, up, k, n):
    wb, gb, ub, cb = lh.upload_bytes(ctx, raw), lh.upload_f32(ctx, gate), lh.upload_f32(ctx, up), lh.GpuBuffer(ctx, 4 * n)
    lh.dispatch_silu_mul_proj_quant(ctx, gb, ub, wb, cb, k, n, lh.Q4_K)
    return cb.read_f32(n)


@pytest.mark.parametrize("kind", [1, 2])
@pytest.mark.parametrize("k,n", [(14336, 4096), (12288, 40), (5120, 33), (16384, 7), (4352, 5)])
def test_fused_silu_kernel_families(ctx, kind, k, n):
    # The fused SiLU down projection on the vector kernel (1) and on int8 matrix cores
    # (2, the automatic choice for k <= 16384), each bit-for-bit repeatable.
    seed = 7000 + k + n
    print(f"fused silu family {kind} k={k} n={n}", flush=True)
    raw = synth.q4k_weight(seed, k, n)
    gate, up = synth.normal(seed + 1, k), synth.normal(seed + 2, k)
    lh.check(lh.lib().lg_set_m1_kernel(kind))
    try:
        y1 = fused_run(ctx, raw, gate, up, k, n)
        y2 = fused_run(ctx, raw, gate, up, k, n)
    finally:
        lh.check(lh.lib().lg_set_m1_kernel(0))
    assert np.array_equal(y1, y2)
    y64, a = orc.proj_quant_f64x(orc.silu_mul_f64(gate, up), raw, orc.Q4_K, k, n)
    parity(y1, y64, a, TOL)


@pytest.mark.parametrize("kind", [1, 2])
def test_fused_silu_outside_digit_range(ctx, kind):
    # Non-finite silu(gate) * up propagates as in the reference's f32 loop on both
    # families; tiny activations send the matrix-core kernel's super-blocks (2) to the
    # per-element loop, while the vector kernel (1) takes them in f32 as they are.  The
    # matrix-core kernel scales per super-block, so a value 10^6 times its neighbours
    # costs it up to 2^-22 of that value per element of the super-block: that case is
    # left to the vector kernel.
    k, n = 14336, 64
    raw = synth.q4k_weight(7100, k, n)
    gate, up = synth.normal(7101, k), synth.normal(7102, k)
    lh.check(lh.lib().lg_set_m1_kernel(kind))
    try:
        for idx, val in [(5, np.inf), (k - 3, -np.inf), (k // 3, np.nan)]:
            print(f"fused silu family {kind} gate[{idx}]={val}", flush=True)
            gs = gate.copy()
            gs[idx] = val
            y64, _ = orc.proj_quant_f64x(orc.silu_mul_f64(gs, up), raw, orc.Q4_K, k, n)
            assert_same_non_finite(fused_run(ctx, raw, gs, up, k, n), y64)
        gh = gate.copy()
        gh[9000] = 8.0  # silu(8) * 4e5 = 3.2e6 >= 2^21
        cases = [("tiny", gate, (up * 1e-20).astype(np.float32))]
        if kind == 1:
            cases.append(("huge", gh, np.where(np.arange(k) == 9000, np.float32(4e5), up).astype(np.float32)))
        for name, gs, us in cases:
            print(f"fused silu family {kind} {name} activations", flush=True)
            y64, a = orc.proj_quant_f64x(orc.silu_mul_f64(gs, us), raw, orc.Q4_K, k, n)
            parity(fused_run(ctx, raw, gs, us, k, n), y64, a, TOL)
    finally:
        lh.check(lh.lib().lg_set_m1_kernel(0))


def test_activation_kernel(ctx):
    n = 14336
    g, u = synth.normal(100, n), synth.normal(101, n)
    gb, ub, hb = lh.upload_f32(ctx, g), lh.upload_f32(ctx, u), lh.GpuBuffer(ctx, 4 * n)
    print("activation n=14336", flush=True)
    lh.dispatch_activation(ctx, gb, ub, hb, n)
    h = hb.read_f32(n).astype(np.float64)
    h64 = orc.silu_mul_f64(g, u)
    assert np.max(np.abs(h - h64) / np.maximum(np.abs(h64), 1e-3)) < 1e-5


def test_zero_k_gives_zeros_and_zero_n_is_no_op(ctx):
    cb = lh.GpuBuffer(ctx, 64)
    cb.fill(0x7F)
    xb, wb = lh.GpuBuffer(ctx, 64), lh.GpuBuffer(ctx, 144)
    print("proj k=0 / n=0", flush=True)
    lh.dispatch_proj_quant(ctx, xb, wb, cb, 0, 16, lh.Q4_K)
    assert np.all(cb.read_f32(16) == 0)
    cb.fill(0x7F)
    lh.dispatch_proj_quant(ctx, xb, wb, cb, 256, 0, lh.Q4_K)
    assert np.all(cb.download() == 0x7F)


def test_extent_checks_reject_short_buffers(ctx):
    k, n = 4096, 64
    raw = synth.q4k_weight(102, k, n)
    wb = lh.upload_bytes(ctx, raw[: raw.size - 144])  # one block short
    xb, cb = lh.upload_f32(ctx, synth.normal(103, k)), lh.GpuBuffer(ctx, 4 * n)
    with pytest.raises(lh.LagunaError) as e:
        lh.dispatch_proj_quant(ctx, xb, wb, cb, k, n, lh.Q4_K)
    assert e.value.status == lh.EINVAL
    small_c = lh.GpuBuffer(ctx, 4 * (n - 1))
    with pytest.raises(lh.LagunaError):
        lh.dispatch_proj_quant(ctx, xb, lh.upload_bytes(ctx, raw), small_c, k, n, lh.Q4_K)


def test_blocking_mode_and_determinism(ctx):
    k, n = 4096, 2048
    raw = synth.q4k_weight(104, k, n)
    x = synth.normal(105, k)
    print("proj blocking + determinism", flush=True)
    lh.check(lh.lib().lg_set_blocking(1))
    try:
        y1 = run_proj(ctx, lh.Q4_K, raw, x, k, n)
    finally:
        lh.check(lh.lib().lg_set_blocking(0))
    y2 = run_proj(ctx, lh.Q4_K, raw, x, k, n)
    assert np.array_equal(y1, y2)


@pytest.mark.parametrize("cap", [1, 7, 256])
def test_grid_cap_launch_shapes(ctx, cap):
    # The workgroup cap changes rows per workgroup (and, for Q4_K, how a row's
    # super-blocks are split over waves, hence the f32 summation order): every shape
    # must meet parity, and a fixed shape must be bit-for-bit repeatable.
    k, n = 4096, 777
    raw = synth.q4k_weight(106, k, n)
    raw8 = synth.q8_0_weight(108, k, n)
    x = synth.normal(107, k)
    print(f"proj grid cap {cap}", flush=True)
    y0 = run_proj(ctx, lh.Q4_K, raw, x, k, n)
    y80 = run_proj(ctx, lh.Q8_0, raw8, x, k, n)
    lh.check(lh.lib().lg_set_m1_grid_cap(cap))
    try:
        y1 = run_proj(ctx, lh.Q4_K, raw, x, k, n)
        y1b = run_proj(ctx, lh.Q4_K, raw, x, k, n)
        y8 = run_proj(ctx, lh.Q8_0, raw8, x, k, n)
    finally:
        lh.check(lh.lib().lg_set_m1_grid_cap(0))
    assert np.array_equal(y1, y1b)
    assert np.array_equal(y8, y80)  # Q8_0 rows are summed in one fixed order
    y64, a = orc.proj_quant_f64(x, raw, orc.Q4_K, k, n)
    parity(y0, y64, a, TOL)
    parity(y1, y64, a, TOL)


@pytest.mark.parametrize("kind", [1, 2])
@pytest.mark.parametrize("k,n", [(4096, 14336), (4096, 16500), (4096, 777), (4096, 57), (4096, 16), (4096, 1),
                                 (1024, 37), (256, 3), (3072, 100), (14336, 100), (12288, 40)])
def test_q4k_kernel_families(ctx, kind, k, n):
    # Family 1 (vector ALU / integer dot products) and family 2 (int8 matrix cores
    # over row ranges of up to 64 rows per workgroup, partial 16-row groups
    # included) both meet parity at every shape; each is bit-for-bit repeatable.
    seed = 5000 + k + n
    print(f"proj q4k kernel family {kind} k={k} n={n}", flush=True)
    raw = synth.q4k_weight(seed, k, n)
    x = synth.normal(seed + 1, k)
    lh.check(lh.lib().lg_set_m1_kernel(kind))
    try:
        y1 = run_proj(ctx, lh.Q4_K, raw, x, k, n)
        y2 = run_proj(ctx, lh.Q4_K, raw, x, k, n)
    finally:
        lh.check(lh.lib().lg_set_m1_kernel(0))
    assert np.array_equal(y1, y2)
    y64, a = orc.proj_quant_f64(x, raw, lh.Q4_K, k, n)
    parity(y1, y64, a, TOL)


@pytest.mark.parametrize("kind", [1, 2])
def test_q4k_kernel_families_outside_digit_range(ctx, kind):
    k, n = 4096, 300
    raw = synth.q4k_weight(5100, k, n)
    x = synth.normal(5101, k)
    lh.check(lh.lib().lg_set_m1_kernel(kind))
    try:
        for idx, val in [(5, np.inf), (k - 3, -np.inf), (k // 3, np.nan)]:
            print(f"proj q4k family {kind} x[{idx}]={val}", flush=True)
            xs = x.copy()
            xs[idx] = val
            y64, _ = orc.proj_quant_f64(xs, raw, lh.Q4_K, k, n)
            assert_same_non_finite(run_proj(ctx, lh.Q4_K, raw, xs, k, n), y64)
        for name, xs in [("tiny", (x * 1e-20).astype(np.float32)),
                         ("wide", np.where(np.arange(k) % 256 == 9, np.float32(30.0), x * np.float32(1e-3))),
                         ("huge", np.where(np.arange(k) == 77, np.float32(3e6), x))]:
            print(f"proj q4k family {kind} {name} activations", flush=True)
            xs = xs.astype(np.float32)
            y64, a = orc.proj_quant_f64(xs, raw, lh.Q4_K, k, n)
            parity(run_proj(ctx, lh.Q4_K, raw, xs, k, n), y64, a, TOL)
    finally:
        lh.check(lh.lib().lg_set_m1_kernel(0))


def test_m1_kernel_hook_rejects_unknown_family(ctx):
    with pytest.raises(lh.LagunaError) as e:
        lh.check(lh.lib().lg_set_m1_kernel(3))
    assert e.value.status == lh.EINVAL
