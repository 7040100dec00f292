"""GPU: the fused SiLU(gate)*up + Q4_K down projection (int8 matrix-core kernel)
against the oracle's f64 accumulation, across k-slice counts and on the inputs
that take its per-element fallback (non-finite or tiny activations) or its f16
scale correction (exponent-0 codes, which the reference decodes as 2^-14 + 2^-24 m)."""
import numpy as np
import pytest

import laguna_hip as lh
import oracle as orc
import synth
from conftest import parity

pytestmark = pytest.mark.gpu

TOL = 1e-4


def run_fused(ctx, raw, gate, up, k, n):
    wb, gb, ub = lh.upload_bytes(ctx, raw), lh.upload_f32(ctx, gate), lh.upload_f32(ctx, up)
    cb = lh.GpuBuffer(ctx, 4 * n)
    lh.dispatch_silu_mul_proj_quant(ctx, gb, ub, wb, cb, k, n, lh.Q4_K)
    return cb.read_f32(n)


def oracle_fused(raw, gate, up, k, n):
    return orc.proj_quant_f64x(orc.silu_mul_f64(gate, up), raw, orc.Q4_K, k, n)


@pytest.mark.parametrize("split", [1, 3, 7, 14, 28, 56])
def test_k_slices(ctx, split):
    # Every slice count meets parity and is bit-for-bit repeatable (slices are
    # added in slice order by whichever workgroup finishes last).
    k, n = 14336, 1000
    print(f"fused split={split} k={k} n={n}", flush=True)
    raw = synth.q4k_weight(200, k, n)
    gate, up = synth.normal(201, k), synth.normal(202, k)
    lh.check(lh.lib().lg_set_m1_split(split))
    try:
        y1 = run_fused(ctx, raw, gate, up, k, n)
        y2 = run_fused(ctx, raw, gate, up, k, n)
    finally:
        lh.check(lh.lib().lg_set_m1_split(0))
    assert np.array_equal(y1, y2)
    y64, a = oracle_fused(raw, gate, up, k, n)
    parity(y1, y64, a, TOL)


@pytest.mark.parametrize("k,n", [(256, 3), (512, 17), (4096, 4096), (12288, 64), (16384, 33), (20480, 40)])
def test_shapes(ctx, k, n):
    print(f"fused k={k} n={n}", flush=True)
    raw = synth.q4k_weight(210 + k, k, n)
    gate, up = synth.normal(211, k), synth.normal(212, k)
    y = run_fused(ctx, raw, gate, up, k, n)
    y64, a = oracle_fused(raw, gate, up, k, n)
    parity(y, y64, a, TOL)


def test_non_finite_activations(ctx):
    # silu(+inf) * up = +-inf, silu(-inf) = -inf * 0 = NaN (the reference's
    # formula): the slices holding them fall back to the per-element loop; every
    # output is non-finite exactly where the f64 accumulation is, with its sign.
    k, n = 4096, 300
    print("fused non-finite activations", flush=True)
    raw = synth.q4k_weight(220, k, n)
    gate, up = synth.normal(221, k), synth.normal(222, k)
    for idx, val in [(5, np.inf), (3000, -np.inf), (1234, np.nan)]:
        g = gate.copy()
        g[idx] = val
        y = run_fused(ctx, raw, g, up, k, n).astype(np.float64)
        y64, _ = oracle_fused(raw, g, up, k, n)
        assert np.array_equal(np.isnan(y), np.isnan(y64)), f"NaN pattern differs for gate[{idx}]={val}"
        assert np.array_equal(np.isinf(y), np.isinf(y64)), f"inf pattern differs for gate[{idx}]={val}"
        inf = np.isinf(y64)
        assert np.array_equal(np.sign(y[inf]), np.sign(y64[inf]))


def test_tiny_and_wide_activations(ctx):
    k, n = 4096, 256
    raw = synth.q4k_weight(230, k, n)
    gate, up = synth.normal(231, k), synth.normal(232, k)
    # |silu(g) up| ~ 1e-36: below 2^-100, the per-element loop
    print("fused tiny activations", flush=True)
    gt, ut = (gate * 1e-18).astype(np.float32), (up * 1e-18).astype(np.float32)
    y64, a = oracle_fused(raw, gt, ut, k, n)
    parity(run_fused(ctx, raw, gt, ut, k, n), y64, a, TOL)
    # one large element per super-block among small ones: the digits keep 22 bits
    # of each super-block's maximum
    print("fused wide activations", flush=True)
    gw = gate.copy() * 1e-3
    gw[::256] = 30.0
    y64, a = oracle_fused(raw, gw, up, k, n)
    parity(run_fused(ctx, raw, gw, up, k, n), y64, a, TOL)


def test_exponent0_scales(ctx):
    # d and dmin codes with exponent 0 and a non-zero mantissa, which the
    # reference decodes as 2^-14 * (1 + m/1024) (src/dflash.rs:314-329)
    k, n = 4096, 128
    print("fused exponent-0 f16 scales", flush=True)
    raw = synth.q4k_weight(240, k, n).reshape(-1, 144).copy()
    h = np.frombuffer(raw[:, 0:4].tobytes(), np.uint16).reshape(-1, 2).copy()
    sel = np.arange(raw.shape[0])
    h[sel % 7 == 0, 0] = 0x0001 + (sel[sel % 7 == 0] % 0x3FF).astype(np.uint16)   # d
    h[sel % 5 == 0, 1] = 0x8000 | (0x0100 + (sel[sel % 5 == 0] % 0x2FF)).astype(np.uint16)  # dmin < 0
    raw[:, 0:4] = h.view(np.uint8).reshape(-1, 4)
    raw = raw.ravel()
    gate, up = synth.normal(241, k), synth.normal(242, k)
    y64, a = oracle_fused(raw, gate, up, k, n)
    parity(run_fused(ctx, raw, gate, up, k, n), y64, a, TOL)
