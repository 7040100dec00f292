"""GPU: target-side verify -- the device argmax of the reference's argmax
(src/lib.rs:456-464), bit for bit against the oracle's fold, alone and on the
logits of the vocab-sized LM head, and the accept decision of
run_target_dflash_verify (src/lib.rs:497-503)."""
import numpy as np
import pytest

import laguna_hip as lh
import oracle as orc
import synth

pytestmark = pytest.mark.gpu


def logits_rows(seed, rows, n, kind):
    rng = np.random.default_rng(seed)
    if kind == "ties":  # few distinct values: many equal maxima
        v = rng.integers(-3, 4, (rows, n)).astype(np.float32)
    else:
        v = rng.standard_normal((rows, n)).astype(np.float32)
    if kind == "special":
        for r in range(rows):
            for _ in range(int(rng.integers(0, 4))):
                v[r, rng.integers(0, n)] = np.nan
            if r % 3 == 0:
                v[r, rng.integers(0, n)] = np.inf
            if r % 4 == 1:
                v[r, -1] = np.nan
            if r % 5 == 2:
                v[r, :] = 0.0
                v[r, rng.integers(0, n)] = -0.0
    return v


def device_argmax(ctx, v, n, rows, ld):
    buf = lh.upload_f32(ctx, np.ascontiguousarray(v, np.float32).ravel())
    return lh.dispatch_argmax(ctx, buf, n, rows, ld)


@pytest.mark.parametrize("n", [1, 2, 15, 16, 17, 4095, 4096, 4097, 8193, 65536, 151936])
@pytest.mark.parametrize("kind", ["normal", "ties", "special"])
def test_argmax_rows(ctx, n, kind):
    rows = 16 if n <= 65536 else 4
    print(f"argmax n={n} rows={rows} kind={kind}", flush=True)
    v = logits_rows(n * 7 + len(kind), rows, n, kind)
    got = device_argmax(ctx, v, n, rows, n)
    want = [orc.argmax(v[r]) for r in range(rows)]
    assert got.tolist() == want


@pytest.mark.parametrize("n,ld", [(5000, 5003), (4096, 4100), (300, 301)])
def test_argmax_strided_rows(ctx, n, ld):
    # rows at a stride: odd strides take the element-wise loads
    rows = 6
    print(f"argmax strided n={n} ld={ld}", flush=True)
    full = logits_rows(n + ld, rows, ld, "ties")
    got = device_argmax(ctx, full, n, rows, ld)
    assert got.tolist() == [orc.argmax(full[r, :n]) for r in range(rows)]


def test_argmax_empty_and_repeat(ctx):
    print("argmax n=0, repeated calls", flush=True)
    ob = lh.GpuBuffer(ctx, 16)
    ob.upload(np.full(4, 0xFFFFFFFF, np.uint32).view(np.uint8))
    assert lh.dispatch_argmax(ctx, None, 0, 4, out=ob).tolist() == [0, 0, 0, 0]  # unwrap_or(0)
    v = logits_rows(77, 3, 20000, "special")
    a = device_argmax(ctx, v, 20000, 3, 20000)
    for _ in range(3):  # arrival counters are left at zero for the next call
        assert np.array_equal(device_argmax(ctx, v, 20000, 3, 20000), a)
    ob.free()


def test_lm_head_block_argmax(ctx):
    # 16 draft hidden states through the vocab-sized LM head (src/target.rs:580-605),
    # then the device argmax of each row of logits
    k, n, m = 4096, 151936, 16
    print("LM head 4096->151936 m=16 + argmax", flush=True)
    raw = synth.q4k_weight(0x5EED000B, k, n)
    x = synth.normal(0x5EED000C, m * k).reshape(m, k)
    xb, wb, cb = lh.upload_f32(ctx, x.ravel()), lh.upload_bytes(ctx, raw), lh.GpuBuffer(ctx, 4 * m * n)
    lh.dispatch_proj_quant_batch(ctx, xb, lh.F32, wb, cb, k, n, m, lh.Q4_K)
    idx = lh.dispatch_argmax(ctx, cb, n, m)
    logits = cb.read_f32(m * n).reshape(m, n)
    assert idx.tolist() == [orc.argmax(logits[r]) for r in range(m)]
    # and each is an argmax of the exact product within the products' tolerance (the
    # f64 reference for the first and last two tokens)
    rows = [0, 1, m - 2, m - 1]
    y64, a = orc.proj_quant_f64(np.ascontiguousarray(x[rows]), raw, lh.Q4_K, k, n)
    for j, r in enumerate(rows):
        assert y64[j].max() - y64[j, idx[r]] <= 2e-4 * a[j].max(), r


def test_verify_step(ctx):
    n = 151936
    print("verify step", flush=True)
    rng = np.random.default_rng(9)
    t = rng.standard_normal(n).astype(np.float32)
    d = rng.standard_normal(n).astype(np.float32)
    t[1234] = d[1234] = 50.0  # agree
    tb, db = lh.upload_f32(ctx, t), lh.upload_f32(ctx, d)
    assert lh.verify_step(ctx, db, tb, n) == (1234, True, 1234, 1234)
    d[777] = 60.0  # the draft now prefers 777: rejected, the target's token is next
    db.upload(d.view(np.uint8))
    assert lh.verify_step(ctx, db, tb, n) == (1234, False, 777, 1234)
