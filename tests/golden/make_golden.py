"""Writes tests/golden/*.npz: small input/output vectors for the oracle.

This is an independent restatement, written from the GGUF block formats rather
than from the oracle's loops: everything is vectorised numpy over whole tensors,
the f16 fields go through numpy's IEEE binary16 decoder (with the reference's
one documented deviation for exponent-0 codes applied on top), and the Q4_K
6-bit scale/min fields are unpacked from the 96-bit field as ggml documents the
packing (sc[0..3] / m[0..3] = low 6 bits of bytes 0..3 / 4..7; sc[4..7] and
m[4..7] = low / high nibble of bytes 8..11 plus the top two bits of bytes 0..3 /
4..7).  The oracle is then checked against these files, so an indexing or
packing mistake in either implementation shows up as a mismatch.

The reference itself (Rust + GLSL) cannot be built or run in this image; the
reference's own known answers are stored too (src/dflash.rs:1334-1356,
src/lib.rs:120-165, src/gguf.rs:660-740).

Run:  python tests/golden/make_golden.py   (rewrites the .npz files)
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def ref_half(codes):
    """binary16 codes -> float32 as the reference decodes them (src/dflash.rs:314-329):
    IEEE for every code except exponent 0 with a non-zero mantissa, which the
    reference reads as 2^-14 * (1 + m/1024)."""
    codes = np.asarray(codes, np.uint16)
    out = codes.view(np.float16).astype(np.float32)
    exp = (codes >> 10) & 0x1F
    mant = (codes & 0x3FF).astype(np.float32)
    sub = (exp == 0) & (mant != 0)
    sign = np.where(codes & 0x8000, np.float32(-1), np.float32(1))
    out = np.where(sub, sign * np.float32(2.0 ** -14) * (np.float32(1) + mant / np.float32(1024)), out)
    # NaN payloads: the reference shifts the mantissa in unchanged (s | 0x7F800000 | m << 13)
    nan = (exp == 31) & (mant != 0)
    bits = ((codes.astype(np.uint32) & 0x8000) << 16) | 0x7F800000 | ((codes.astype(np.uint32) & 0x3FF) << 13)
    out = np.where(nan, bits.view(np.float32), out)
    return out.astype(np.float32)


def q8_0_decode(raw, n):
    blocks = raw.reshape(-1, 34)
    d = ref_half(blocks[:, 0:2].copy().view(np.uint16)[:, 0])
    q = blocks[:, 2:].view(np.int8).astype(np.float32)
    return (q * d[:, None]).astype(np.float32).ravel()[:n]


def q4k_unpack_scales(sc12):
    """[nb, 12] scale bytes -> (sc[nb, 8], m[nb, 8]) per the ggml K-quant packing."""
    s = sc12.astype(np.uint32)
    sc = np.empty((s.shape[0], 8), np.uint32)
    mn = np.empty((s.shape[0], 8), np.uint32)
    sc[:, 0:4] = s[:, 0:4] & 63
    mn[:, 0:4] = s[:, 4:8] & 63
    sc[:, 4:8] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:8] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, mn


def q4k_decode(raw, n):
    blocks = raw.reshape(-1, 144)
    nb = blocks.shape[0]
    d = ref_half(blocks[:, 0:2].copy().view(np.uint16)[:, 0])
    dmin = ref_half(blocks[:, 2:4].copy().view(np.uint16)[:, 0])
    sc, mn = q4k_unpack_scales(blocks[:, 4:16])
    qs = blocks[:, 16:144].reshape(nb, 4, 32)          # [block][group64][byte]
    q = np.empty((nb, 4, 2, 32), np.float32)           # [block][group][low/high][i]
    q[:, :, 0, :] = qs & 15
    q[:, :, 1, :] = qs >> 4
    q = q.reshape(nb, 8, 32)                           # sub-block j = 2*group + (high)
    a = (d[:, None] * sc.astype(np.float32)).astype(np.float32)
    b = (dmin[:, None] * mn.astype(np.float32)).astype(np.float32)
    w = (a[:, :, None] * q).astype(np.float32) - b[:, :, None]
    return w.astype(np.float32).ravel()[:n]


def legacy_q4k_closed_forms():
    """src/dflash.rs:398-436 on hand-built blocks: bf16 d = 1.0, k4 = 0.5, signs < 0
    selects -k4; even i reads bits 4-6 of byte 6+i/2, odd i bits 0-2."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([0x3F80], np.uint16).view(np.uint8)  # bf16 1.0
    blk[2:4] = np.array([0x3F00], np.uint16).view(np.uint8)  # bf16 0.5
    blk[4:6] = np.array([0xBF80], np.uint16).view(np.uint8)  # bf16 -1.0 -> s = -1
    t = np.arange(128)
    blk[6:134] = ((t % 8) << 4) | (7 - t % 8)                # byte 6+t: high bits t%8, low 7-t%8
    out = np.empty(256, np.float32)
    out[0::2] = (t % 8) - 0.5                                 # element 2t: (byte >> 4) & 7 = t%8
    out[1::2] = (7 - t % 8) - 0.5                             # element 2t+1: byte & 7
    return blk, out


def main():
    rng = np.random.default_rng(20261201)

    # ---- f16 decode of every code
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    half_bits = ref_half(codes).view(np.uint32)

    # ---- Q8_0: random blocks plus special scales (d = 1, min normal, max, subnormal quirk, +-0)
    nb8 = 40
    raw8 = rng.integers(0, 256, size=(nb8, 34), dtype=np.uint8)
    special_d = [0x3C00, 0x0400, 0x7BFF, 0x0001, 0x03FF, 0x8000, 0x0000, 0xBC00]
    for i, h in enumerate(special_d):
        raw8[i, 0:2] = np.array([h], np.uint16).view(np.uint8)
    for i in range(len(special_d), nb8):  # realistic scales
        raw8[i, 0:2] = np.array([rng.uniform(1e-4, 4e-3)], np.float16).view(np.uint8)
    raw8[0, 2:] = np.array([-128, -1, 0, 1, 127] * 6 + [5, -5], np.int8).view(np.uint8)
    raw8 = raw8.ravel()
    n8 = nb8 * 32 - 7  # ragged tail
    deq8 = q8_0_decode(raw8, n8)

    # ---- Q4_K: random blocks plus special headers
    nb4 = 24
    raw4 = rng.integers(0, 256, size=(nb4, 144), dtype=np.uint8)
    for i in range(nb4):
        dd = rng.uniform(1e-4, 4e-3, size=2).astype(np.float16)
        raw4[i, 0:4] = dd.view(np.uint8)
    raw4[0, 0:4] = np.array([0x3C00, 0x0000], np.uint16).view(np.uint8)  # d=1, dmin=0
    raw4[1, 0:4] = np.array([0x0001, 0x03FF], np.uint16).view(np.uint8)  # subnormal quirk on both
    raw4[2, 0:4] = np.array([0x3C00, 0x3C00], np.uint16).view(np.uint8)
    raw4[2, 4:16] = 0xFF                                                  # every scale/min = 63
    raw4 = raw4.ravel()
    n4 = nb4 * 256 - 100
    deq4 = q4k_decode(raw4, n4)

    # ---- matvec: f64 accumulation of the decoded weights
    k4, n4r = 512, 6
    w4 = raw4[: n4r * k4 // 256 * 144]
    x4 = rng.standard_normal(k4).astype(np.float32)
    W4 = q4k_decode(w4, n4r * k4).reshape(n4r, k4).astype(np.float64)
    y4 = W4 @ x4.astype(np.float64)
    a4 = np.abs(W4 * x4.astype(np.float64)).sum(axis=1)

    k8, n8r = 256, 5
    w8 = raw8[: n8r * k8 // 32 * 34]
    x8 = rng.standard_normal(k8).astype(np.float32)
    W8 = q8_0_decode(w8, n8r * k8).reshape(n8r, k8).astype(np.float64)
    y8 = W8 @ x8.astype(np.float64)
    a8 = np.abs(W8 * x8.astype(np.float64)).sum(axis=1)

    # ---- reference known answers
    a = np.arange(8, dtype=np.float32) * np.float32(0.1)     # src/lib.rs:123
    b = np.arange(24, dtype=np.float32) * np.float32(0.01)   # src/lib.rs:124
    mm_expected = np.array([sum(np.float64(a[i]) * np.float64(b[j * 8 + i]) for i in range(8)) for j in range(3)])

    leg_blk, leg_out = legacy_q4k_closed_forms()

    np.savez_compressed(os.path.join(HERE, "golden.npz"),
             half_bits=half_bits,
             q8_raw=raw8, q8_n=np.int64(n8), q8_deq=deq8,
             q4_raw=raw4, q4_n=np.int64(n4), q4_deq=deq4,
             mv4_k=np.int64(k4), mv4_n=np.int64(n4r), mv4_x=x4, mv4_y=y4, mv4_abs=a4,
             mv8_k=np.int64(k8), mv8_n=np.int64(n8r), mv8_x=x8, mv8_y=y8, mv8_abs=a8,
             mm_a=a, mm_b=b, mm_expected=mm_expected,
             legacy_blk=leg_blk, legacy_out=leg_out)
    print("wrote", os.path.join(HERE, "golden.npz"))


if __name__ == "__main__":
    main()
