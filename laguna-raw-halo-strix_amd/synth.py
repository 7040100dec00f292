"""Seeded synthetic inputs for the quantized-projection workloads.

Everything is derived from SplitMix64 streams so a workload is fully named by
its seed and shape:

* uniform doubles: the top 53 bits of each SplitMix64 output;
* normals: Box-Muller on pairs of uniforms, in float64, rounded to float32;
* Q8_0 weights: float32 N(0, sigma) quantized by the ggml Q8_0 rule (32-element
  blocks, d = max|x|/127 stored as IEEE f16 with round-to-nearest-even,
  q = roundf(x * (1/d)) with the float32 1/d taken before d is stored);
* Q4_K weights: random valid super-blocks of 144 bytes, d and dmin =
  f16(U[1e-4, 4e-3]), 12 uniform random scale/min bytes (every byte pattern
  decodes to 6-bit scales and mins in [0, 63]) and 128 uniform random bytes of
  4-bit quants.

Byte layouts are GGUF's (src/gguf.rs:97,101): Q8_0 block = f16 d + 32 int8,
Q4_K super-block = f16 d, f16 dmin, 12 scale bytes, 128 quant bytes.
"""
import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
QK8_0, Q8_0_BYTES = 32, 34
QK_K, Q4_K_BYTES = 256, 144


def splitmix64(seed, count):
    """count consecutive SplitMix64 outputs for the given seed (vectorised)."""
    with np.errstate(over="ignore"):
        s = np.uint64(seed) + GOLDEN * np.arange(1, count + 1, dtype=np.uint64)
        z = s
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def uniform(seed, count):
    """Doubles in [0, 1)."""
    return (splitmix64(seed, count) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed, count, sigma=1.0):
    """float32 N(0, sigma^2) via Box-Muller in float64."""
    pairs = (count + 1) // 2
    u = uniform(seed, 2 * pairs)
    u1 = 1.0 - u[0::2]  # (0, 1]: log is finite
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * pairs, np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (z[:count] * sigma).astype(np.float32)


def random_bytes(seed, count):
    words = splitmix64(seed, (count + 7) // 8)
    return words.view(np.uint8)[:count].copy()


def _roundf(v):
    """C roundf: halves away from zero (numpy's round is half-to-even)."""
    return np.sign(v) * np.floor(np.abs(v) + np.float32(0.5))


def quantize_q8_0(x):
    """ggml Q8_0 of a float32 tensor whose size is a multiple of 32 -> raw bytes."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, QK8_0)
    amax = np.max(np.abs(x), axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    q = _roundf((x * idv[:, None]).astype(np.float32))
    q = np.clip(q, -127, 127).astype(np.int8)
    out = np.empty((x.shape[0], Q8_0_BYTES), np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.ravel()


def random_q4k(seed, n_blocks, dlo=1e-4, dhi=4e-3):
    """n_blocks random valid Q4_K super-blocks -> raw bytes (144 per block)."""
    out = random_bytes(seed, n_blocks * Q4_K_BYTES).reshape(n_blocks, Q4_K_BYTES)
    u = uniform(seed ^ 0xD1B54A32D192ED03, 2 * n_blocks).reshape(n_blocks, 2)
    dd = (dlo + (dhi - dlo) * u).astype(np.float16)
    out[:, 0:4] = dd.view(np.uint8).reshape(n_blocks, 4)
    return out.ravel()


def centered_q4k(seed, n_blocks, sigma=0.02):
    """n_blocks Q4_K super-blocks of zero-mean weights with standard deviation near
    sigma, fast (numpy's PCG64, not SplitMix64: bulk data for benchmarks): random
    nibbles q, every sub-block's scale 2 and min 15 (so w =
    d (2q - 15), zero-mean over q in 0..15, standard deviation 9.2 d), and d = dmin
    drawn per block uniform in [0.75, 1.25] sigma / 9.2."""
    rng = np.random.Generator(np.random.PCG64(seed))  # bulk bytes at memory speed
    out = rng.bit_generator.random_raw(n_blocks * Q4_K_BYTES // 8).view(np.uint8).reshape(n_blocks, Q4_K_BYTES)
    d = ((0.75 + 0.5 * rng.random(n_blocks)) * sigma / 9.2).astype(np.float16)
    out[:, 0:2] = d.view(np.uint8).reshape(n_blocks, 2)
    out[:, 2:4] = d.view(np.uint8).reshape(n_blocks, 2)
    # 6-bit (scale, min) pairs of the 8 sub-blocks: bytes 4-7 the scales of 0-3,
    # 8-11 the mins of 0-3, 12-15 the low nibbles of 4-7's scale and min
    out[:, 4:16] = np.array([2] * 4 + [15] * 4 + [2 | (15 << 4)] * 4, np.uint8)
    return out.ravel()


def q8_0_weight(seed, k, n, sigma=0.02):
    """[n rows][k] weight, GGUF layout (k contiguous per output row), as Q8_0 bytes."""
    return quantize_q8_0(normal(seed, k * n, sigma))


def q4k_weight(seed, k, n):
    assert (k * n) % QK_K == 0
    return random_q4k(seed, k * n // QK_K)


def quantize_q4k(x):
    """f32 values (a multiple of 256) -> ggml Q4_K blocks: per 32-element sub-block
    an offset m >= -min and a scale (max + m) / 15, both as 6-bit multiples of the
    super-block's f16 dmin and d; nibbles q = round((x + dmin m) / (d sc)).
    Decodes (kernels/proj_q4k.comp:46-87) to d sc q - dmin m."""
    x = np.asarray(x, np.float32).reshape(-1, 8, 32).astype(np.float64)
    nb = x.shape[0]
    mn = np.maximum(-x.min(axis=2), 0.0)                     # [nb, 8]
    sc = (x.max(axis=2) + mn) / 15.0
    d = (sc.max(axis=1) / 63.0).astype(np.float16)
    dmin = (mn.max(axis=1) / 63.0).astype(np.float16)
    d64, dm64 = d.astype(np.float64)[:, None], dmin.astype(np.float64)[:, None]
    sc6 = np.clip(np.rint(np.divide(sc, d64, out=np.zeros_like(sc), where=d64 > 0)), 0, 63).astype(np.uint32)
    m6 = np.clip(np.rint(np.divide(mn, dm64, out=np.zeros_like(mn), where=dm64 > 0)), 0, 63).astype(np.uint32)
    step = (d64 * sc6)[:, :, None]
    q = np.clip(np.rint(np.divide(x + (dm64 * m6)[:, :, None], step, out=np.zeros_like(x), where=step > 0)), 0,
                15).astype(np.uint8)
    out = np.zeros((nb, Q4_K_BYTES), np.uint8)
    out[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    out[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    sb = np.zeros((nb, 12), np.uint32)
    for j in range(4):
        sb[:, j] = sc6[:, j] & 63
        sb[:, j + 4] = m6[:, j] & 63
    for j in range(4, 8):
        sb[:, j + 4] = (sc6[:, j] & 15) | ((m6[:, j] & 15) << 4)
        sb[:, j - 4] |= (sc6[:, j] >> 4) << 6
        sb[:, j] |= (m6[:, j] >> 4) << 6
    out[:, 4:16] = sb.astype(np.uint8)
    for g in range(4):  # bytes 32g + l: low nibble element 64g + l, high nibble 64g + 32 + l
        out[:, 16 + 32 * g:48 + 32 * g] = q[:, 2 * g, :] | (q[:, 2 * g + 1, :] << 4)
    return out.ravel()


def q4k_weight_normal(seed, k, n, sigma=0.02):
    """[n rows][k] N(0, sigma) weight quantized to Q4_K (realistic magnitudes)."""
    return quantize_q4k(normal(seed, k * n, sigma))


def weight_bytes(dtype, k, n):
    from laguna_hip import Q4_K, Q8_0, F32
    if dtype == Q4_K:
        return k * n // QK_K * Q4_K_BYTES
    if dtype == Q8_0:
        return k * n // QK8_0 * Q8_0_BYTES
    if dtype == F32:
        return k * n * 4
    raise ValueError(dtype)


# ---- DFlash draft model (random init) ------------------------------------------------

DFLASH_PROJ = ("attn_q", "attn_k", "attn_v", "attn_gate", "attn_output", "ffn_gate", "ffn_up", "ffn_down")
DFLASH_NORMS = ("attn_norm", "attn_q_norm", "attn_k_norm", "ffn_norm")


def dflash_shapes(hp):
    """(k, n) of each projection of a layer (src/dflash.rs:68-79)."""
    E, QD, KVD = hp.n_embd, hp.n_heads * hp.head_dim, hp.n_kv * hp.head_dim
    return {"attn_q": (E, QD), "attn_k": (E, KVD), "attn_v": (E, KVD), "attn_gate": (E, hp.n_heads),
            "attn_output": (QD, E), "ffn_gate": (E, hp.n_ff), "ffn_up": (E, hp.n_ff), "ffn_down": (hp.n_ff, E)}


def _weight(seed, dtype, k, n):
    from laguna_hip import Q4_K, Q8_0, F32
    if dtype == Q4_K:
        return q4k_weight(seed, k, n)
    if dtype == Q8_0:
        return q8_0_weight(seed, k, n)
    if dtype == F32:
        return normal(seed, k * n, 0.02)
    raise ValueError(dtype)


def dflash_model(seed, hp, n_layers, types=None, norm_sigma=0.0, trained_scale=False):
    """Random-init draft model: (encoder dict, list of layer dicts), keys as the
    oracle's forward_block takes them.  Default types: Q4_K everywhere except
    Q8_0 attn_output.  Norm weights are 1 + N(0, norm_sigma).  Q4_K weights are
    random valid blocks (values up to a few units, far from zero-mean), or with
    trained_scale N(0, 0.02) values quantized to Q4_K."""
    from laguna_hip import Q4_K, Q8_0
    types = {**{p: Q4_K for p in DFLASH_PROJ}, "attn_output": Q8_0, "fc": Q4_K, **(types or {})}
    shapes = dflash_shapes(hp)
    sub = iter(splitmix64(seed, 64 + 16 * n_layers))

    def norm(n):
        return (1.0 + normal(int(next(sub)), n, norm_sigma)).astype(np.float32) if norm_sigma else np.ones(n, np.float32)

    def weight(s, dtype, k, n):
        return q4k_weight_normal(s, k, n) if trained_scale and dtype == Q4_K else _weight(s, dtype, k, n)

    A = hp.n_aux * hp.n_embd
    W = {"enc_aux_norm": norm(A), "fc": weight(int(next(sub)), types["fc"], A, hp.n_embd), "fc_dtype": types["fc"],
         "enc_output_norm": norm(hp.n_embd), "output_norm": norm(hp.n_embd)}
    layers = []
    for _ in range(n_layers):
        L = {"attn_norm": norm(hp.n_embd), "attn_q_norm": norm(hp.head_dim), "attn_k_norm": norm(hp.head_dim),
             "ffn_norm": norm(hp.n_embd)}
        for p in DFLASH_PROJ:
            k, n = shapes[p]
            L[p] = weight(int(next(sub)), types[p], k, n)
            L[p + "_dtype"] = types[p]
        layers.append(L)
    return W, layers


def dflash_inputs(seed, hp, n_layers, m, ctx_len):
    """features [m][n_aux*n_embd], tokens [m][n_embd], per-layer context K and V
    [ctx_len][n_kv*head_dim], all f32 N(0, 1)."""
    s = splitmix64(seed, 4 + 2 * n_layers)
    feat = normal(int(s[0]), m * hp.n_aux * hp.n_embd).reshape(m, -1)
    tok = normal(int(s[1]), m * hp.n_embd).reshape(m, -1)
    kvd = hp.n_kv * hp.head_dim
    k_ctx = [normal(int(s[4 + 2 * i]), ctx_len * kvd).reshape(ctx_len, kvd) for i in range(n_layers)]
    v_ctx = [normal(int(s[5 + 2 * i]), ctx_len * kvd).reshape(ctx_len, kvd) for i in range(n_layers)]
    return feat, tok, k_ctx, v_ctx


# ---- dense target model (random init) -------------------------------------------------

def target_model(seed, hp, types=None, gate_layers=None, n_q_heads=None, norm_sigma=0.1, output_dtype=None,
                 emb_dtype=None):
    """Random-init dense target (src/target.rs:30-43 tensors): (layers, extras).
    layers: dicts keyed as the target oracle and TargetModel take them; attn_gate
    only in gate_layers (default: every layer); n_q_heads per layer (default
    hp.n_heads).  extras: output_norm, output (+ dtype), tok_embd (+ dtype).
    Default types: Q4_K projections with a Q8_0 attn_output, Q4_K LM head, Q8_0
    embeddings; every weight is N(0, 0.02) quantized to its type."""
    from laguna_hip import Q4_K, Q8_0
    types = {**{p: Q4_K for p in DFLASH_PROJ}, "attn_output": Q8_0, **(types or {})}
    output_dtype = Q4_K if output_dtype is None else output_dtype
    emb_dtype = Q8_0 if emb_dtype is None else emb_dtype
    gate_layers = range(hp.n_layers) if gate_layers is None else gate_layers
    sub = iter(splitmix64(seed, 8 + 16 * hp.n_layers))

    def norm(n):
        return (1.0 + normal(int(next(sub)), n, norm_sigma)).astype(np.float32)

    def weight(s, dtype, k, n):  # N(0, 0.02) weights, as a trained model's are
        if dtype == Q4_K:
            return q4k_weight_normal(s, k, n)
        return _weight(s, dtype, k, n)

    E, HD, KVD = hp.n_embd, hp.head_dim, hp.n_kv * hp.head_dim
    layers = []
    for li in range(hp.n_layers):
        H = hp.n_heads if n_q_heads is None else n_q_heads[li]
        shapes = {"attn_q": (E, H * HD), "attn_k": (E, KVD), "attn_v": (E, KVD), "attn_gate": (E, H),
                  "attn_output": (H * HD, E), "ffn_gate": (E, hp.n_ff), "ffn_up": (E, hp.n_ff),
                  "ffn_down": (hp.n_ff, E)}
        L = {"attn_norm": norm(E), "attn_q_norm": norm(HD), "attn_k_norm": norm(HD), "ffn_norm": norm(E),
             "n_q_heads": H}
        for p in DFLASH_PROJ:
            k, n = shapes[p]
            s = int(next(sub))
            if p == "attn_gate" and li not in gate_layers:
                L[p], L[p + "_dtype"] = None, None
                continue
            L[p] = weight(s, types[p], k, n)
            L[p + "_dtype"] = types[p]
        layers.append(L)
    extras = {"output_norm": norm(E), "output": weight(int(next(sub)), output_dtype, E, hp.n_vocab),
              "output_dtype": output_dtype, "tok_embd": weight(int(next(sub)), emb_dtype, E, hp.n_vocab),
              "tok_embd_dtype": emb_dtype}
    return layers, extras
