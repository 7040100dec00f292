"""f64 restatement of the DFlash draft forward -- TEST INFRASTRUCTURE ONLY.

Only the tests, the smoke check and the benchmark's CPU-baseline leg use this
module, as the checker.  Every op follows the reference shader or host code it
names (paths relative to the reference repository root), computed in float64 on
the exactly dequantized weights (the C oracle's decoders).

The block forward generalises DFlashModel::forward_injected_decode_hidden
(src/dflash.rs:877-976) from one token to a block of M tokens over C cached
context positions:

* the encoder (src/dflash.rs:157-234) runs on each of the M feature rows;
* per layer, the sequence the queries attend to is
      [context K/V (positions 0..C-1)] ++ [injected K/V of the M encoder rows
      (positions C..C+M-1)] ++ [K/V of the M tokens (positions C+M..C+2M-1)];
  injected keys are roped at their positions, token queries and keys at theirs;
* query t attends causally (mha_attn.comp with causal = 1) with q_pos = C+M+t,
  i.e. to the whole context, every injected entry and tokens 0..t.
With M = 1 and C = 0 this is the reference exactly: sequence [injected (pos 0),
token (pos 1)], seq_len 2, q_pos 1 (src/dflash.rs:945-954).

Pinning (tests/test_dflash_oracle.py): closed forms per op (constant vectors
through RMSNorm, zero rotation at pos 0, norm preservation and an exact quarter
turn of RoPE, one-key and equal-score attention, the softplus threshold), the
reference's own constants (eps 1e-5 / 1e-6, theta 5e5, threshold 20, scale
1/sqrt(head_dim)), and the composite against closed forms -- zero attention
output and FFN down weights leave rmsnorm(token) * output_norm; zero attention
norm weights make every score equal, so each token averages the context values
over exactly the positions it may see, times softplus(0) -- and against a
loop-by-loop restatement at a tiny size.  No reference test or fixture covers
these ops: beyond those checks their parity is unpinned.
"""
import numpy as np

import oracle as orc

RMS_EPS = 1e-5       # src/dflash.rs:987 (dispatch_rmsnorm), :162 (encode)
QK_EPS = 1e-6        # src/dflash.rs:1105 (dispatch_qk_norm_rope)
SOFTPLUS_T = 20.0    # src/dflash.rs:957


def rmsnorm(x, w, eps=RMS_EPS):
    """kernels/rmsnorm.comp:23-34 per row: y = x * w * (mean(x^2) + eps)^-1/2."""
    x = np.asarray(x, np.float64)
    ms = np.mean(x * x, axis=-1, keepdims=True)
    return x * np.asarray(w, np.float64) / np.sqrt(ms + eps)


def enc_aux_norm(x, w, n_feat, n_aux, eps=RMS_EPS):
    """kernels/enc_aux_norm.comp:21-43: RMSNorm of each n_feat chunk of a token's
    n_aux*n_feat features, times w[aux*n_feat + feat]."""
    x = np.asarray(x, np.float64).reshape(-1, n_aux, n_feat)
    ms = np.mean(x * x, axis=-1, keepdims=True)
    y = x / np.sqrt(ms + eps) * np.asarray(w, np.float64).reshape(1, n_aux, n_feat)
    return y.reshape(-1, n_aux * n_feat)


def rope_freq(rope_dim, base=500000.0):
    """src/dflash.rs:898-904: freq[i] = 1 / base^(2i/rope_dim), computed in f32 on
    the host and uploaded; the kernels and this oracle use the same f32 table."""
    i = np.arange(rope_dim // 2, dtype=np.float32)
    return (np.float32(1.0) / np.power(np.float32(base), (np.float32(2.0) * i) / np.float32(rope_dim))).astype(np.float32)


def qk_norm_rope(x, w, freq, pos, n_heads, head_dim, rope_dim, eps=QK_EPS):
    """kernels/qk_norm_rope.comp:23-67 for rows x[r] at positions pos[r]: per-head
    RMSNorm times w[dim], then GPT-NeoX rotation of dims < rope_dim with partner
    dim +- head_dim/2 and angle = freq[dim % (rope_dim/2)] * pos (f32 product).
    Only rope_dim == head_dim (the draft model) or 0 is defined: for a smaller
    rope_dim the shader's second-half partner index (i - head_dim/2, :58-60) falls
    into the previous head, or before the buffer for head 0."""
    assert rope_dim in (0, head_dim), "partial rotary is undefined in the reference shader"
    x = np.asarray(x, np.float64).reshape(-1, n_heads, head_dim)
    pos = np.asarray(pos).reshape(-1)
    ms = np.mean(x * x, axis=-1, keepdims=True)
    nrm = x * np.asarray(w, np.float64) / np.sqrt(ms + eps)
    y = nrm.copy()
    half = rope_dim // 2
    hd2 = head_dim // 2
    for r in range(x.shape[0]):
        ang = (freq.astype(np.float32) * np.float32(pos[r])).astype(np.float64)  # f32 angle
        c, s = np.cos(ang), np.sin(ang)
        for d in range(rope_dim):
            hf = d % half
            if d < half:
                y[r, :, d] = nrm[r, :, d] * c[hf] - nrm[r, :, d + hd2] * s[hf]
            else:
                y[r, :, d] = nrm[r, :, d] * c[hf] + nrm[r, :, d - hd2] * s[hf]
    return y.reshape(-1, n_heads * head_dim)


def attention(q, K, V, q_pos, n_q, n_kv, head_dim, causal=True):
    """kernels/mha_attn.comp:28-72: for each query row r and head h, softmax over
    positions p <= q_pos[r] (causal) of (q . K[p, kv_h]) / sqrt(head_dim), with
    kv_h = h * n_kv / n_q, applied to V.  q: [R][n_q*hd], K, V: [S][n_kv*hd]."""
    q = np.asarray(q, np.float64).reshape(-1, n_q, head_dim)
    K = np.asarray(K, np.float64).reshape(-1, n_kv, head_dim)
    V = np.asarray(V, np.float64).reshape(-1, n_kv, head_dim)
    scale = 1.0 / np.sqrt(head_dim)  # src/dflash.rs:1173 (f32 there)
    out = np.zeros_like(q)
    for r in range(q.shape[0]):
        n = q_pos[r] + 1 if causal else K.shape[0]
        for h in range(n_q):
            kh = h * n_kv // n_q
            s = K[:n, kh, :] @ q[r, h] * scale
            s = np.exp(s - s.max())
            out[r, h] = (s / s.sum()) @ V[:n, kh, :]
    return out.reshape(-1, n_q * head_dim)


def softplus_gate(g):
    """src/dflash.rs:957: g > 20 ? g : ln(1 + e^g)."""
    g = np.asarray(g, np.float64)
    return np.where(g > SOFTPLUS_T, g, np.log1p(np.exp(np.minimum(g, SOFTPLUS_T))))


def gate_mul(attn, gate, n_heads, head_dim):
    """kernels/gate_mul.comp:21-30: attn[i] * gate[i / head_dim] per row."""
    a = np.asarray(attn, np.float64).reshape(-1, n_heads, head_dim)
    return (a * np.asarray(gate, np.float64).reshape(-1, n_heads, 1)).reshape(-1, n_heads * head_dim)


def silu_mul(g, u):
    """kernels/activation.comp:21-28 in f64."""
    g = np.asarray(g, np.float64)
    return g * (0.5 + 0.5 * np.tanh(0.5 * g)) * np.asarray(u, np.float64)  # g * sigmoid(g), no overflow


def weight_f64(raw, dtype, k, n):
    """[n][k] dequantized weight (ggml Q4_K of kernels/proj_q4k.comp, Q8_0, or f32)."""
    if dtype == orc.F32:
        return np.asarray(raw, np.float32).reshape(n, k).astype(np.float64)
    return orc.dequant(raw, dtype, k * n).reshape(n, k).astype(np.float64)


def proj(x, raw, dtype, k, n):
    """c[r][i] = sum_j x[r][j] * W[i,j] (proj.comp / proj_q4k.comp / proj_q8_0.comp
    semantics, GGUF layout) in f64."""
    W = weight_f64(raw, dtype, k, n)
    return np.asarray(x, np.float64).reshape(-1, k) @ W.T


class Hparams:
    def __init__(self, n_embd=4096, n_heads=32, n_kv=8, head_dim=128, rope_dim=128, n_ff=14336, n_aux=3,
                 rope_base=500000.0):
        self.n_embd, self.n_heads, self.n_kv, self.head_dim = n_embd, n_heads, n_kv, head_dim
        self.rope_dim, self.n_ff, self.n_aux, self.rope_base = rope_dim, n_ff, n_aux, rope_base


def encode(feat, W, hp):
    """DFlashModel::encode (src/dflash.rs:157-234) per feature row."""
    h = enc_aux_norm(feat, W["enc_aux_norm"], hp.n_embd, hp.n_aux)
    h = proj(h, W["fc"], W["fc_dtype"], hp.n_aux * hp.n_embd, hp.n_embd)
    return rmsnorm(h, W["enc_output_norm"])


def forward_block(feat, tok, W, layers, k_ctx, v_ctx, ctx_len, hp):
    """Block forward (module docstring).  feat: [M][n_aux*n_embd], tok: [M][n_embd],
    layers: list of per-layer dicts (raw weights + dtypes), k_ctx/v_ctx: per layer
    [ctx_len][n_kv*head_dim] (keys already normed and roped).  Returns the final
    hidden [M][n_embd] (after output_norm when W has one)."""
    M = np.asarray(tok).reshape(-1, hp.n_embd).shape[0]
    C = ctx_len
    E, H, KV, HD, FF = hp.n_embd, hp.n_heads, hp.n_kv, hp.head_dim, hp.n_ff
    freq = rope_freq(hp.rope_dim, hp.rope_base)
    enc = encode(feat, W, hp)
    x = np.asarray(tok, np.float64).reshape(M, E).copy()
    pos_inj = np.arange(C, C + M)
    pos_tok = np.arange(C + M, C + 2 * M)
    for li, L in enumerate(layers):
        en = rmsnorm(enc, L["attn_norm"])
        k_inj = proj(en, L["attn_k"], L["attn_k_dtype"], E, KV * HD)
        v_inj = proj(en, L["attn_v"], L["attn_v_dtype"], E, KV * HD)
        k_inj = qk_norm_rope(k_inj, L["attn_k_norm"], freq, pos_inj, KV, HD, hp.rope_dim)
        nx = rmsnorm(x, L["attn_norm"])
        q = proj(nx, L["attn_q"], L["attn_q_dtype"], E, H * HD)
        k = proj(nx, L["attn_k"], L["attn_k_dtype"], E, KV * HD)
        v = proj(nx, L["attn_v"], L["attn_v_dtype"], E, KV * HD)
        q = qk_norm_rope(q, L["attn_q_norm"], freq, pos_tok, H, HD, hp.rope_dim)
        k = qk_norm_rope(k, L["attn_k_norm"], freq, pos_tok, KV, HD, hp.rope_dim)
        K = np.concatenate([np.asarray(k_ctx[li], np.float64).reshape(C, KV * HD), k_inj, k])
        V = np.concatenate([np.asarray(v_ctx[li], np.float64).reshape(C, KV * HD), v_inj, v])
        a = attention(q, K, V, pos_tok, H, KV, HD)
        g = softplus_gate(proj(nx, L["attn_gate"], L["attn_gate_dtype"], E, H))
        a = gate_mul(a, g, H, HD)
        x = x + proj(a, L["attn_output"], L["attn_output_dtype"], H * HD, E)
        h = rmsnorm(x, L["ffn_norm"])
        f = silu_mul(proj(h, L["ffn_gate"], L["ffn_gate_dtype"], E, FF), proj(h, L["ffn_up"], L["ffn_up_dtype"], E, FF))
        x = x + proj(f, L["ffn_down"], L["ffn_down_dtype"], FF, E)
    if W.get("output_norm") is not None:
        x = rmsnorm(x, W["output_norm"])
    return x
