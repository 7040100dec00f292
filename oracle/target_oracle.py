"""f64 restatement of the dense target forward and the verify loop -- TEST
INFRASTRUCTURE ONLY.

Only the tests and the smoke check use this module, as the checker.  It follows
TargetModel::forward_token_impl (src/target.rs:314-578) for dense layers, op by
op, in float64 on the exactly dequantized weights, reusing the draft oracle's ops
(rmsnorm.comp, qk_norm_rope.comp, mha_attn.comp, activation.comp, proj*.comp),
plus kernels/gate_attn.comp, and run_target_dflash_verify (src/lib.rs:466-520).

The reference's constants: RMSNorm eps 1e-5 (src/target.rs:970), QK-norm eps 1e-6
(:897, :936), RoPE bases 500000 and 10000 for the sliding-window table
(:352, :367), SWA layers are those with index % 4 != 0 (:440), attention scale
1/sqrt(head_dim) (:776).

Pinning (tests/test_target_oracle.py): closed forms of the composite (zero
attention output and FFN down weights leave logits = W_out rmsnorm(input) *
output_norm; one-position attention returns V, so the logits do not depend on the
query weights; a constant-V cache gives the same output at every position), the
capture order against the reference's rule, the cache against the uncached forward
at position 0, and gate_attn's formula at its special values.  No reference test
or fixture covers the target forward: beyond those checks its parity is unpinned.
"""
import numpy as np

import dflash_oracle as dfo
import oracle as orc

RMS_EPS = 1e-5         # src/target.rs:970
QK_EPS = 1e-6          # src/target.rs:897
ROPE_BASE = 500000.0   # src/target.rs:352
ROPE_BASE_SWA = 10000.0  # src/target.rs:367

PROJ = ("attn_q", "attn_k", "attn_v", "attn_gate", "attn_output", "ffn_gate", "ffn_up", "ffn_down")
NORMS = ("attn_norm", "attn_q_norm", "attn_k_norm", "ffn_norm")


class Hparams:
    """Dense target hyperparameters (Model::from_reader, src/model.rs:29-129)."""

    def __init__(self, n_embd, n_heads, n_kv, head_dim, n_ff, n_layers, n_vocab, rope_dim, rope_dim_swa=0,
                 swa=False, rope_base=ROPE_BASE, rope_base_swa=ROPE_BASE_SWA):
        self.n_embd, self.n_heads, self.n_kv, self.head_dim = n_embd, n_heads, n_kv, head_dim
        self.n_ff, self.n_layers, self.n_vocab = n_ff, n_layers, n_vocab
        self.rope_dim, self.rope_dim_swa, self.swa = rope_dim, rope_dim_swa, swa
        self.rope_base, self.rope_base_swa = rope_base, rope_base_swa


class KvCache:
    """TargetKvCache (src/target.rs:74-101): per layer, the normed and roped keys and
    the raw values of the cached positions."""

    def __init__(self, n_layers):
        self.k = [[] for _ in range(n_layers)]
        self.v = [[] for _ in range(n_layers)]
        self.len = 0


def gate_attn(attn, gate, n_heads, head_dim):
    """kernels/gate_attn.comp:21-30: attn[i] * log(1 + exp(gate[i / head_dim])), no
    threshold (in f32 the factor is infinite above about 88.7; here near 709)."""
    g = np.log1p(np.exp(np.asarray(gate, np.float64)))
    return (np.asarray(attn, np.float64).reshape(n_heads, head_dim) * g.reshape(n_heads, 1)).ravel()


def capture_order(n_layers, layer_indices):
    """The states forward_token returns (src/target.rs:391-395, 558-560): the input
    of every layer when layer_indices is None, else of each listed layer in
    ascending layer order, then the final state if n_layers is listed."""
    if layer_indices is None:
        return list(range(n_layers))
    want = set(int(i) for i in layer_indices)
    return [l for l in range(n_layers + 1) if l in want]


def forward_token(inp, layers, hp, output_norm=None, output=None, output_dtype=None, layer_indices=None,
                  cache=None):
    """TargetModel::forward_token(_cached) (src/target.rs:298-578), dense layers.
    layers: dicts with the f32 norms of NORMS, raw projection bytes p and p + "_dtype"
    for p in PROJ (attn_gate may be None) and optionally "n_q_heads".
    Returns (logits, [captured states]); logits are the normed final state when
    there is no output weight."""
    E, KV, HD, FF = hp.n_embd, hp.n_kv, hp.head_dim, hp.n_ff
    KVD = KV * HD
    pos = cache.len if cache is not None else 0
    x = np.asarray(inp, np.float64).reshape(E).copy()
    cap = set(capture_order(hp.n_layers, layer_indices))
    captured = []
    freq = dfo.rope_freq(hp.rope_dim, hp.rope_base)
    freq_swa = dfo.rope_freq(hp.rope_dim_swa, hp.rope_base_swa)
    for li, L in enumerate(layers):
        if li in cap:
            captured.append(x.copy())
        H = L.get("n_q_heads", hp.n_heads)
        QD = H * HD
        nx = dfo.rmsnorm(x, L["attn_norm"], RMS_EPS)
        q = dfo.proj(nx, L["attn_q"], L["attn_q_dtype"], E, QD)[0]
        k = dfo.proj(nx, L["attn_k"], L["attn_k_dtype"], E, KVD)[0]
        v = dfo.proj(nx, L["attn_v"], L["attn_v_dtype"], E, KVD)[0]
        swa = hp.swa and li % 4 != 0
        f, rd = (freq_swa, hp.rope_dim_swa) if swa else (freq, hp.rope_dim)
        q = dfo.qk_norm_rope(q, L["attn_q_norm"], f, [pos], H, HD, rd, QK_EPS)[0]
        k = dfo.qk_norm_rope(k, L["attn_k_norm"], f, [pos], KV, HD, rd, QK_EPS)[0]
        if cache is not None:
            cache.k[li].append(k)
            cache.v[li].append(v)
            K, V = np.stack(cache.k[li]), np.stack(cache.v[li])
            a = dfo.attention(q, K, V, [K.shape[0] - 1], H, KV, HD)[0]
        else:
            a = dfo.attention(q, k.reshape(1, KVD), v.reshape(1, KVD), [0], H, KV, HD)[0]
        if L.get("attn_gate") is not None:
            g = dfo.proj(nx, L["attn_gate"], L["attn_gate_dtype"], E, H)[0]
            a = gate_attn(a, g, H, HD)
        x = x + dfo.proj(a, L["attn_output"], L["attn_output_dtype"], QD, E)[0]
        h = dfo.rmsnorm(x, L["ffn_norm"], RMS_EPS)
        act = dfo.silu_mul(dfo.proj(h, L["ffn_gate"], L["ffn_gate_dtype"], E, FF)[0],
                           dfo.proj(h, L["ffn_up"], L["ffn_up_dtype"], E, FF)[0])
        x = x + dfo.proj(act, L["ffn_down"], L["ffn_down_dtype"], FF, E)[0]
    if hp.n_layers in cap and layer_indices is not None:
        captured.append(x.copy())
    if cache is not None:
        cache.len += 1
    if output_norm is not None:
        x = dfo.rmsnorm(x, output_norm, RMS_EPS)
    if output is None:
        return x, captured
    return dfo.proj(x, output, output_dtype, E, hp.n_vocab)[0], captured


def token_embedding(raw, dtype, n_embd, token):
    """target_token_embedding (src/lib.rs:431-454): row `token` of the dequantized
    token_embd tensor.  The reference decodes with dequant_to_f32, whose Q4_K branch
    is its legacy non-ggml decode (src/dflash.rs:398-436); Q4_K rows here, as on the
    device, are ggml blocks (the decode of kernels/proj_q4k.comp)."""
    n = (token + 1) * n_embd
    b = np.ascontiguousarray(raw).view(np.uint8).ravel()  # the tensor's bytes, whatever the array type
    return orc.dequant(b, dtype, n)[token * n_embd:n].astype(np.float32)
