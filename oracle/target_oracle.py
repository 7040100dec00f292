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

The MoE FFN of TargetModel::dispatch_moe_ffn (src/target.rs:607-748) is moe_ffn
below, pinned in tests/test_moe_oracle.py.

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


# ---- MoE FFN (src/target.rs:607-748) ---------------------------------------------------

F16_SAFE = 32768.0             # src/target.rs:699: the expert hidden is scaled to this L2 norm
MOE_NORM_MIN = 6.103515625e-5  # src/target.rs:666: floor of the selected scores' sum
MOE_TENSORS = ("ffn_gate_inp", "ffn_gate_exps", "ffn_up_exps", "ffn_down_exps", "ffn_gate_shexp", "ffn_up_shexp",
               "ffn_down_shexp")


def expert_offset(e, n_embd, n_ff_exp):
    """src/target.rs:684,687: the expert's first element, cast to u32 as there."""
    return (e * n_embd * n_ff_exp) & 0xFFFFFFFF


def proj_expert(x64, raw, dtype, k, n, elem_offset=0):
    """dispatch_proj_quant_expert in float64: the element offset moves the weights for
    Q4_K only; Q8_0 and F32 ignore it (src/target.rs:1115-1138).  Returns (y, absdot)."""
    if dtype == orc.F32:
        w = np.ascontiguousarray(raw, np.float32).view(np.uint8).ravel()
    else:
        w = np.frombuffer(raw, np.uint8) if isinstance(raw, (bytes, bytearray)) else np.asarray(raw, np.uint8)
        if dtype == orc.Q4_K and elem_offset:
            assert elem_offset % 256 == 0
            w = w[elem_offset // 256 * 144:]
    return orc.proj_quant_f64x(x64, w, dtype, k, n)


def moe_ffn(norm_x, w, bias, n_embd, n_expert, n_expert_used, n_ff_exp, n_shexp, expert_weights_norm=False,
            expert_weights_scale=1.0):
    """TargetModel::dispatch_moe_ffn (src/target.rs:607-748) in float64.

    w maps each name of MOE_TENSORS to (raw, dtype); bias is exp_probs_b (n_expert f32).
    Router logits, sigmoid probabilities, selection by probability + bias (a stable
    descending sort, the first n_expert_used), scores = the selected probabilities,
    divided by max(their sum, 2^-14) when expert_weights_norm, times expert_weights_scale
    unless it is 0 or 1.  Each selected expert: h = silu(gate x) * (up x), the down
    projection of h * 32768 / ||h|| (||h|| clamped to [1e-8, 1e30]), multiplied back by
    ||h|| / 32768 * score only when score > 0 (the reference adds it unscaled otherwise);
    then the shared expert's FFN.  Returns (out, absdot, selected, scores), absdot the sum
    of |term| over every product that reaches out."""
    x64 = np.asarray(norm_x, np.float32).astype(np.float64)
    logits, _ = proj_expert(x64, *w["ffn_gate_inp"], n_embd, n_expert)
    probs = 1.0 / (1.0 + np.exp(-logits))
    sel = probs + np.asarray(bias, np.float32).astype(np.float64)
    chosen = [int(i) for i in np.argsort(-sel, kind="stable")[:n_expert_used]]
    scores = probs[chosen].copy()
    if expert_weights_norm:
        scores = scores / max(float(scores.sum()), MOE_NORM_MIN)
    if expert_weights_scale != 0.0 and expert_weights_scale != 1.0:
        scores = scores * expert_weights_scale
    out = np.zeros(n_embd)
    absdot = np.zeros(n_embd)
    for e, sc in zip(chosen, scores):
        off = expert_offset(e, n_embd, n_ff_exp)
        g, _ = proj_expert(x64, *w["ffn_gate_exps"], n_embd, n_ff_exp, off)
        u, _ = proj_expert(x64, *w["ffn_up_exps"], n_embd, n_ff_exp, off)
        h = g / (1.0 + np.exp(-g)) * u
        col_l2 = min(max(float(np.sqrt(np.sum(h * h))), 1e-8), 1e30)
        d, a = proj_expert(h * F16_SAFE / col_l2, *w["ffn_down_exps"], n_ff_exp, n_embd, off)
        f = col_l2 / F16_SAFE * sc if sc > 0.0 else 1.0
        out += f * d
        absdot += abs(f) * a
    g, _ = proj_expert(x64, *w["ffn_gate_shexp"], n_embd, n_shexp)
    u, _ = proj_expert(x64, *w["ffn_up_shexp"], n_embd, n_shexp)
    d, a = proj_expert(g / (1.0 + np.exp(-g)) * u, *w["ffn_down_shexp"], n_shexp, n_embd)
    return out + d, absdot + a, chosen, scores
