// Dense target forward with hidden-state capture: TargetModel::forward_token and
// forward_token_cached (src/target.rs:298-578), dense layers only.
//
// One token per call, every tensor resident on the device.  Per layer
// (src/target.rs:401-556): RMSNorm, the Q/K/V (and attention-gate) projections
// of the raw GGUF blocks through the M = 1 kernels, QK-norm + NeoX RoPE at the
// token's position (the sliding-window table on SWA layers), attention over the
// token itself or the device-resident cache, the gate, the output projection and
// residual, RMSNorm, and the SwiGLU FFN (the SiLU fused into the Q4_K down
// projection) and residual.  Hidden states are captured on the device as
// they enter the selected layers.  The reference's host round trips (reading
// the captured states, re-uploading the whole K/V cache every token) become
// device copies; its per-call buffers become one workspace per stream.
#include <cstring>

#include "lg_common.hpp"

namespace {

using namespace lg;

constexpr uint32_t TABLE_FLOATS = 128;  // rope_dim <= head_dim <= 256

struct TgtLayout {
    float *x, *nx, *q, *k, *v, *att, *gate, *g, *u, *o, *freq, *freq_swa, *part, *x2;
    uint64_t total;
};

uint64_t max_q_dim(const lg_target_model *md) {
    uint64_t m = 0;
    for (uint32_t l = 0; l < md->hp.n_layers; l++) m = md->layers[l].n_q_heads > m ? md->layers[l].n_q_heads : m;
    return m;
}

uint64_t layout(const lg_target_model *md, uint32_t seq_len, uint8_t *base, TgtLayout &L) {
    const lg_target_hparams &hp = md->hp;
    const uint64_t E = hp.n_embd, H = max_q_dim(md), QD = H * hp.head_dim, KVD = (uint64_t)hp.n_kv_heads * hp.head_dim;
    const uint64_t FF = hp.n_ff;
    const uint64_t floats[] = {E, E, QD, KVD, KVD, QD, H, FF, FF, E, TABLE_FLOATS, TABLE_FLOATS,
                               glue_attn_partial_bytes(seq_len, hp.n_kv_heads) / 4, E};
    float **dst[] = {&L.x, &L.nx, &L.q, &L.k, &L.v, &L.att, &L.gate, &L.g, &L.u, &L.o, &L.freq, &L.freq_swa, &L.part,
                     &L.x2};
    // the two RoPE tables first, at fixed offsets whatever seq_len is, so that an
    // uploaded table stays valid across calls
    uint64_t off = 0;
    const int order[] = {10, 11, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 13, 12};
    for (int i : order) {
        *dst[i] = reinterpret_cast<float *>(base + off);
        off += (floats[i] * 4 + 255) & ~(uint64_t)255;
    }
    L.total = off;
    return off;
}

// A table's identity: (rope_dim, bits of base).
uint64_t table_tag(uint32_t rope_dim, float base) {
    uint32_t b = 0;
    std::memcpy(&b, &base, 4);
    return (uint64_t)rope_dim << 32 | b;
}

float base_or(float b, float dflt) { return b > 0.0f ? b : dflt; }

// Both RoPE tables of the reference (src/target.rs:343-376) at L.freq / L.freq_swa,
// uploaded unless the buffer's tags say they already are.
int upload_tables(uint64_t (&tag)[2], const lg_target_hparams &hp, const TgtLayout &L, hipStream_t s) {
    const float base = base_or(hp.rope_base, 500000.0f), base_swa = base_or(hp.rope_base_swa, 10000.0f);
    const uint64_t t0 = table_tag(hp.rope_dim, base), t1 = table_tag(hp.swa ? hp.rope_dim_swa : 0, base_swa);
    if (tag[0] == t0 && tag[1] == t1) return LG_OK;
    {  // a new table is a host copy and a synchronise, which a capturing stream cannot take
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        LG_HIP_TRY(hipStreamIsCapturing(s, &cs));
        LG_REQUIRE(cs == hipStreamCaptureStatusNone, "the RoPE table of this model cannot be uploaded while the stream "
                   "is being captured; make the same call once before capturing");
    }
    float f[2 * TABLE_FLOATS] = {0.0f};
    glue_rope_table(hp.rope_dim, base, f);
    if (hp.swa) glue_rope_table(hp.rope_dim_swa, base_swa, f + TABLE_FLOATS);
    LG_HIP_TRY(hipMemcpyAsync(L.freq, f, TABLE_FLOATS * 4, hipMemcpyHostToDevice, s));
    LG_HIP_TRY(hipMemcpyAsync(L.freq_swa, f + TABLE_FLOATS, TABLE_FLOATS * 4, hipMemcpyHostToDevice, s));
    LG_HIP_TRY(hipStreamSynchronize(s));  // f is released on return
    tag[0] = t0;
    tag[1] = t1;
    return LG_OK;
}

// The workspace of stream s laid out for seq_len positions, tables uploaded.  The
// lease (and with it the registry lock, which the products take too) ends on return;
// eager calls on one stream are ordered by the caller and calls on different streams
// never share the buffer.
int eager_ws(const lg_target_model *md, uint32_t seq_len, TgtLayout &L, hipStream_t s) {
    BufLease lease;
    LG_TRY(stream_buffer(BUF_TARGET, s, layout(md, seq_len, nullptr, L), lease, "target forward"));
    layout(md, seq_len, static_cast<uint8_t *>(lease.buf->ptr), L);
    return upload_tables(lease.buf->tag, md->hp, L, s);
}

bool proj_type_ok(int t) { return t == LG_F32 || t == LG_Q8_0 || t == LG_Q4_K; }

int check_model(const lg_target_model *md, const char *name) {
    LG_REQUIRE(md, "%s: null model", name);
    const lg_target_hparams &hp = md->hp;
    LG_REQUIRE(md->layers && hp.n_layers, "%s: no layers", name);
    LG_REQUIRE(hp.n_embd && hp.n_kv_heads && hp.head_dim && hp.n_ff, "%s: zero hyperparameter", name);
    const uint32_t rd_swa = hp.swa ? hp.rope_dim_swa : 0;
    LG_REQUIRE(hp.head_dim <= 256 && hp.head_dim % 2 == 0 && (hp.rope_dim == 0 || hp.rope_dim == hp.head_dim) &&
                   (rd_swa == 0 || rd_swa == hp.head_dim),
               "%s: head_dim %u / rope_dim %u / rope_dim_swa %u unsupported (a rope dimension must be 0 or head_dim)",
               name, hp.head_dim, hp.rope_dim, rd_swa);
    LG_REQUIRE(!md->output || (hp.n_vocab && proj_type_ok(md->output_type)), "%s: output weight needs n_vocab and a "
               "type of F32, Q8_0 or Q4_K", name);
    for (uint32_t l = 0; l < hp.n_layers; l++) {
        const lg_target_layer &L = md->layers[l];
        LG_REQUIRE(L.attn_norm && L.attn_q_norm && L.attn_k_norm && L.ffn_norm && L.attn_q && L.attn_k && L.attn_v &&
                       L.attn_output && L.ffn_gate && L.ffn_up && L.ffn_down,
                   "%s: layer %u is missing a tensor", name, l);
        LG_REQUIRE(L.n_q_heads && L.n_q_heads % hp.n_kv_heads == 0, "%s: layer %u has %u query heads for %u KV heads",
                   name, l, L.n_q_heads, hp.n_kv_heads);
        const int types[] = {L.attn_q_type, L.attn_k_type, L.attn_v_type, L.attn_output_type, L.ffn_gate_type,
                             L.ffn_up_type, L.ffn_down_type, L.attn_gate ? L.attn_gate_type : LG_F32};
        for (int t : types) LG_REQUIRE(proj_type_ok(t), "%s: layer %u has a projection of type %d", name, l, t);
    }
    return LG_OK;
}

// Captured states in the reference's order (src/target.rs:391-395, 558-560): before
// layer l for every l in the list (all layers when the list is null), in ascending l,
// then the final state when n_layers is in the list.  slot[l] = output row or -1.
uint32_t capture_plan(uint32_t n_layers, const uint32_t *list, uint32_t n_list, int32_t *slot) {
    uint32_t c = 0;
    for (uint32_t l = 0; l <= n_layers; l++) {
        bool want = list == nullptr ? l < n_layers : false;
        for (uint32_t i = 0; list && i < n_list; i++) want = want || list[i] == l;
        slot[l] = want ? (int32_t)c++ : -1;
    }
    return c;
}

int proj(const float *x, const void *w, int type, float *c, uint32_t k, uint32_t n, hipStream_t s) {
    return lg_dispatch_proj_quant(x, w, c, k, n, type, s);
}

bool a16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool q4k16(int type, const void *w) { return type == LG_Q4_K && a16(w); }

// Whether the forward can build each layer's inputs inside its products
// (forward_in): every attention and FFN input projection Q4_K on the M = 1
// integer-dot path, 16-byte aligned activations, norms and outputs.
bool inputs_foldable(const lg_target_model *md, const float *input, const float *captured, const float *hidden) {
    const lg_target_hparams &hp = md->hp;
    if (!fold_norms() || hp.n_embd > 4096 || hp.n_embd % QK_K || !a16(input) || !a16(captured) || !a16(hidden) ||
        !a16(md->output_norm))
        return false;
    for (uint32_t l = 0; l < hp.n_layers; l++) {
        const lg_target_layer &L = md->layers[l];
        if (!q4k16(L.attn_q_type, L.attn_q) || !q4k16(L.attn_k_type, L.attn_k) || !q4k16(L.attn_v_type, L.attn_v) ||
            (L.attn_gate && !q4k16(L.attn_gate_type, L.attn_gate)) || !q4k16(L.ffn_gate_type, L.ffn_gate) ||
            !q4k16(L.ffn_up_type, L.ffn_up) || !a16(L.attn_norm) || !a16(L.ffn_norm))
            return false;
    }
    return true;
}

// TargetModel::forward_token_impl with each layer's inputs built inside the M = 1
// products that take them: the residual add (src/target.rs:526-532, 553-555) and the
// RMSNorm (:426-437, :533-537) run in the launch of Q, K, V and the gate together,
// and in the launch of the FFN's gate and up together (proj_m1_in), whose first
// workgroup also writes the residual stream, alternating between two buffers.  The
// LM head takes the last add and the output norm the same way when it is Q4_K.
int forward_in(const lg_target_model *md, const TgtLayout &W, const float *input, const int32_t *slot,
               float *captured, float *logits, float *hidden, lg_target_kv_cache *cache, hipStream_t s) {
    const lg_target_hparams &hp = md->hp;
    const uint32_t E = hp.n_embd, KV = hp.n_kv_heads, HD = hp.head_dim, FF = hp.n_ff, KVD = KV * HD;
    const uint32_t pos = cache ? cache->len : 0;
    const float *cur = input;  // the residual stream, before the pending add
    const float *add = nullptr;
    float *bufs[2] = {W.x, W.x2};
    uint32_t nb = 0;
    for (uint32_t li = 0; li < hp.n_layers; li++) {
        const lg_target_layer &L = md->layers[li];
        const uint32_t H = L.n_q_heads, QD = H * HD;
        const bool swa = hp.swa && li % 4 != 0;  // src/target.rs:438-461
        const float *freq = swa ? W.freq_swa : W.freq;
        const uint32_t rd = swa ? hp.rope_dim_swa : hp.rope_dim;
        float *kdst = W.k, *vdst = W.v;
        const float *kseq = W.k, *vseq = W.v;
        uint32_t seq = 1;
        if (cache) {
            const uint64_t slot_off = ((uint64_t)li * cache->capacity + pos) * KVD;
            kdst = cache->k + slot_off;
            vdst = cache->v + slot_off;
            kseq = cache->k + (uint64_t)li * cache->capacity * KVD;
            vseq = cache->v + (uint64_t)li * cache->capacity * KVD;
            seq = pos + 1;
        }
        // the state entering the layer (captured here), normed: Q, K, V and the gate
        M1In a;
        a.w[0] = L.attn_q, a.type[0] = L.attn_q_type, a.y[0] = W.q, a.n[0] = QD;
        // with the one-token attention the key goes straight to its slot and is normed there
        const bool tok = glue_attention_token_ok(HD, H, KV, rd) && (reinterpret_cast<uintptr_t>(kseq) & 15u) == 0 &&
                         (reinterpret_cast<uintptr_t>(vseq) & 15u) == 0;
        a.w[1] = L.attn_k, a.type[1] = L.attn_k_type, a.y[1] = tok ? kdst : W.k, a.n[1] = KVD;
        a.w[2] = L.attn_v, a.type[2] = L.attn_v_type, a.y[2] = vdst, a.n[2] = KVD;
        a.count = 3;
        if (L.attn_gate) {
            a.w[3] = L.attn_gate, a.type[3] = L.attn_gate_type, a.y[3] = W.gate, a.n[3] = H;
            a.count = 4;
        }
        a.xadd = add, a.nw = L.attn_norm, a.eps = hp.rms_eps;
        a.xout = add ? bufs[nb] : nullptr;
        a.xcap = slot[li] >= 0 ? captured + (uint64_t)slot[li] * E : nullptr;
        LG_TRY(proj_m1_in(cur, a, E, s));
        if (add) {
            cur = bufs[nb];
            nb ^= 1u;
            add = nullptr;
        }
        if (tok) {
            LG_TRY(glue_attention_token(W.q, L.attn_q_norm, L.attn_k_norm, freq, rd, pos, hp.qk_eps,
                                        kdst - (uint64_t)(seq - 1) * KVD, vseq, seq, H, KV, HD,
                                        L.attn_gate ? W.gate : nullptr, W.att, W.part, s));
        } else {
            LG_TRY(glue_qk_norm_rope2(W.q, L.attn_q_norm, W.q, H, W.k, L.attn_k_norm, kdst, KV, HD, rd, pos, freq,
                                      hp.qk_eps, s));
            LG_TRY(glue_attention(W.q, kseq, vseq, seq, seq - 1, H, KV, HD, W.att, W.part, s,
                                  L.attn_gate ? W.gate : nullptr));
        }
        LG_TRY(proj(W.att, L.attn_output, L.attn_output_type, W.o, QD, E, s));
        // x + o_proj, normed: the FFN's gate and up, each pair of rows written as
        // silu(gate) * up (src/target.rs:530-545), then the down projection of that
        M1In f;
        f.w[0] = L.ffn_gate, f.type[0] = L.ffn_gate_type, f.y[0] = W.g, f.n[0] = FF;
        f.w[1] = L.ffn_up, f.type[1] = L.ffn_up_type, f.y[1] = W.u, f.n[1] = FF;
        f.count = 2;
        f.glu = true;
        f.xadd = W.o, f.nw = L.ffn_norm, f.eps = hp.rms_eps, f.xout = bufs[nb];
        LG_TRY(proj_m1_in(cur, f, E, s));
        cur = bufs[nb];
        nb ^= 1u;
        LG_TRY(proj(W.g, L.ffn_down, L.ffn_down_type, W.o, FF, E, s));
        add = W.o;
    }
    float *fcap = slot[hp.n_layers] >= 0 ? captured + (uint64_t)slot[hp.n_layers] * E : nullptr;
    if (md->output && q4k16(md->output_type, md->output)) {  // src/target.rs:558-577 in one launch
        M1In o;
        o.w[0] = md->output, o.type[0] = md->output_type, o.y[0] = logits, o.n[0] = hp.n_vocab;
        o.count = 1;
        o.xadd = add, o.nw = md->output_norm, o.eps = hp.rms_eps, o.xcap = fcap, o.nxout = hidden;
        return proj_m1_in(cur, o, E, s);
    }
    LG_TRY(glue_add(cur, add, W.x, E, s));
    if (fcap) LG_TRY(glue_copy(W.x, fcap, E, s));
    if (md->output_norm) LG_TRY(glue_rmsnorm(W.x, md->output_norm, W.x, E, 1, hp.rms_eps, s));
    if (hidden) LG_TRY(glue_copy(W.x, hidden, E, s));
    if (md->output) return proj(W.x, md->output, md->output_type, logits, E, hp.n_vocab, s);
    return glue_copy(W.x, logits, E, s);
}

// TargetModel::forward_token_impl (src/target.rs:314-578) for a dense model.
int forward(const lg_target_model *md, const TgtLayout &W, const float *input, const int32_t *slot, float *captured,
            float *logits, float *hidden, lg_target_kv_cache *cache, hipStream_t s) {
    const lg_target_hparams &hp = md->hp;
    const uint32_t E = hp.n_embd, KV = hp.n_kv_heads, HD = hp.head_dim, FF = hp.n_ff, KVD = KV * HD;
    const uint32_t pos = cache ? cache->len : 0;
    if (inputs_foldable(md, input, captured, hidden))
        return forward_in(md, W, input, slot, captured, logits, hidden, cache, s);
    LG_TRY(glue_copy(input, W.x, E, s));
    for (uint32_t li = 0; li < hp.n_layers; li++) {
        const lg_target_layer &L = md->layers[li];
        const uint32_t H = L.n_q_heads, QD = H * HD;
        if (slot[li] >= 0) LG_TRY(glue_copy(W.x, captured + (uint64_t)slot[li] * E, E, s));
        LG_TRY(glue_rmsnorm(W.x, L.attn_norm, W.nx, E, 1, hp.rms_eps, s));
        // src/target.rs:438-461: SWA layers (index % 4 != 0) rotate with the SWA table
        const bool swa = hp.swa && li % 4 != 0;
        const float *freq = swa ? W.freq_swa : W.freq;
        const uint32_t rd = swa ? hp.rope_dim_swa : hp.rope_dim;
        // the normed, roped key goes straight to its cache slot, and so does the value
        // as projected
        float *kdst = W.k, *vdst = W.v;
        const float *kseq = W.k, *vseq = W.v;
        uint32_t seq = 1;
        if (cache) {
            const uint64_t slot_off = ((uint64_t)li * cache->capacity + pos) * KVD;
            kdst = cache->k + slot_off;
            vdst = cache->v + slot_off;
            kseq = cache->k + (uint64_t)li * cache->capacity * KVD;
            vseq = cache->v + (uint64_t)li * cache->capacity * KVD;
            seq = pos + 1;
        }
        LG_TRY(proj(W.nx, L.attn_q, L.attn_q_type, W.q, E, QD, s));
        LG_TRY(proj(W.nx, L.attn_k, L.attn_k_type, W.k, E, KVD, s));
        LG_TRY(proj(W.nx, L.attn_v, L.attn_v_type, vdst, E, KVD, s));
        // src/target.rs:496-507: the gate, applied to each head inside the attention
        if (L.attn_gate) LG_TRY(proj(W.nx, L.attn_gate, L.attn_gate_type, W.gate, E, H, s));
        LG_TRY(glue_qk_norm_rope2(W.q, L.attn_q_norm, W.q, H, W.k, L.attn_k_norm, kdst, KV, HD, rd, pos, freq,
                                  hp.qk_eps, s));
        // src/target.rs:466-494: one position (no cache: the token itself) or the cached sequence
        LG_TRY(glue_attention(W.q, kseq, vseq, seq, seq - 1, H, KV, HD, W.att, W.part, s,
                              L.attn_gate ? W.gate : nullptr));
        LG_TRY(proj(W.att, L.attn_output, L.attn_output_type, W.o, QD, E, s));
        LG_TRY(glue_add(W.x, W.o, W.x, E, s));
        LG_TRY(glue_rmsnorm(W.x, L.ffn_norm, W.nx, E, 1, hp.rms_eps, s));
        LG_TRY(proj(W.nx, L.ffn_gate, L.ffn_gate_type, W.g, E, FF, s));
        LG_TRY(proj(W.nx, L.ffn_up, L.ffn_up_type, W.u, E, FF, s));
        if (L.ffn_down_type == LG_Q4_K) {  // silu(gate) * up inside the down projection
            LG_TRY(lg_dispatch_silu_mul_proj_quant(W.g, W.u, L.ffn_down, W.o, FF, E, LG_Q4_K, s));
        } else {
            LG_TRY(lg_dispatch_activation(W.g, W.u, W.g, FF, s));
            LG_TRY(proj(W.g, L.ffn_down, L.ffn_down_type, W.o, FF, E, s));
        }
        LG_TRY(glue_add(W.x, W.o, W.x, E, s));
    }
    if (slot[hp.n_layers] >= 0) LG_TRY(glue_copy(W.x, captured + (uint64_t)slot[hp.n_layers] * E, E, s));
    if (md->output_norm) LG_TRY(glue_rmsnorm(W.x, md->output_norm, W.x, E, 1, hp.rms_eps, s));
    if (hidden) LG_TRY(glue_copy(W.x, hidden, E, s));
    // src/target.rs:570-577: the LM head, or the final hidden when the model has none
    if (md->output) return proj(W.x, md->output, md->output_type, logits, E, hp.n_vocab, s);
    return glue_copy(W.x, logits, E, s);
}

}  // namespace

extern "C" {

int lg_target_capture_count(uint32_t n_layers, const uint32_t *capture_layers, uint32_t n_capture,
                            uint32_t *count) {
    clear_error();
    LG_REQUIRE(count, "lg_target_capture_count: null count");
    LG_REQUIRE(n_layers <= 4096, "lg_target_capture_count: %u layers", n_layers);
    int32_t slot[4097];
    *count = capture_plan(n_layers, capture_layers, n_capture, slot);
    return LG_OK;
}

int lg_target_forward_token(const lg_target_model *model, const float *input, const uint32_t *capture_layers,
                            uint32_t n_capture, float *captured, uint32_t *n_captured, float *logits, float *hidden,
                            lg_target_kv_cache *cache, void *stream) {
    clear_error();
    const char *name = "lg_target_forward_token";
    LG_TRY(check_model(model, name));
    const lg_target_hparams &hp = model->hp;
    LG_REQUIRE(hp.n_layers <= 4096, "%s: %u layers", name, hp.n_layers);
    LG_REQUIRE(input && logits, "%s: null input or logits", name);
    int32_t slot[4097];
    const uint32_t nc = capture_plan(hp.n_layers, capture_layers, n_capture, slot);
    if (n_captured) *n_captured = nc;
    LG_REQUIRE(nc == 0 || captured, "%s: %u states to capture and no buffer", name, nc);
    const uint64_t E = hp.n_embd;
    LG_EXTENT(input, E * 4, name);
    if (nc) LG_EXTENT(captured, nc * E * 4, name);
    LG_EXTENT(logits, (model->output ? (uint64_t)hp.n_vocab : E) * 4, name);
    if (hidden) LG_EXTENT(hidden, E * 4, name);
    uint32_t seq = 1;
    if (cache) {
        LG_REQUIRE(cache->k && cache->v, "%s: cache without buffers", name);
        LG_REQUIRE(cache->len < cache->capacity, "%s: the cache is full (%u of %u positions)", name, cache->len,
                   cache->capacity);
        const uint64_t bytes = (uint64_t)hp.n_layers * cache->capacity * hp.n_kv_heads * hp.head_dim * 4;
        LG_EXTENT(cache->k, bytes, name);
        LG_EXTENT(cache->v, bytes, name);
        seq = cache->len + 1;
    }
    hipStream_t s = (hipStream_t)stream;
    TgtLayout W;
    LG_TRY(eager_ws(model, seq, W, s));
    int st;
    {
        DeferSync d;
        st = forward(model, W, input, slot, captured, logits, hidden, cache, s);
    }
    if (st != LG_OK) return st;
    if (cache) cache->len += 1;  // src/target.rs:562-564
    return after_launch(name, s);
}

}  // extern "C"
