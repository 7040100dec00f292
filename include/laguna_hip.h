/*
 * laguna_hip.h -- C ABI of the MI355X (gfx950) quantized-projection library.
 *
 * This is the drop-in boundary for laguna-raw's projection path.  It replaces
 * the reference's Vulkan runtime (src/vulkan.rs) and the projection shaders
 * (kernels/proj_q4k.comp, proj_q8_0.comp, proj.comp, activation.comp,
 * dequant_q4k.comp, matmul.comp) with HIP kernels for gfx950, behind entry
 * points whose names and argument order follow the reference's dispatch_*
 * functions minus the shader handles.
 *
 * Conventions
 *   - Plain pointers and sizes only.  Device pointers come from lg_buf_alloc
 *     (or any other hipMalloc'd memory); `stream` is a hipStream_t passed as
 *     void* (NULL = the null stream).
 *   - Weight tensors follow GGUF: a [k, n] tensor has ne0 = k contiguous, so
 *     output row i is linear elements i*k .. i*k+k-1 (kernels/proj_q4k.comp:67,
 *     kernels/proj.comp:29).  Quantized tensors are the raw GGUF blocks, uploaded
 *     byte for byte (src/model.rs:174-184).
 *   - Every call returns an lg_status.  Nothing aborts or throws across the
 *     ABI; the text of the last failure on the calling thread is returned by
 *     lg_last_error().  Launches are asynchronous on `stream`; lg_sync()
 *     waits.  The reference blocks after every dispatch
 *     (src/vulkan.rs:326-334); lg_set_blocking(1) restores that behaviour.
 *   - When a pointer was returned by lg_buf_alloc, the library checks that the
 *     extent the call reads or writes lies inside that allocation and returns
 *     LG_EINVAL otherwise (the reference binds whole buffers and never checks).
 *   - Device workspaces belong to a stream.  The entry points that split work
 *     over workgroups (the small-M products, the fused SiLU down projection,
 *     lg_dispatch_argmax, lg_dispatch_mha_attn, the eager draft forward) keep
 *     partial results and arrival counters in memory the library owns per
 *     (device, stream): calls on different streams may run at the same time;
 *     calls on one stream run in order.  A workspace grows between calls (the
 *     stream is synchronised first) and never while its stream is being
 *     captured: make the same call once before capturing it into a HIP graph.
 *     A graph captured from a stream uses that stream's workspace, so it must
 *     not run at the same time as direct calls on that stream.  A draft-forward
 *     graph (lg_dflash_graph_create) owns its workspace.  lg_stream_destroy
 *     releases a stream's workspaces; a stream destroyed without it leaves them
 *     to the next stream that gets the same handle.  hipStreamPerThread gets
 *     one workspace per host thread.  One stream is driven from one host thread
 *     at a time (a workspace that grows is freed under calls racing on it).
 *   - Registries inside the library are locked; the launch-shape hooks of
 *     laguna_hip_tuning.h are atomic.
 */
#ifndef LAGUNA_HIP_H
#define LAGUNA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type ids, as TensorType::from_u32 (src/gguf.rs:46-84) and
 * WeightType (src/target.rs:7-22) use them. */
typedef enum {
    LG_F32 = 0,
    LG_F16 = 1,
    LG_Q8_0 = 8,
    LG_Q4_K = 12,
    LG_BF16 = 30,
    /* Not GGUF types: Q8_0 / Q4_K blocks repacked by lg_repack_tiled into 16-row
     * tiles for the small-M products (block verify, the draft forward). */
    LG_Q8_0_T16 = 1008,
    LG_Q4_K_T16 = 1012
} lg_dtype;

typedef enum {
    LG_OK = 0,
    LG_EINVAL = 1,      /* bad argument: null pointer, size, dtype, extent */
    LG_EHIP = 2,        /* a HIP runtime call failed (text in lg_last_error) */
    LG_ENOMEM = 3,      /* device allocation failed */
    LG_EUNSUPPORTED = 4,/* valid request this build does not implement */
    LG_EIO = 5,         /* file I/O or format error (GGUF) */
    LG_ENODEV = 6,      /* no HIP device */
    LG_ENOTFOUND = 7    /* no such tensor or metadata key (the reference's Option::None) */
} lg_status;

/* ---- runtime (replaces VulkanContext / GpuBuffer, src/vulkan.rs:16-452) ---- */

/* Thread-local text of the last failure ("" if none). */
const char *lg_last_error(void);
/* Library version string. */
const char *lg_version(void);
/* Number of HIP devices (0 on a host without a GPU; never an error). */
int lg_device_count(int *count);
/* Select the device for this thread and create its per-device state
 * (VulkanContext::init, src/vulkan.rs:16-100, which takes pdevices[0]). */
int lg_init(int device);
/* 1 = every launch is followed by a stream synchronise (the reference's
 * fence wait, src/vulkan.rs:326-334); 0 = asynchronous (default). */
int lg_set_blocking(int blocking);

/* Device buffers (GpuBuffer::new / upload / read_f32, src/vulkan.rs:350-452).
 * HBM via hipMalloc; the caller owns and frees them. */
int lg_buf_alloc(void **dptr, uint64_t bytes);
int lg_buf_free(void *dptr);
int lg_buf_upload(void *dst, const void *src, uint64_t bytes, void *stream);
int lg_buf_download(void *dst, const void *src, uint64_t bytes, void *stream);
int lg_buf_memset(void *dst, int value, uint64_t bytes, void *stream);
/* Device-to-device copy (no counterpart in the reference, whose buffers are
 * host-visible and copied through the host); asynchronous on `stream`. */
int lg_buf_copy(void *dst, const void *src, uint64_t bytes, void *stream);
int lg_stream_create(void **stream);
int lg_stream_destroy(void *stream);
int lg_sync(void *stream);

/* ---- dequantization ---- */

/* dequant_to_f32 (src/dflash.rs:331-465) on the device: `n_elements` values
 * from the raw tensor bytes `data` (`data_len` bytes) into `out`.
 *   LG_Q8_0   value = float(int8 q) * d (src/dflash.rs:379-397), bit-exact.
 *   LG_Q4_K   ggml Q4_K, value = (d*sc)*q - dmin*m, the decode every
 *             quantized projection applies (kernels/proj_q4k.comp:28-87);
 *             the reference's Rust Q4_K branch (src/dflash.rs:398-436) is a
 *             different, non-ggml format and is not reproduced.
 *   LG_F32, LG_F16, LG_BF16  as the reference's branches (:333-378, :437-462;
 *             its "BF16" branch decodes IEEE f16 and is reproduced as such).
 *   other     zeros, as the reference's fallback arm (:463).
 * A block that would run past data_len ends decoding; the remaining outputs
 * are 0, as the reference's `break` (:385, :403).
 * Replaces kernels/dequant_q4k.comp, which is never dispatched. */
int lg_dequant_to_f32(const void *data, uint64_t data_len, int dtype, uint64_t n_elements,
                      float *out, void *stream);

/* ---- projections (M = 1) ---- */

/* dispatch_proj_quant (src/target.rs:1086-1099): c[i] = sum_j x[j] * W[i,j]
 * for i < n, j < k; W is raw Q8_0 / Q4_K blocks, or f32 (then proj.comp
 * semantics, row_major = 0).  x: f32[k], c: f32[n]. */
int lg_dispatch_proj_quant(const float *x, const void *w, float *c, uint32_t k, uint32_t n,
                           int dtype, void *stream);

/* dispatch_proj_quant_expert (src/target.rs:1101-1162): as above with W[i,j]
 * taken at linear element expert_offset + i*k + j (kernels/proj_q4k.comp:67).
 * As in the reference, expert_offset applies to Q4_K only: the Q8_0 and F32
 * arms ignore it (src/target.rs:1115-1138). */
int lg_dispatch_proj_quant_expert(const float *x, const void *w, float *c, uint32_t k,
                                  uint32_t n, int dtype, uint32_t expert_offset,
                                  void *stream);

/* dispatch_proj / dispatch_proj_row (src/dflash.rs:1009-1051), f32 weights,
 * kernels/proj.comp:23-33: c[i] = sum_j x[j] * w[row_major ? j*n+i : i*k+j]. */
int lg_dispatch_proj(const float *x, const float *w, float *c, uint32_t k, uint32_t n,
                     void *stream);
int lg_dispatch_proj_row(const float *x, const float *w, float *c, uint32_t k, uint32_t n,
                         uint32_t row_major, void *stream);

/* dispatch_proj_read (src/dflash.rs:1054-1090): f32 projection whose result
 * is copied to host memory `out` (n floats); synchronous. */
int lg_dispatch_proj_read(const float *x, const float *w, uint32_t k, uint32_t n, float *out,
                          void *stream);

/* dispatch_activation (src/dflash.rs:1305-1327), kernels/activation.comp:
 * h[i] = silu(gate[i]) * up[i], silu(x) = x * (1/(1+exp(-x))). */
int lg_dispatch_activation(const float *gate, const float *up, float *h, uint32_t n,
                           void *stream);

/* Fused dispatch_activation + dispatch_proj_quant for the FFN down
 * projection (src/dflash.rs:967-968): c = W * (silu(gate) * up), with
 * gate, up: f32[k].  The activation is computed inside the projection kernel
 * and never written to memory. */
int lg_dispatch_silu_mul_proj_quant(const float *gate, const float *up, const void *w,
                                    float *c, uint32_t k, uint32_t n, int dtype,
                                    void *stream);

/* ---- small-M products (replaces kernels/matmul.comp) ---- */

/* Block-verify product: c[r][i] = sum_j x[r][j] * W[i,j] for r < m, i < n.
 * x is row-major [m][k] of x_dtype LG_F32 or LG_BF16 (raw bf16 bits); c is
 * f32 [m][n]; W is Q4_K or Q8_0 raw blocks, repacked (LG_Q4_K_T16, LG_Q8_0_T16), or f32.  1 <= m <= 64; m = 1 is the
 * same product as lg_dispatch_proj_quant. */
int lg_dispatch_proj_quant_batch(const void *x, int x_dtype, const void *w, float *c,
                                 uint32_t k, uint32_t n, uint32_t m, int w_dtype,
                                 void *stream);

/* lg_dispatch_proj_quant_batch without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results, bit for bit; the split-k partial sums and arrival
 * counters live in a fixed 16 MiB + 64 KiB device array that
 * every GPU the library runs on holds until the process ends (set up by lg_init,
 * or by the first call on a device).  Shapes whose workspace
 * (lg_proj_quant_batch_ws_bytes) exceeds it are LG_EINVAL.  Calls on one GPU share
 * the array: calls that overlap in time on one GPU, on any stream, race. */
int lg_dispatch_proj_quant_batch_static(const void *x, int x_dtype, const void *w, float *c,
                                        uint32_t k, uint32_t n, uint32_t m, int w_dtype,
                                        void *stream);

/* Device workspace bytes lg_dispatch_proj_quant_batch needs for this shape on the
 * current device (0: the shape takes the element-wise path, which needs none).  No
 * counterpart in the reference.  It is 64 KiB of arrival counters plus, when the
 * product splits k over slices, the split-k partial sums: slices * n' * 16 * tiles * 4
 * bytes, n' = n rounded up to whole workgroup columns (64 or 128 rows) and tiles =
 * ceil(min(m, 32) / 16) (slices chosen for about two workgroups per CU).
 * lg_dispatch_proj_quant_batch_static accepts a shape when this is at most
 * 16 MiB + 64 KiB. */
uint64_t lg_proj_quant_batch_ws_bytes(uint32_t k, uint32_t n, uint32_t m, int w_dtype);

/* Q4_K and Q8_0 weights repacked for the small-M products (no counterpart in the
 * reference, which reads GGUF blocks in place; for callers that load a model once
 * and run many block products).  Tiles hold 16 rows x 256 elements and are stored
 * row tile by row tile, k in order; rows past n, up to a multiple of 16, are zero
 * blocks.
 *   LG_Q4_K_T16 tile (2304 bytes): the 16 rows' 16-byte block headers (d, dmin,
 *     scales) in row order, then the quant bytes as [32-byte group g][8-byte
 *     piece p][row r] (row r's bytes 32g+8p .. 32g+8p+7 at 256 + 512g + 128p + 8r).
 *   LG_Q8_0_T16 tile (4352 bytes, blocks 8c..8c+7): the 16 rows' 8 f16 scales
 *     (row r, block j at 16r + 2j), then the quants as [block j][8-byte piece p]
 *     [row r] (row r's quants 8p .. 8p+7 of block j at 256 + 512j + 128p + 8r),
 *     each biased to unsigned (q XOR 0x80, as the products take them).
 * The repack is a byte permutation (and that bias), and the products over tiled weights
 * (lg_dispatch_proj_quant_batch, lg_dispatch_silu_gate_up_batch, the draft
 * forward) equal those over the raw blocks bit for bit; a workgroup then reads
 * whole tiles instead of short pieces of rows that lie a row apart.  dtype
 * LG_Q4_K or LG_Q8_0 (the raw type), k a multiple of 256; lg_tiled_bytes is 0
 * for anything else. */
uint64_t lg_tiled_bytes(int dtype, uint32_t k, uint32_t n);
int lg_repack_tiled(const void *w, int dtype, uint32_t k, uint32_t n, void *out, void *stream);

/* The FFN's gate and up projections and dispatch_activation of a block in one
 * launch (src/dflash.rs:963-965): h[r][i] = silu(g[r][i]) * u[r][i] with
 * g[r][i] = sum_j x[r][j] W_gate[i,j] and u likewise with W_up (both n rows of
 * w_dtype, f32 x [m][k], 1 <= m <= 64).  Each workgroup computes the same rows of
 * both products, so g and u are never written; u_scratch (f32 [m][n]) is used
 * only by inputs outside the matrix-core path, which compute g and u apart. */
int lg_dispatch_silu_gate_up_batch(const float *x, const void *w_gate, const void *w_up, float *h,
                                   float *u_scratch, uint32_t k, uint32_t n, uint32_t m, int w_dtype,
                                   void *stream);

/* ---- target-side verify ---- */

/* argmax (src/lib.rs:456-464) of each of `rows` rows of n logits (row r at
 * logits + r*ld, ld >= n), on the device: out[r] is the reference's index bit for
 * bit -- the last of equal maxima, and a NaN restarts the search after it (its
 * fold with partial_cmp(..).unwrap_or(Equal)); n = 0 gives 0.  Used on the LM
 * head's logits of the target (one row) and of a draft block (m rows). */
int lg_dispatch_argmax(const float *logits, uint32_t n, uint32_t rows, uint64_t ld, uint32_t *out,
                       void *stream);

/* ---- DFlash draft glue (src/dflash.rs dispatch_* helpers, rows >= 1) ---- */

/* dispatch_rmsnorm (src/dflash.rs:978-1007), kernels/rmsnorm.comp: for each of
 * `rows` rows of n floats, out = x * w * (mean(x^2) + eps)^-1/2.  The reference
 * passes eps = 1e-5 and one row. */
int lg_dispatch_rmsnorm(const float *w, const float *x, float *out, uint32_t n, uint32_t rows, float eps,
                        void *stream);

/* dispatch_enc_aux_norm (src/dflash.rs:1200-1233), kernels/enc_aux_norm.comp:
 * out[i] = x[i] * (mean(x[chunk]^2) + 1e-5)^-1/2 * aux_norm_w[i % (n_aux*n_feat)]
 * for i < n_total, where chunk is the n_feat-float chunk that holds i.  Same
 * arguments as the reference (n_total = n_aux*n_feat for its one token); n_total
 * may be any whole number of tokens. */
int lg_dispatch_enc_aux_norm(const float *x, const float *aux_norm_w, float *out, uint32_t n_feat,
                             uint32_t n_aux, uint32_t n_total, void *stream);

/* dispatch_qk_norm_rope (src/dflash.rs:1092-1128), kernels/qk_norm_rope.comp:
 * per-head RMSNorm times norm_w[dim], then GPT-NeoX rotation of dims < rope_dim
 * with angle freq[dim % (rope_dim/2)] * pos.  Row r (of `rows`, each
 * n_heads*head_dim floats) is at position pos + r.  head_dim <= 256 and even;
 * rope_dim is head_dim or 0 (for a smaller rope_dim the shader's partner index of
 * the second rotary half, i - head_dim/2, leaves the head).  The reference passes
 * eps = 1e-6. */
int lg_dispatch_qk_norm_rope(const float *x, const float *norm_w, const float *freq, float *out,
                             uint32_t n_heads, uint32_t head_dim, uint32_t rope_dim, uint32_t pos,
                             uint32_t rows, float eps, void *stream);

/* dispatch_mha_attn_seq (src/dflash.rs:1158-1194), kernels/mha_attn.comp:
 * out[r][h] = softmax_p(q[r][h] . k_seq[p][kv(h)] / sqrt(head_dim)) v_seq[p][kv(h)]
 * over p < seq_len (and p <= q_pos + r when causal), kv(h) = h * n_kv / n_q.
 * q: [rows][n_q*head_dim], k_seq, v_seq: [seq_len][n_kv*head_dim]. */
int lg_dispatch_mha_attn(const float *q, const float *k_seq, const float *v_seq, float *out, uint32_t n_q_heads,
                         uint32_t n_kv_heads, uint32_t head_dim, uint32_t seq_len, uint32_t q_pos,
                         uint32_t rows, int causal, void *stream);

/* dispatch_gate_mul (src/dflash.rs:1236-1266), kernels/gate_mul.comp, same
 * argument order: attn_out[i] = v_rep[i] * gate[i / head_dim] for i < n_hd
 * (n_heads does not enter the result, as in the shader). */
int lg_dispatch_gate_mul(float *attn_out, const float *v_rep, const float *gate, uint32_t n_hd,
                         uint32_t n_heads, uint32_t head_dim, void *stream);

/* The attention gate of src/dflash.rs:956-959 on the device, arguments as
 * dispatch_gate_mul: the reference applies softplus on the host
 * (g > 20 ? g : ln(1 + e^g)) and then gate_mul;
 * attn_out[i] = v_rep[i] * softplus(gate[i / head_dim]). */
int lg_dispatch_softplus_gate_mul(float *attn_out, const float *v_rep, const float *gate, uint32_t n_hd,
                                  uint32_t n_heads, uint32_t head_dim, void *stream);

/* dispatch_gate_attn (src/target.rs:992-1020), kernels/gate_attn.comp, same
 * argument order: result[i] = attn_out[i] * log(1 + exp(gate[i / head_dim])) for
 * i < n_heads*head_dim.  No threshold, as in the shader: a gate above about 88.7
 * gives an infinite factor.  result may be attn_out (the target's in-place call). */
int lg_dispatch_gate_attn(const float *attn_out, const float *gate, float *result, uint32_t n_heads,
                          uint32_t head_dim, void *stream);

/* dispatch_add (src/dflash.rs:1284-1303), kernels/add.comp: out = a + b. */
int lg_dispatch_add(const float *a, const float *b, float *out, uint32_t n, void *stream);

/* ---- GGUF v3 reader (replaces GGUFReader, src/gguf.rs:321-514, and the tensor
 * loads of Model, src/model.rs:137-184).  Host code; only lg_gguf_upload_tensor
 * touches the device.  The file stays open until lg_gguf_close; strings returned
 * by the reader live as long as it does. ---- */

typedef struct lg_gguf lg_gguf;

#define LG_GGUF_MAX_DIMS 8
#define LG_GGUF_MAX_TARGET_LAYERS 64

/* TensorInfo (src/gguf.rs:172-201).  shape[0] is ne0, the contiguous dimension;
 * data_offset is relative to the tensor data section; n_bytes = whole blocks of
 * the type (the reference's table, lg_gguf_type_info). */
typedef struct {
    const char *name;
    uint32_t n_dims;
    uint64_t shape[LG_GGUF_MAX_DIMS];
    int dtype;
    uint64_t data_offset;
    uint64_t n_elements;
    uint64_t n_bytes;
} lg_gguf_tensor;

/* The GGUFMetadata fields the draft and target models read (populate_metadata,
 * src/gguf.rs:517-637, with its key aliases: "laguna.", "dflash." or no prefix).
 * A field is valid when its LG_GGUF_HAS_* bit is set in `present`.  Every other
 * key is reachable through lg_gguf_field / lg_gguf_get_*. */
enum {
    LG_GGUF_HAS_ARCHITECTURE = 1u << 0,
    LG_GGUF_HAS_GENERAL_NAME = 1u << 1,
    LG_GGUF_HAS_FILE_TYPE = 1u << 2,
    LG_GGUF_HAS_ALIGNMENT = 1u << 3,
    LG_GGUF_HAS_BLOCK_COUNT = 1u << 4,
    LG_GGUF_HAS_CONTEXT_LENGTH = 1u << 5,
    LG_GGUF_HAS_EMBEDDING_LENGTH = 1u << 6,
    LG_GGUF_HAS_FEED_FORWARD_LENGTH = 1u << 7,
    LG_GGUF_HAS_HEAD_COUNT = 1u << 8,
    LG_GGUF_HAS_HEAD_COUNT_KV = 1u << 9,
    LG_GGUF_HAS_KEY_LENGTH = 1u << 10,
    LG_GGUF_HAS_VALUE_LENGTH = 1u << 11,
    LG_GGUF_HAS_RMS_EPSILON = 1u << 12,
    LG_GGUF_HAS_ROPE_FREQ_BASE = 1u << 13,
    LG_GGUF_HAS_ROPE_DIMENSION_COUNT = 1u << 14,
    LG_GGUF_HAS_EXPERT_COUNT = 1u << 15,
    LG_GGUF_HAS_EXPERT_USED_COUNT = 1u << 16,
    LG_GGUF_HAS_VOCAB_SIZE = 1u << 17,
    LG_GGUF_HAS_TARGET_LAYERS = 1u << 18,
    LG_GGUF_HAS_DECODER_ARCH = 1u << 19,
    LG_GGUF_HAS_EXPERT_WEIGHTS_NORM = 1u << 20
};

typedef struct {
    uint32_t present;
    char architecture[64], general_name[256], decoder_arch[64];
    uint64_t file_type, alignment, block_count, context_length, embedding_length, feed_forward_length;
    uint64_t head_count, head_count_kv, key_length, value_length, rope_dimension_count;
    uint64_t expert_count, expert_used_count, vocab_size;
    float rms_epsilon, rope_freq_base;
    int expert_weights_norm;
    uint32_t n_target_layers;
    int64_t target_layers[LG_GGUF_MAX_TARGET_LAYERS];
} lg_gguf_meta;

/* TensorType::block_size / block_elements / is_supported / is_quantized
 * (src/gguf.rs:91-170) for a GGUF type id; LG_EINVAL for ids from_u32 rejects. */
int lg_gguf_type_info(int dtype, uint32_t *block_bytes, uint32_t *block_elements, int *supported, int *quantized);

/* GGUFReader::open (src/gguf.rs:321-405): magic "GGUF", version 3 only, the
 * metadata fields, the tensor infos, and the data section at the next multiple of
 * general.alignment (default 32).  LG_EIO for a missing, foreign, truncated or
 * inconsistent file (the reference returns io::Error or panics). */
int lg_gguf_open(const char *path, lg_gguf **out);
int lg_gguf_close(lg_gguf *g);
int lg_gguf_header(const lg_gguf *g, uint32_t *version, uint64_t *tensor_count, uint64_t *field_count,
                   uint64_t *tensor_data_offset);
int lg_gguf_metadata(const lg_gguf *g, lg_gguf_meta *out);
int lg_gguf_tensor_info(const lg_gguf *g, uint64_t index, lg_gguf_tensor *out);
/* tensor_by_name (src/gguf.rs:407-409): the first tensor of that name, or LG_ENOTFOUND. */
int lg_gguf_find_tensor(const lg_gguf *g, const char *name, uint64_t *index);
/* read_tensor_data (src/gguf.rs:415-421): the tensor's n_bytes raw bytes into host
 * memory `dst` (at least n_bytes).  LG_EIO when they run past the end of the file. */
int lg_gguf_read_tensor(const lg_gguf *g, uint64_t index, void *dst, uint64_t dst_bytes);
/* Model::upload_tensor_quantized (src/model.rs:174-184): the same bytes, unchanged,
 * into device memory `dptr` (at least n_bytes), streamed through pinned staging
 * memory; returns after the copy has completed. */
int lg_gguf_upload_tensor(const lg_gguf *g, uint64_t index, void *dptr, uint64_t dst_bytes, void *stream);

/* Raw metadata fields in file order (raw_fields, src/gguf.rs:341-355).  type is
 * the GGUF value type (0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool,
 * 8 string, 9 array, 10 u64, 11 i64, 12 f64); arrays report their length and the
 * type of their first element. */
int lg_gguf_field_count(const lg_gguf *g, uint64_t *count);
int lg_gguf_field(const lg_gguf *g, uint64_t index, const char **key, int *type, uint64_t *n_elements,
                  int *element_type);
/* The index of the first field named `key`, or LG_ENOTFOUND. */
int lg_gguf_find_field(const lg_gguf *g, const char *key, uint64_t *index);
/* Typed reads of field `field`, or of element `elem` of an array field
 * (elem = UINT64_MAX reads the field itself).  u64, f32 and bool convert as
 * GGUFValue::as_u64 / as_f32 / as_bool (src/gguf.rs:232-272); i64 reads any
 * integer (signed ones sign-extended); f64 reads f32 or f64.  LG_EINVAL for a
 * value of another kind. */
int lg_gguf_get_u64(const lg_gguf *g, uint64_t field, uint64_t elem, uint64_t *out);
int lg_gguf_get_i64(const lg_gguf *g, uint64_t field, uint64_t elem, int64_t *out);
int lg_gguf_get_f32(const lg_gguf *g, uint64_t field, uint64_t elem, float *out);
int lg_gguf_get_f64(const lg_gguf *g, uint64_t field, uint64_t elem, double *out);
int lg_gguf_get_bool(const lg_gguf *g, uint64_t field, uint64_t elem, int *out);
int lg_gguf_get_str(const lg_gguf *g, uint64_t field, uint64_t elem, const char **out, uint64_t *len);


/* ---- DFlash draft model (src/dflash.rs DFlashModel) ---- */

typedef struct {
    uint32_t n_embd, n_heads, n_kv_heads, head_dim, rope_dim, n_ff, n_aux, n_layers;
    float rope_base;  /* rope_freq_base (src/dflash.rs:898-904; default 500000) */
    float rms_eps;    /* 1e-5 (src/dflash.rs:987) */
    float qk_eps;     /* 1e-6 (src/dflash.rs:1105) */
} lg_dflash_hparams;

/* One decoder layer: device pointers to the tensors of src/dflash.rs:68-79
 * (raw GGUF blocks for the projections, f32 for the norms), their GGUF types,
 * and the layer's cached context keys (normed and roped) and values, each
 * [ctx_len][n_kv_heads*head_dim] f32. */
typedef struct {
    const float *attn_norm, *attn_q_norm, *attn_k_norm, *ffn_norm;
    const void *attn_q, *attn_k, *attn_v, *attn_gate, *attn_output, *ffn_gate, *ffn_up, *ffn_down;
    int attn_q_type, attn_k_type, attn_v_type, attn_gate_type, attn_output_type, ffn_gate_type, ffn_up_type,
        ffn_down_type;
    const float *k_ctx, *v_ctx;
} lg_dflash_layer;

typedef struct {
    lg_dflash_hparams hp;
    const float *enc_aux_norm;    /* [n_aux*n_embd] */
    const void *fc;               /* [n_aux*n_embd -> n_embd] */
    int fc_type;
    const float *enc_output_norm; /* [n_embd] */
    const float *output_norm;     /* [n_embd] or NULL */
    const lg_dflash_layer *layers;
} lg_dflash_model;

/* DFlashModel::encode (src/dflash.rs:157-234) for m feature rows:
 * enc_aux_norm, fc, rmsnorm(enc_output_norm).  features: [m][n_aux*n_embd],
 * out: [m][n_embd]. */
int lg_dflash_encode(const lg_dflash_model *model, const float *features, uint32_t m, float *out, void *stream);

/* DFlashModel::forward_injected_decode_hidden (src/dflash.rs:877-976) for a block
 * of m tokens over ctx_len cached positions.  Per layer the queries attend
 * causally to [context (0..ctx_len-1)] ++ [the m injected encoder keys/values at
 * positions ctx_len..ctx_len+m-1] ++ [the m token keys/values at ctx_len+m..];
 * token t is at ctx_len+m+t.  With m = 1 and ctx_len = 0 this is the
 * reference's sequence exactly.  features: [m][n_aux*n_embd], tokens:
 * [m][n_embd] (token inputs), out: [m][n_embd] final hidden (after output_norm
 * when present).  1 <= m <= 32; head_dim 128 uses the matrix-core attention. */
int lg_dflash_forward_block(const lg_dflash_model *model, const float *features, const float *tokens,
                            uint32_t m, uint32_t ctx_len, float *out, void *stream);

/* The same forward captured once into a HIP graph on `stream` (the eager call is
 * made first to size the workspaces) and replayed by lg_dflash_graph_launch.
 * Inputs and outputs are read and written at the captured addresses. */
int lg_dflash_graph_create(const lg_dflash_model *model, const float *features, const float *tokens, uint32_t m,
                           uint32_t ctx_len, float *out, void *stream, void **graph);
int lg_dflash_graph_launch(void *graph, void *stream);
int lg_dflash_graph_destroy(void *graph);

/* ---- Dense target model (src/target.rs TargetModel, dense layers) ---- */

typedef struct {
    uint32_t n_embd, n_heads, n_kv_heads, head_dim, n_ff, n_layers;
    uint32_t n_vocab;      /* rows of `output` (vocab_size, src/target.rs:287-291) */
    uint32_t rope_dim;     /* rope.dimension_count: 0 or head_dim */
    uint32_t rope_dim_swa; /* rope.dimension_count_swa: 0 or head_dim */
    int swa;               /* rope_dim_swa > 0 or attention.sliding_window > 0 (src/target.rs:331);
                            * layers whose index % 4 != 0 then use the SWA table (:440) */
    float rope_base;       /* rope.freq_base, 0 = the reference's default 500000 (:350) */
    float rope_base_swa;   /* rope.freq_base_swa, 0 = 10000 (:366) */
    float rms_eps;         /* 1e-5 (src/target.rs:970) */
    float qk_eps;          /* 1e-6 (src/target.rs:897) */
} lg_target_hparams;

/* One dense layer (TargetDenseLayer, src/target.rs:30-43): f32 norms, raw GGUF
 * blocks (LG_Q4_K, LG_Q8_0) or f32 for the projections, attn_gate optional (NULL:
 * no gate), and the layer's query head count (attn_q rows / head_dim,
 * src/target.rs:236-246). */
typedef struct {
    const float *attn_norm, *attn_q_norm, *attn_k_norm, *ffn_norm;
    const void *attn_q, *attn_k, *attn_v, *attn_gate, *attn_output, *ffn_gate, *ffn_up, *ffn_down;
    int attn_q_type, attn_k_type, attn_v_type, attn_gate_type, attn_output_type, ffn_gate_type, ffn_up_type,
        ffn_down_type;
    uint32_t n_q_heads;
} lg_target_layer;

typedef struct {
    lg_target_hparams hp;
    const lg_target_layer *layers;
    const float *output_norm; /* [n_embd] or NULL */
    const void *output;       /* LM head [n_vocab][n_embd] or NULL (logits = final hidden) */
    int output_type;
} lg_target_model;

/* Device-resident K/V cache (replaces TargetKvCache, src/target.rs:74-101, which
 * the reference keeps on the host and re-uploads whole every token): layer l's
 * normed, roped key and raw value of position p at [l][p][n_kv_heads*head_dim]
 * of k and v, for p < len. */
typedef struct {
    float *k, *v;
    uint32_t capacity; /* positions per layer */
    uint32_t len;      /* tokens cached: the position of the next token */
} lg_target_kv_cache;

/* TargetModel::forward_token (cache NULL) and forward_token_cached
 * (src/target.rs:298-578) for a dense model: one token `input` [n_embd] at
 * position cache ? cache->len : 0.  Hidden states are captured as they enter
 * layer l for each l in capture_layers (every layer when capture_layers is NULL,
 * the reference's None), in ascending l, plus the final state (before
 * output_norm) when n_layers is listed; *n_captured receives their number and
 * captured[i*n_embd ..] the states.  logits: [n_vocab] (LM head of the normed
 * final state), or [n_embd] holding that normed state when the model has no
 * output weight; hidden (optional): the normed final state.  With a cache, the
 * token's K/V are stored at position len, attention runs over 0..len, and len
 * is incremented.  MoE layers are not supported. */
int lg_target_forward_token(const lg_target_model *model, const float *input, const uint32_t *capture_layers,
                            uint32_t n_capture, float *captured, uint32_t *n_captured, float *logits, float *hidden,
                            lg_target_kv_cache *cache, void *stream);

/* The number of states lg_target_forward_token captures for this list (host only). */
int lg_target_capture_count(uint32_t n_layers, const uint32_t *capture_layers, uint32_t n_capture,
                            uint32_t *count);

#ifdef __cplusplus
}
#endif
#endif /* LAGUNA_HIP_H */
