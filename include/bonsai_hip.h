/*
 * bonsai_hip.h -- C ABI of the MI355X (gfx950) fused layer kernels of
 * ternary-bonsai-inference.
 *
 * The reference engine is Rust; its hot-path kernels are free functions over
 * f32 slices in src/kernels.rs and src/rope.rs.  Every entry point below
 * replaces one of those functions (or one composition site of them in
 * src/forward.rs) and cites it.  The ABI is plain C: pointers, sizes, scalars
 * and an opaque stream handle, so a Rust `extern "C"` block binds it directly.
 *
 * Two families:
 *   bh_*       device entry points.  Every pointer is DEVICE memory owned by
 *              the caller; work is enqueued on `stream` (a hipStream_t, NULL =
 *              the default stream) and the call returns without synchronising.
 *   bh_host_*  host-slice mirrors with the exact Rust signatures: host
 *              pointers in and out, the call copies to the GPU, runs the
 *              device kernel and copies back before returning.
 *
 * Status codes: 0 on success, otherwise one of BH_ERR_*.  The message the
 * Rust code would put in Err(String) is available from bh_last_error()
 * (thread-local, valid until the next bh_* call on the same thread).
 *
 * Numerics follow the reference CPU path: f32 storage, f64 accumulation where
 * the Rust accumulates in f64 (l2_norm_rows, softmax_rows), libm-accurate
 * expf/logf/sinf/cosf, no FMA contraction -- except the two passes of the
 * softmax over rows too wide for one workgroup, which use the hardware base-2
 * exponential with an FMA-compensated argument (a few 1e-7 relative, inside
 * the softmax tolerance of 2e-5).  The PQ2_0 decode is bit-exact.
 *
 * Threading: every device entry point is re-entrant per stream, except
 * bh_softmax_rows on rows too wide for one workgroup, bh_attention,
 * bh_attention_planar, bh_pq2_embed_gather_rms on batches of at least 16
 * ids per compute unit (4096 on MI355X; it keeps the row scales there), and
 * the PQ2_0 products (bh_pq2_matvec_range, bh_pq2_matmul_n) with more than 4
 * tokens or on shapes outside the integer path, and bh_gdn_step on batches
 * of 128 or more tokens at s = 128, which use per-device scratch buffers:
 * each must not run concurrently with itself on one device.
 *
 * Scratch and HIP graphs: a scratch buffer grows (allocates) the first time
 * a call needs more than it holds.  The buffer it replaces is kept until the
 * process ends, so a graph captured earlier still replays on valid memory.
 * Growth is refused while the stream is capturing (BH_ERR_HIP, with a
 * message): run a scratch-using call once outside capture at its largest
 * shape before capturing it.  The other entry points allocate nothing.
 */
#ifndef BONSAI_HIP_H
#define BONSAI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BH_OK 0
#define BH_ERR_SHAPE (-1) /* the Rust Err(String) shape checks            */
#define BH_ERR_RANGE (-2) /* token id >= n_rows (src/weights.rs:337-341)    */
#define BH_ERR_HIP (-3)   /* HIP runtime failure (launch, copy, malloc)     */
#define BH_ERR_ARG (-4)   /* NULL pointer, unknown mode, unsupported layout */

/* Opaque stream handle: a hipStream_t.  NULL selects the default stream. */
typedef void *bh_stream;

/* Message of the last failing call on this thread ("" after a success). */
const char *bh_last_error(void);
/* Library identification string (version, target architecture). */
const char *bh_version(void);

/* Scratch housekeeping (no counterpart in the reference, whose kernels run
 * on the host).  A scratch buffer that grows keeps the buffer it replaces
 * until the process ends (a captured graph may still hold its address);
 * bh_scratch_retired_bytes reports how many bytes those retired buffers hold
 * on all devices, and bh_scratch_release synchronizes each device that has
 * any and frees them -- for callers that know no captured graph still uses
 * an old buffer (e.g. after a one-off very large call).  Not to be called
 * while other threads run library calls. */
size_t bh_scratch_retired_bytes(void);
int bh_scratch_release(void);

/* ---------------------------------------------------------------------------
 * Normalisation (src/kernels.rs:58-145)
 * ------------------------------------------------------------------------- */

/* kernels::rms_norm (src/kernels.rs:59-75) and rms_norm_inplace (:80-93):
 * out = x * (1/sqrt(mean(x^2) + eps)) * w over one vector of n.  out may
 * equal x (in place).  n == 0 is a no-op. */
int bh_rms_norm(const float *x, const float *w, size_t n, float eps, float *out,
                bh_stream stream);

/* kernels::rms_norm_rows (src/kernels.rs:97-122): RMSNorm of each of the
 * x_len/row_len consecutive rows with the shared weight w[row_len].
 * BH_ERR_SHAPE when w_len != row_len or x_len % row_len != 0. */
int bh_rms_norm_rows(const float *x, size_t x_len, const float *w, size_t w_len,
                     size_t row_len, float eps, float *out, bh_stream stream);

/* Residual add + RMSNorm, the composition at src/forward.rs:708-713
 * (cur[i] += attn_out[i]; ffn_in = rms_norm(cur, post_w, eps)), per row:
 * sum_out = x + residual; out = rms_norm_rows(sum_out, w, row_len, eps).
 * sum_out may alias x (the in-place `cur +=` of the reference). */
int bh_add_rms_norm_rows(const float *x, const float *residual, size_t x_len,
                         const float *w, size_t w_len, size_t row_len, float eps,
                         float *sum_out, float *out, bh_stream stream);

/* kernels::l2_norm_rows (src/kernels.rs:126-145): per row, f64 sum of x^2,
 * scale = 1 / max(sqrt((f32)sum), eps), out = x * scale. */
int bh_l2_norm_rows(const float *x, size_t x_len, size_t row_len, float eps,
                    float *out, bh_stream stream);

/* SiLU then L2 rows: the conv output path of src/forward.rs:524 (silu) and
 * :539-540 (l2_norm_rows) fused: out = l2_norm_rows(silu(x), row_len, eps). */
int bh_silu_l2_norm_rows(const float *x, size_t x_len, size_t row_len, float eps,
                         float *out, bh_stream stream);

/* ---------------------------------------------------------------------------
 * Activations (src/kernels.rs:148-171; shaders/elem.comp modes 0-4)
 * ------------------------------------------------------------------------- */

#define BH_SILU 0        /* kernels::silu     x / (1 + exp(-x))               */
#define BH_SIGMOID 1     /* kernels::sigmoid  1 / (1 + exp(-x))               */
#define BH_SOFTPLUS 2    /* kernels::softplus x > 20 ? x : ln(1 + exp(x))     */
#define BH_SILU_MUL 3    /* b * silu(a): FFN gate-up (src/forward.rs:574),
                            GDN output gate (src/forward.rs:549-551)          */
#define BH_SIGMOID_MUL 4 /* b * sigmoid(a): attention gate
                            (src/forward.rs:379-382)                         */

/* kernels::map_inplace(x, f) (src/kernels.rs:167-171) for modes 0-2 (b is
 * ignored and may be NULL), and the fused gated products for modes 3-4.
 * out may alias a or b. */
int bh_unary(int mode, const float *a, const float *b, size_t n, float *out,
             bh_stream stream);

/* GDN gate prep (src/forward.rs:497-507), n_tok x n_head:
 *   beta_out = sigmoid(beta_raw)
 *   gate_out = softplus(alpha_raw + dt_bias[h]) * ssm_a[h]
 * dt_bias and ssm_a have n_head entries.  Either output may be NULL (then
 * its inputs are not read). */
int bh_gdn_gate_prep(const float *alpha_raw, const float *dt_bias,
                     const float *ssm_a, const float *beta_raw, size_t n_tok,
                     size_t n_head, float *gate_out, float *beta_out,
                     bh_stream stream);

/* All of the recurrent layer's small ops for n_tok tokens in ONE launch
 * (src/forward.rs:497-507, 524, 539-540, 549-551 / :379-382):
 *   conv_out[t]  = silu(conv[t]); its first l2_dim channels are then
 *                  l2-normalised per head_dim group (q and k heads);
 *   gated_out[t] = y[t] * silu(z[t])    (gate_mode BH_SILU_MUL, GDN) or
 *                  y[t] * sigmoid(z[t]) (gate_mode BH_SIGMOID_MUL, attention);
 *   gate_out[t]  = softplus(alpha_raw[t] + dt_bias) * ssm_a;
 *   beta_out[t]  = sigmoid(beta_raw[t]).
 * Each group is skipped when its output pointer is NULL. */
typedef struct bh_gdn_prep_args {
  const float *conv;  /* [n_tok][conv_dim]                          */
  float *conv_out;    /* [n_tok][conv_dim], may alias conv          */
  const float *z;     /* [n_tok][inner_dim] gate pre-activation     */
  const float *y;     /* [n_tok][inner_dim] gated tensor            */
  float *gated_out;   /* [n_tok][inner_dim], may alias y or z       */
  const float *alpha_raw; /* [n_tok][n_v_head]                      */
  const float *dt_bias;   /* [n_v_head]                             */
  const float *ssm_a;     /* [n_v_head]                             */
  const float *beta_raw;  /* [n_tok][n_v_head]                      */
  float *gate_out;        /* [n_tok][n_v_head]                      */
  float *beta_out;        /* [n_tok][n_v_head]                      */
  size_t n_tok;
  size_t conv_dim;  /* channels per token row of conv            */
  size_t l2_dim;    /* leading channels that get the L2 norm     */
  size_t head_dim;  /* L2 group width (128 in Ternary-Bonsai-27B) */
  size_t inner_dim; /* width of z / y                            */
  size_t n_v_head;  /* 48 in Ternary-Bonsai-27B                  */
  int gate_mode;    /* BH_SILU_MUL or BH_SIGMOID_MUL             */
  float eps;
  /* Optional causal conv1d in front (src/forward.rs:508-533): when conv_w is
   * non-NULL, `conv` holds the raw qkv projections and the channels are
   * convolved with conv_w [conv_dim][conv_k] over the tokens and the cache
   * conv_state [conv_dim][conv_k - 1] (oldest first) before the SiLU; the
   * cache is then advanced by n_tok tokens, in place.  conv_out must not
   * alias conv in this mode.  Zero these fields to leave it off. */
  const float *conv_w;
  float *conv_state;
  size_t conv_k;
} bh_gdn_prep_args;

int bh_gdn_prep_fused(const bh_gdn_prep_args *args, bh_stream stream);

/* Causal conv1d + SiLU over n_tok tokens (src/forward.rs:508-533 applied per
 * token): out[t][c] = silu(sum_j w[c][j] * s_{t-k+1+j}) with s_p = x[p][c]
 * and, for p < 0, the cache state[c][p + k - 1] (k - 1 inputs per channel,
 * oldest first); the cache is then advanced by n_tok tokens in place.
 * x, out: [n_tok][ch] (out must not alias x); w: [ch][k]; 1 <= k <= 64. */
int bh_conv1d_silu(const float *x, float *state, const float *w, size_t n_tok,
                   size_t ch, size_t k, float *out, bh_stream stream);

/* KV cache storage types of bh_kv_store / bh_attention. */
#define BH_KV_F32 0 /* f32 cache (AttnCache::k / v)                          */
#define BH_KV_F16 1 /* f16 bits (AttnCache::k16 / v16, BONSAI_KV=f16)        */

/* AttnCache::append / append_f16 (src/forward.rs:90-95, 120-125) for n_tok
 * tokens: rows k, v [n_tok][n_kv_elems] (f32) are written at positions
 * pos0 .. pos0 + n_tok - 1 of the caches [cap][n_kv_elems], as f32 or as
 * gguf::f32_to_half bits (src/gguf.rs:914-944, bit for bit). */
int bh_kv_store(const float *k, const float *v, size_t n_tok, size_t n_kv_elems,
                void *k_cache, void *v_cache, size_t pos0, int kv_dtype, bh_stream stream);

/* The GQA block of full_attention_layer (src/forward.rs:282-375) for n_q
 * query tokens at positions pos0 .. pos0 + n_q - 1: query i, head hq reads
 * kv head hq / (n_head / n_kv) over cache positions 0 .. pos0 + i;
 * scores = q.k / sqrtf(hd), probs = softmax_rows(scores), out = probs . V.
 * q, out: [n_q][n_head][hd] f32; caches [>= pos0 + n_q][n_kv * hd] of
 * kv_dtype, the query tokens' own rows already stored.  hd = 256 with
 * n_head / n_kv in {1, 2, 3, 4, 6, 8} and 16-byte aligned pointers takes the
 * split-position kernels; anything else a per-head kernel with the
 * reference's softmax sequence.  Uses library scratch. */
int bh_attention(const float *q, size_t n_q, size_t pos0, const void *k_cache,
                 const void *v_cache, int kv_dtype, size_t n_head, size_t n_kv, size_t hd,
                 float *out, bh_stream stream);

/* Planar-quantized KV cache (src/kvquant.rs, PlanarQuant; BONSAI_KV=planarN
 * and planarNk).  Per (position, kv head) a cache row holds the norm |x|
 * (f32) and, for the Givens-rotated unit vector, one Lloyd-Max centroid
 * index per coordinate packed LSB first at `bits` bits (1..8): kq/vq are
 * [cap][n_kv][packed_len] bytes, kn/vn [cap][n_kv] f32.  hd = 256 (the
 * model's head size).  The codebook and rotation table are the reference's
 * (computed by the library). */

/* Bytes of one packed row: ceil(hd_even * bits / 8) (packed_len,
 * src/kvquant.rs:332-334). */
size_t bh_planar_packed_len(size_t hd, unsigned bits);

/* AttnCache::append_k_quantized / append_v_quantized / append_v
 * (src/forward.rs:99-140): rows k, v [n_tok][n_kv * hd] (f32, 16-byte
 * aligned) quantized into positions pos0 .. pos0 + n_tok - 1; indices and
 * norms bit for bit the reference's.  vq = vn = NULL keeps V in f32
 * (planarNk): v is copied into v_f32 [cap][n_kv * hd].  No scratch. */
int bh_kv_store_planar(const float *k, const float *v, size_t n_tok, size_t n_kv, size_t hd,
                       unsigned bits, uint8_t *kq, float *kn, uint8_t *vq, float *vn,
                       float *v_f32, size_t pos0, bh_stream stream);

/* The quantized-cache branches of full_attention_layer (src/forward.rs
 * :296-349) for n_q query tokens at positions pos0 ..: q rotated once per
 * head, score_j = (q_rot . centroids(k_j)) |k_j| / sqrtf(hd), softmax_rows,
 * V quantized: the (p_j |v_j|)-weighted centroid sum turned back by the
 * inverse rotation; V in f32 (vq = vn = NULL): p . v_f32.  q, out
 * [n_q][n_head][hd]; n_head / n_kv in {1, 2, 3, 4, 6, 8}.  Uses library
 * scratch (like bh_attention).  A position whose probability is 0 adds
 * nothing, as the reference skips it (src/forward.rs:335) -- except on the
 * matrix-core path (many queries per kv head), where a quantized V row with
 * an infinite norm |v_j| gives NaN outputs for the rows that do not see it
 * (0 x inf inside the tile product); finite norms are unaffected. */
int bh_attention_planar(const float *q, size_t n_q, size_t pos0, const uint8_t *kq,
                        const float *kn, const uint8_t *vq, const float *vn, const float *v_f32,
                        unsigned bits, size_t n_head, size_t n_kv, size_t hd, float *out,
                        bh_stream stream);

/* Gated delta-net recurrence over n_tok tokens (src/gdn.rs:17-77, gdn_step,
 * applied per token; the reference fixes s = 128, h_k = 16, h_v = 48).  Per
 * token t and v-head h (q/k head h % h_k), with M = state[h] (s x s, row j
 * contiguous): M *= expf(gate[t][h]); delta[j] = (v[t][h][j] - M[j].k) *
 * beta[t][h]; M[j] += k * delta[j]; attn[t][h][j] = (M[j].q) / sqrtf(s).
 * q, k: [n_tok][h_k][s]; v, attn: [n_tok][h_v][s]; gate, beta: [n_tok][h_v];
 * state: [h_v][s][s], updated in place.  n_tok = 0 is a no-op.  With s = 128
 * and 128 or more tokens the batch runs in 64-token chunks on matrix cores
 * and uses library scratch (about 33 KB per chunk and v-head); fewer tokens
 * use none.  In that chunked form a non-finite q, k or v at token t also
 * makes the outputs of the chunk's earlier tokens non-finite (the chunk's
 * products include it with weight 0, and 0 x inf is NaN), where the
 * per-token reference leaves them finite; finite inputs are unaffected. */
int bh_gdn_step(const float *q, const float *k, const float *v, const float *gate,
                const float *beta, float *state, float *attn, size_t n_tok, size_t h_k,
                size_t h_v, size_t s, bh_stream stream);

/* ---------------------------------------------------------------------------
 * Softmax (src/kernels.rs:175-202; temperature: src/sampler.rs:85, 110)
 * ------------------------------------------------------------------------- */

/* out = softmax_rows(x * inv_temp, row_len): per row, max in f32,
 * e = expf(v - max), f64 sum, out = e * (1 / (f32)sum).  -inf entries give 0.
 * inv_temp = 1.0f is the plain kernels::softmax_rows; the sampler passes
 * 1.0f / temp.  BH_ERR_SHAPE when x_len % row_len != 0. */
int bh_softmax_rows(const float *x, size_t x_len, size_t row_len,
                    float inv_temp, float *out, bh_stream stream);

/* bh_softmax_rows with options.  flags = 0 is bh_softmax_rows;
 * BH_SOFTMAX_SAMPLER_NORM normalises as the sampler does
 * (src/sampler.rs:118-126: inv_sum = 1.0 / sum in f64, out =
 * (e as f64 * inv_sum) as f32) instead of kernels::softmax_rows'
 * e * (1 / (f32)sum) (src/kernels.rs:197-200); the two differ by at most
 * two f32 ulps.  Unknown flags: BH_ERR_ARG. */
#define BH_SOFTMAX_SAMPLER_NORM 1
int bh_softmax_rows_ex(const float *x, size_t x_len, size_t row_len,
                       float inv_temp, int flags, float *out, bh_stream stream);

/* No counterpart in the reference: bh_softmax_rows for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments, kernels and results as
 * bh_softmax_rows, but rows too wide for one workgroup keep their partials
 * in a fixed 1 MiB per-device array of the library (12 bytes per 4096-element
 * chunk of a row: up to 87381 chunks, e.g. 1432 rows of 248320) instead of
 * the growable scratch; larger inputs return BH_ERR_SHAPE.  Nothing is
 * allocated or freed.  Every call on one device shares that array: calls
 * that overlap in time on one device race. */
int bh_softmax_rows_noalloc(const float *x, size_t x_len, size_t row_len,
                            float inv_temp, float *out, bh_stream stream);

/* ---------------------------------------------------------------------------
 * Rotary embedding (src/rope.rs:9-70)
 * ------------------------------------------------------------------------- */

/* rope::rope_imrope over every head of n_tok tokens, in place:
 * heads[t][h][0..head_dim), positions pos[t][0..4) = (p_t, p_h, p_w, p_e).
 * theta_scale = powf(freq_base, -2/n_dims) is evaluated on the host with the
 * C library, and theta for pair j is the chain p * theta_scale * ... (j
 * multiplies in f32), as in the reference loop.  n_dims must be even and
 * <= head_dim. */
int bh_rope_imrope(float *heads, size_t n_tok, size_t n_head, size_t head_dim,
                   const int32_t *pos, size_t n_dims, const int32_t sections[4],
                   float freq_base, bh_stream stream);

/* Attention pre-block, fused (src/forward.rs:237-270):
 *   q_out = rope_imrope(rms_norm_rows(q, wq, head_dim, eps))
 *   k_out = rope_imrope(rms_norm_rows(k, wk, head_dim, eps))
 * q heads are read with stride q_head_stride floats: head_dim for a plain
 * [n_tok][n_q_head][head_dim] tensor, 2*head_dim for the fused attn_q output
 * whose rows are [q | gate] per head (src/forward.rs:237-241).  With
 * gate_out != NULL (requires q_head_stride == 2*head_dim) the gate half is
 * split out and passed through sigmoid (src/forward.rs:379):
 * gate_out[t][h] = sigmoid(gate).  k may be NULL when n_k_head == 0. */
typedef struct bh_qk_norm_rope_args {
  const float *q;      /* [n_tok][n_q_head][q_head_stride]  */
  float *q_out;        /* [n_tok][n_q_head][head_dim]       */
  float *gate_out;     /* [n_tok][n_q_head][head_dim] or NULL */
  const float *k;      /* [n_tok][n_k_head][head_dim]       */
  float *k_out;        /* [n_tok][n_k_head][head_dim]       */
  const float *wq;     /* [head_dim] attn_q_norm.weight     */
  const float *wk;     /* [head_dim] attn_k_norm.weight     */
  const int32_t *pos;  /* [n_tok][4] (p_t, p_h, p_w, p_e)   */
  size_t n_tok, n_q_head, n_k_head, head_dim, q_head_stride, n_dims;
  int32_t sections[4];
  float freq_base;
  float eps;
} bh_qk_norm_rope_args;

int bh_qk_norm_rope(const bh_qk_norm_rope_args *args, bh_stream stream);

/* ---------------------------------------------------------------------------
 * PQ2_0 ternary embedding rows (src/kernels.rs:204-229, src/gguf.rs:881-911)
 * ------------------------------------------------------------------------- */

/* kernels::pq2_row_bytes (src/kernels.rs:209-211): ceil(ne0/128) * 34. */
size_t bh_pq2_row_bytes(size_t ne0);

/* Batched Weights::row_f32 on a PQ2_0 tensor (src/weights.rs:333-349,
 * src/prefill.rs:143-154): out[i] = decode_pq2_0_row(table row ids[i]),
 * bit-exact.  table holds n_rows rows of bh_pq2_row_bytes(ne0) bytes.  An id
 * >= n_rows yields a zero row and, when bad_id != NULL, its value is stored
 * to *bad_id (device word; the caller presets it, e.g. to 0xFFFFFFFF, and
 * reads it after the stream completes). */
int bh_pq2_embed_gather(const uint8_t *table, size_t ne0, size_t n_rows,
                        const uint32_t *ids, size_t n_ids, float *out,
                        uint32_t *bad_id, bh_stream stream);

/* Embedding gather fused with the first RMSNorm (src/forward.rs:691, 701-702):
 * out_embed[i] = decode_pq2_0_row(row ids[i])      (bit-exact, the residual)
 * out_norm[i]  = rms_norm(out_embed[i], w, eps)    (blk.0.attn_norm)
 * Both outputs bit-exact: the row's sum of squares is the reference's
 * sequential f32 sum.  Batches of at least 16 ids per compute unit keep
 * their row scales in library scratch (n_ids * 4 bytes; see Threading).
 * BH_ERR_SHAPE when w_len != ne0. */
int bh_pq2_embed_gather_rms(const uint8_t *table, size_t ne0, size_t n_rows,
                            const uint32_t *ids, size_t n_ids, const float *w,
                            size_t w_len, float eps, float *out_embed,
                            float *out_norm, uint32_t *bad_id, bh_stream stream);

/* ---------------------------------------------------------------------------
 * PQ2_0 products (matrix cores).  payload is the tensor's whole PQ2_0 data on
 * the device (payload_len bytes, rows of bh_pq2_row_bytes(ne0) back to back);
 * the product reads rows base_row .. base_row + n_rows - 1.  Results agree
 * with the reference's scalar row dot to <= 1e-5 of the output's largest
 * magnitude (the summation order differs, as the reference's AVX2 path's
 * does).  Up to 4 tokens on rows of whole 1024-weight chunks (16-byte
 * aligned) the products keep x in LDS and use no scratch; otherwise they
 * use the library's per-device scratch (x fragments): such calls must not
 * overlap on one device.
 * ------------------------------------------------------------------------- */

/* kernels::pq2_matvec_range (src/kernels.rs:283-333):
 * y[r] = sum_j x[j] * W[base_row + r][j] for r < n_rows.  Errors (text of the
 * reference): x_len != ne0, y_len < n_rows, byte length overflow, rows past
 * payload_len. */
int bh_pq2_matvec_range(const uint8_t *payload, size_t payload_len, size_t ne0,
                        uint64_t base_row, size_t n_rows, const float *x,
                        size_t x_len, float *y, size_t y_len, bh_stream stream);

/* kernels::pq2_matmul_n (src/kernels.rs:340-423): x is [n_tok][ne0], y is
 * [n_tok][n_rows] (token-major), Y[t][r] = sum_j X[t][j] * W[base_row + r][j].
 * Each weight row is read once for all tokens.  Errors as the reference. */
int bh_pq2_matmul_n(const uint8_t *payload, size_t payload_len, size_t ne0,
                    uint64_t base_row, size_t n_rows, const float *x,
                    size_t x_len, size_t n_tok, float *y, size_t y_len,
                    bh_stream stream);

/* ---------------------------------------------------------------------------
 * Host-slice mirrors: the Rust signatures, host memory in and out.  Outputs
 * are caller-allocated with the length the Rust function would return.
 * ------------------------------------------------------------------------- */

/* kernels::rms_norm (src/kernels.rs:59); w has n entries. */
int bh_host_rms_norm(const float *x, size_t n, const float *w, float eps,
                     float *out);
/* kernels::rms_norm_rows (src/kernels.rs:97); out has x_len entries. */
int bh_host_rms_norm_rows(const float *x, size_t x_len, const float *w,
                          size_t w_len, size_t row_len, float eps, float *out);
/* kernels::l2_norm_rows (src/kernels.rs:126). */
int bh_host_l2_norm_rows(const float *x, size_t x_len, size_t row_len,
                         float eps, float *out);
/* kernels::map_inplace(x, silu|sigmoid|softplus) (src/kernels.rs:167). */
int bh_host_map_inplace(float *x, size_t n, int mode);
/* kernels::softmax_rows (src/kernels.rs:175). */
int bh_host_softmax_rows(const float *x, size_t x_len, size_t row_len,
                         float *out);
/* rope::rope_imrope on one head (src/rope.rs:9), in place. */
int bh_host_rope_imrope(float *head, size_t head_len, int64_t p_t, int64_t p_h,
                        int64_t p_w, int64_t p_e, size_t n_dims,
                        const int32_t sections[4], float freq_base);
/* kernels::decode_pq2_0_row (src/kernels.rs:214); raw has raw_len bytes
 * (>= bh_pq2_row_bytes(ne0)); out has ne0 entries. */
int bh_host_decode_pq2_0_row(const uint8_t *raw, size_t raw_len, size_t ne0,
                             float *out);
/* prefill::batch_embed (src/prefill.rs:143) over a PQ2_0 payload of n_rows
 * rows: out[k] = row_f32(tokens[k]); BH_ERR_RANGE on a token >= n_rows with
 * the message of src/weights.rs:337-341. */
int bh_host_batch_embed(const uint8_t *payload, size_t payload_len, size_t ne0,
                        size_t n_rows, const uint32_t *tokens, size_t n_tok,
                        float *out);
/* kernels::dot_pq2_0_row (src/kernels.rs:233-262): *out = row `row` . x. */
int bh_host_dot_pq2_0_row(const uint8_t *payload, size_t payload_len, size_t ne0,
                          uint64_t row, const float *x, size_t x_len, float *out);
/* kernels::pq2_matvec_range (src/kernels.rs:283-333), host slices; y has
 * y_len entries of which the first n_rows are written. */
int bh_host_pq2_matvec_range(const uint8_t *payload, size_t payload_len, size_t ne0,
                             uint64_t base_row, size_t n_rows, const float *x,
                             size_t x_len, float *y, size_t y_len);
/* kernels::pq2_matmul_n (src/kernels.rs:340-423), host slices. */
int bh_host_pq2_matmul_n(const uint8_t *payload, size_t payload_len, size_t ne0,
                         uint64_t base_row, size_t n_rows, const float *x,
                         size_t x_len, size_t n_tok, float *y, size_t y_len);

/* gdn_step, src/gdn.rs:17-77, with its fixed shape (s = 128, h_k = 16,
 * h_v = 48) and one token: q, k [16*128], v [48*128], gate, beta [48],
 * state [48*128*128] (advanced in place), attn [48*128] (written).  A slice
 * shorter than that is an error "gdn_step: <name> len L < N" (the
 * reference's indexing would panic). */
int bh_host_gdn_step(const float *q, size_t q_len, const float *k, size_t k_len, const float *v,
                     size_t v_len, const float *gate, size_t gate_len, const float *beta,
                     size_t beta_len, float *state, size_t state_len, float *attn,
                     size_t attn_len);

#ifdef __cplusplus
}
#endif

#endif /* BONSAI_HIP_H */
