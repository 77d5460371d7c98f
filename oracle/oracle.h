/*
 * oracle.h -- CPU restatement of the reference's hot-path kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker the HIP library is compared
 * against; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  The product path never calls it.
 *
 * Each function restates, operation for operation, a Rust function of the
 * reference (citations per function).  Built with gcc -O2 -ffp-contract=off
 * and no fast-math against glibc libm, it reproduces the x86-64 build of the
 * reference: same f32/f64 types, same summation order, same libm calls
 * (Rust's f32::exp/ln/powf/sin/cos call expf/logf/powf/sinf/cosf).
 */
#ifndef BONSAI_ORACLE_H
#define BONSAI_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_OK 0
#define OR_ERR_SHAPE (-1)
#define OR_ERR_RANGE (-2)

/* src/gguf.rs:881-911 */
float or_half_to_f32(uint16_t h);
/* src/gguf.rs:914-944 */
uint16_t or_f32_to_half(float v);
/* vector forms of the two above (n values) */
void or_half_to_f32_n(const uint16_t *h, size_t n, float *out);
void or_f32_to_half_n(const float *v, size_t n, uint16_t *out);

/* src/kernels.rs:148-164 */
float or_silu(float x);
float or_softplus(float x);
float or_sigmoid(float x);
/* mode 0 silu, 1 sigmoid, 2 softplus (b unused), 3 b*silu(a), 4 b*sigmoid(a) */
void or_unary(int mode, const float *a, const float *b, size_t n, float *out);

/* src/kernels.rs:59-75 */
void or_rms_norm(const float *x, size_t n, const float *w, float eps, float *out);
/* src/kernels.rs:97-122 */
int or_rms_norm_rows(const float *x, size_t x_len, const float *w, size_t w_len,
                     size_t row_len, float eps, float *out);
/* src/forward.rs:708-713: sum = x + r; out = rms_norm_rows(sum) */
int or_add_rms_norm_rows(const float *x, const float *r, size_t x_len, const float *w,
                         size_t w_len, size_t row_len, float eps, float *sum_out, float *out);
/* src/kernels.rs:126-145 */
int or_l2_norm_rows(const float *x, size_t x_len, size_t row_len, float eps, float *out);
/* src/kernels.rs:175-202 applied to x * inv_temp (src/sampler.rs:85, 110) */
int or_softmax_rows(const float *x, size_t x_len, size_t row_len, float inv_temp, float *out);
/* flags & 1: the sampler's normalisation, (e as f64 * (1.0 / sum)) as f32
 * (src/sampler.rs:118-126) */
int or_softmax_rows_ex(const float *x, size_t x_len, size_t row_len, float inv_temp, int flags,
                       float *out);

/* src/rope.rs:9-70, in place on one head */
void or_rope_imrope(float *head, size_t head_len, int64_t p_t, int64_t p_h, int64_t p_w,
                    int64_t p_e, size_t n_dims, const int32_t sections[4], float freq_base);
/* src/forward.rs:237-270 + :379: per token, split q|gate (q_head_stride),
 * rms_norm_rows on q and k heads, rope_imrope per head (pos[t][4]), and
 * gate_out = sigmoid(gate) when non-NULL. */
int or_qk_norm_rope(const float *q, float *q_out, float *gate_out, const float *k, float *k_out,
                    const float *wq, const float *wk, const int32_t *pos, size_t n_tok,
                    size_t n_q_head, size_t n_k_head, size_t head_dim, size_t q_head_stride,
                    size_t n_dims, const int32_t sections[4], float freq_base, float eps);

/* src/kernels.rs:209-211 */
size_t or_pq2_row_bytes(size_t ne0);
/* src/kernels.rs:214-229 */
void or_decode_pq2_0_row(const uint8_t *raw, size_t ne0, float *out);
/* src/prefill.rs:143-154 via src/weights.rs:333-349, then optionally the
 * first rms_norm (src/forward.rs:701-702) when out_norm != NULL.
 * Returns OR_ERR_RANGE (and *bad = token) on the first token >= n_rows. */
int or_embed_gather(const uint8_t *payload, size_t ne0, size_t n_rows, const uint32_t *tokens,
                    size_t n_tok, const float *w, float eps, float *out, float *out_norm,
                    uint32_t *bad);

/* src/forward.rs:497-507 */
void or_gdn_gate_prep(const float *alpha_raw, const float *dt_bias, const float *ssm_a,
                      const float *beta_raw, size_t n_tok, size_t n_head, float *gate_out,
                      float *beta_out);
/* src/forward.rs:524 + 539-540: conv_out = silu(conv), then l2_norm_rows over
 * the first l2_dim channels of each token row, head_dim at a time. */
int or_silu_l2_part(const float *conv, size_t n_tok, size_t conv_dim, size_t l2_dim,
                    size_t head_dim, float eps, float *conv_out);

/* src/kernels.rs:633-653 (row_dot_scalar) */
float or_pq2_row_dot(const uint8_t *raw, size_t ne0, const float *x);
/* src/kernels.rs:340-423 / :283-333: y [n_tok][n_rows] */
void or_pq2_matmul_n(const uint8_t *payload, size_t ne0, uint64_t base_row, size_t n_rows,
                     const float *x, size_t n_tok, float *y);

/* src/forward.rs:508-533, per token in order; state [ch][k-1] in/out, k <= 64 */
void or_conv1d_silu(const float *x, float *state, const float *w, size_t n_tok, size_t ch,
                    size_t k, float *out);

/* src/gdn.rs:17-77 over n_tok tokens; state [h_v][s][s] in/out */
void or_kv_store(const float *k, const float *v, size_t n_tok, size_t n_kv_elems, void *k_cache,
                 void *v_cache, size_t pos0, int kv_f16);
int or_attention(const float *q, size_t n_q, size_t pos0, const void *k_cache,
                 const void *v_cache, int kv_f16, size_t n_head, size_t n_kv, size_t hd,
                 float *out);
void or_gdn_step(const float *q, const float *k, const float *v, const float *gate,
                 const float *beta, float *state, float *attn, size_t n_tok, size_t h_k,
                 size_t h_v, size_t s);

/* Planar-quantized KV cache, src/kvquant.rs (PlanarQuant) and
 * src/forward.rs:99-112, 128-140, 296-349.  bits 1..8, hd even. */
void or_planar_codebook(size_t d, unsigned bits, float *out);          /* 2^bits centroids */
double or_planar_distortion(size_t d, unsigned bits);                  /* expected MSE */
void or_planar_givens(size_t d, float *c, float *s);                   /* ceil(d/2) pairs */
size_t or_planar_packed_len(size_t hd, unsigned bits);
void or_planar_pack(const uint8_t *idx, size_t n, unsigned bits, uint8_t *out);
void or_planar_unpack(const uint8_t *packed, size_t n, unsigned bits, uint8_t *out);
void or_planar_rotate(const float *x, size_t hd, const float *c, const float *s, float *out);
void or_planar_quantize(const float *x, size_t hd, unsigned bits, uint8_t *packed, float *norm);
void or_planar_dequantize(const uint8_t *packed, float norm, size_t hd, unsigned bits, float *out);
float or_planar_dot_rotated(const float *q_rot, const uint8_t *packed, float norm, size_t hd,
                            unsigned bits);
void or_kv_store_planar(const float *k, const float *v, size_t n_tok, size_t n_kv, size_t hd,
                        unsigned bits, uint8_t *kq, float *kn, uint8_t *vq, float *vn,
                        float *v_f32, size_t pos0);
int or_attention_planar(const float *q, size_t n_q, size_t pos0, const uint8_t *kq,
                        const float *kn, const uint8_t *vq, const float *vn, const float *v_f32,
                        unsigned bits, size_t n_head, size_t n_kv, size_t hd, float *out);

#ifdef __cplusplus
}
#endif

#endif
