/*
 * oracle.c -- CPU restatement of the reference's hot-path kernels.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product): loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
 *
 * Every function follows the cited Rust source of herlangga72/
 * ternary-bonsai-inference operation for operation.  Build flags (see
 * oracle/Makefile): -O2 -ffp-contract=off, no fast-math, glibc libm.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- f16 <-> f32 (src/gguf.rs:881-944) --------------------------------- */

static float bits_f32(uint32_t b) {
  float f;
  memcpy(&f, &b, 4);
  return f;
}

static uint32_t f32_bits(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return b;
}

/* src/gguf.rs:881-911 */
float or_half_to_f32(uint16_t h) {
  uint32_t sign = (h >> 15) & 1u;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign << 31;
    } else {
      int e = 127 - 15 + 1;
      uint32_t m = man;
      while ((m & 0x400u) == 0) {
        m <<= 1;
        e -= 1;
      }
      m &= 0x3ffu;
      bits = (sign << 31) | ((uint32_t)e << 23) | (m << 13);
    }
  } else if (exp == 0x1f) {
    bits = man == 0 ? ((sign << 31) | 0x7f800000u) : ((sign << 31) | 0x7f800000u | (man << 13));
  } else {
    bits = (sign << 31) | ((exp + 127 - 15) << 23) | (man << 13);
  }
  return bits_f32(bits);
}

/* src/gguf.rs:914-944 */
uint16_t or_f32_to_half(float v) {
  uint32_t b = f32_bits(v);
  uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
  int32_t exp = (int32_t)((b >> 23) & 0xffu);
  uint32_t man = b & 0x7fffffu;
  if (exp == 0xff) {
    uint16_t m = man != 0 ? 0x200 : 0;
    return (uint16_t)(sign | 0x7c00 | m);
  }
  int32_t e = exp - 127 + 15;
  if (e >= 0x1f) return (uint16_t)(sign | 0x7c00);
  if (e <= 0) {
    if (e < -10) return sign;
    uint32_t m = (man | 0x800000u) >> (uint32_t)(1 - e);
    uint16_t half = (uint16_t)(m >> 13);
    uint32_t rem = m & 0x1fffu;
    uint16_t out = (uint16_t)(half + ((rem > 0x1000u || (rem == 0x1000u && (half & 1u) == 1u)) ? 1 : 0));
    return (uint16_t)(sign | out);
  }
  uint16_t half = (uint16_t)(((uint32_t)e << 10) | (man >> 13));
  uint32_t rem = man & 0x1fffu;
  uint16_t out = (uint16_t)(half + ((rem > 0x1000u || (rem == 0x1000u && (half & 1u) == 1u)) ? 1 : 0));
  return (uint16_t)(sign | out);
}

void or_half_to_f32_n(const uint16_t *h, size_t n, float *out) {
  for (size_t i = 0; i < n; ++i) out[i] = or_half_to_f32(h[i]);
}

void or_f32_to_half_n(const float *v, size_t n, uint16_t *out) {
  for (size_t i = 0; i < n; ++i) out[i] = or_f32_to_half(v[i]);
}

/* ---- activations (src/kernels.rs:148-164) -------------------------------- */

float or_silu(float x) { return x / (1.0f + expf(-x)); }

float or_softplus(float x) { return x > 20.0f ? x : logf(1.0f + expf(x)); }

float or_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* map_inplace (src/kernels.rs:167-171) for modes 0-2; modes 3/4 are the
 * gated products at src/forward.rs:549-551 (normed[i] *= silu(z[i])) and
 * :379-382 (out[i] *= sigmoid(gate[i])). */
void or_unary(int mode, const float *a, const float *b, size_t n, float *out) {
  for (size_t i = 0; i < n; ++i) {
    float r;
    switch (mode) {
      case 0: r = or_silu(a[i]); break;
      case 1: r = or_sigmoid(a[i]); break;
      case 2: r = or_softplus(a[i]); break;
      case 3: r = b[i] * or_silu(a[i]); break;
      default: r = b[i] * or_sigmoid(a[i]); break;
    }
    out[i] = r;
  }
}

/* ---- norms ------------------------------------------------------------- */

/* src/kernels.rs:59-75 */
void or_rms_norm(const float *x, size_t n, const float *w, float eps, float *out) {
  if (n == 0) return;
  float ss = 0.0f;
  for (size_t i = 0; i < n; ++i) ss += x[i] * x[i];
  float mean = ss / (float)n;
  float scale = 1.0f / sqrtf(mean + eps);
  for (size_t i = 0; i < n; ++i) out[i] = x[i] * scale * w[i];
}

/* src/kernels.rs:97-122 */
int or_rms_norm_rows(const float *x, size_t x_len, const float *w, size_t w_len, size_t row_len,
                     float eps, float *out) {
  if (w_len != row_len) return OR_ERR_SHAPE;
  if (row_len == 0 || x_len % row_len != 0) return OR_ERR_SHAPE;
  for (size_t r = 0; r < x_len / row_len; ++r) {
    const float *src = x + r * row_len;
    float *dst = out + r * row_len;
    float ss = 0.0f;
    for (size_t i = 0; i < row_len; ++i) ss += src[i] * src[i];
    float scale = 1.0f / sqrtf(ss / (float)row_len + eps);
    for (size_t i = 0; i < row_len; ++i) dst[i] = src[i] * scale * w[i];
  }
  return OR_OK;
}

/* src/forward.rs:708-713 (cur[i] += attn_out[i]; rms_norm(cur, post_w, eps)) */
int or_add_rms_norm_rows(const float *x, const float *r, size_t x_len, const float *w,
                         size_t w_len, size_t row_len, float eps, float *sum_out, float *out) {
  if (w_len != row_len) return OR_ERR_SHAPE;
  if (row_len == 0 || x_len % row_len != 0) return OR_ERR_SHAPE;
  for (size_t i = 0; i < x_len; ++i) sum_out[i] = x[i] + r[i];
  return or_rms_norm_rows(sum_out, x_len, w, w_len, row_len, eps, out);
}

/* src/kernels.rs:126-145 */
int or_l2_norm_rows(const float *x, size_t x_len, size_t row_len, float eps, float *out) {
  if (row_len == 0 || x_len % row_len != 0) return OR_ERR_SHAPE;
  memmove(out, x, x_len * sizeof(float));
  for (size_t r = 0; r < x_len / row_len; ++r) {
    float *chunk = out + r * row_len;
    double sum = 0.0;
    for (size_t i = 0; i < row_len; ++i) sum += (double)chunk[i] * (double)chunk[i];
    float nrm = sqrtf((float)sum);
    /* f32::max returns the non-NaN operand, as fmaxf does */
    float scale = 1.0f / fmaxf(nrm, eps);
    for (size_t i = 0; i < row_len; ++i) chunk[i] *= scale;
  }
  return OR_OK;
}

/* ---- softmax (src/kernels.rs:175-202) ---------------------------------- */

int or_softmax_rows(const float *x, size_t x_len, size_t row_len, float inv_temp, float *out) {
  return or_softmax_rows_ex(x, x_len, row_len, inv_temp, 0, out);
}

/* flags & 1: the sampler's normalisation (src/sampler.rs:118-126): the sum
 * is the same f64 sum of the f32 exponentials, then inv_sum = 1.0 / sum in
 * f64 and each output is (e as f64 * inv_sum) as f32. */
int or_softmax_rows_ex(const float *x, size_t x_len, size_t row_len, float inv_temp, int flags,
                       float *out) {
  if (row_len == 0 || x_len % row_len != 0) return OR_ERR_SHAPE;
  float *y = (float *)malloc(row_len * sizeof(float));
  if (y == NULL) return OR_ERR_SHAPE;
  for (size_t r = 0; r < x_len / row_len; ++r) {
    const float *src = x + r * row_len;
    float *dst = out + r * row_len;
    /* src/sampler.rs:110: logits[i] * inv_t */
    for (size_t i = 0; i < row_len; ++i) y[i] = src[i] * inv_temp;
    float max = -INFINITY;
    for (size_t i = 0; i < row_len; ++i)
      if (y[i] > max) max = y[i];
    double sum = 0.0;
    for (size_t i = 0; i < row_len; ++i) {
      float e = expf(y[i] - max);
      dst[i] = e;
      sum += (double)e;
    }
    if (flags & 1) {
      double inv_sum = 1.0 / sum;
      for (size_t i = 0; i < row_len; ++i) dst[i] = (float)((double)dst[i] * inv_sum);
    } else {
      float inv = 1.0f / (float)sum;
      for (size_t i = 0; i < row_len; ++i) dst[i] *= inv;
    }
  }
  free(y);
  return OR_OK;
}

/* ---- IMROPE (src/rope.rs:9-70) ----------------------------------------- */

void or_rope_imrope(float *head, size_t head_len, int64_t p_t, int64_t p_h, int64_t p_w,
                    int64_t p_e, size_t n_dims, const int32_t sections[4], float freq_base) {
  (void)head_len;
  int64_t sect_dims = (int64_t)sections[0] + sections[1] + sections[2] + sections[3];
  float theta_scale = powf(freq_base, -2.0f / (float)n_dims);
  float th = (float)p_t, hh = (float)p_h, wh = (float)p_w, eh = (float)p_e;
  int64_t s0 = sections[0], s1 = sections[1], s2 = sections[2];
  float *cache = (float *)malloc((n_dims ? n_dims : 1) * sizeof(float));
  if (cache == NULL) return;
  for (size_t i0 = 0; i0 < n_dims; i0 += 2) {
    int64_t sector = ((int64_t)i0 / 2) % sect_dims;
    float theta;
    if (sector % 3 == 1 && sector < 3 * s1)
      theta = hh;
    else if (sector % 3 == 2 && sector < 3 * s2)
      theta = wh;
    else if (sector % 3 == 0 && sector < 3 * s0)
      theta = th;
    else
      theta = eh;
    cache[i0] = cosf(theta);
    cache[i0 + 1] = sinf(theta);
    th *= theta_scale;
    hh *= theta_scale;
    wh *= theta_scale;
    eh *= theta_scale;
  }
  size_t half = n_dims / 2;
  for (size_t j = 0; j < half; ++j) {
    float c = cache[2 * j], s = cache[2 * j + 1];
    float x0 = head[j], x1 = head[j + half];
    head[j] = x0 * c - x1 * s;
    head[j + half] = x0 * s + x1 * c;
  }
  free(cache);
}

/* src/forward.rs:237-270 (and the gate sigmoid of :379) for n_tok tokens */
int or_qk_norm_rope(const float *q, float *q_out, float *gate_out, const float *k, float *k_out,
                    const float *wq, const float *wk, const int32_t *pos, size_t n_tok,
                    size_t n_q_head, size_t n_k_head, size_t head_dim, size_t q_head_stride,
                    size_t n_dims, const int32_t sections[4], float freq_base, float eps) {
  float *qs = (float *)malloc((n_q_head * head_dim + 1) * sizeof(float));
  if (qs == NULL) return OR_ERR_SHAPE;
  for (size_t t = 0; t < n_tok; ++t) {
    const int32_t *p = pos + 4 * t;
    /* split [q | gate] per head (src/forward.rs:237-241) */
    for (size_t h = 0; h < n_q_head; ++h) {
      const float *src = q + (t * n_q_head + h) * q_head_stride;
      memcpy(qs + h * head_dim, src, head_dim * sizeof(float));
      if (gate_out != NULL)
        for (size_t d = 0; d < head_dim; ++d)
          gate_out[(t * n_q_head + h) * head_dim + d] = or_sigmoid(src[head_dim + d]);
    }
    float *qo = q_out + t * n_q_head * head_dim;
    int st = or_rms_norm_rows(qs, n_q_head * head_dim, wq, head_dim, head_dim, eps, qo);
    if (st != OR_OK) {
      free(qs);
      return st;
    }
    for (size_t h = 0; h < n_q_head; ++h)
      or_rope_imrope(qo + h * head_dim, head_dim, p[0], p[1], p[2], p[3], n_dims, sections,
                     freq_base);
    if (n_k_head > 0) {
      float *ko = k_out + t * n_k_head * head_dim;
      st = or_rms_norm_rows(k + t * n_k_head * head_dim, n_k_head * head_dim, wk, head_dim,
                            head_dim, eps, ko);
      if (st != OR_OK) {
        free(qs);
        return st;
      }
      for (size_t h = 0; h < n_k_head; ++h)
        or_rope_imrope(ko + h * head_dim, head_dim, p[0], p[1], p[2], p[3], n_dims, sections,
                       freq_base);
    }
  }
  free(qs);
  return OR_OK;
}

/* ---- PQ2_0 (src/kernels.rs:204-229) ------------------------------------ */

size_t or_pq2_row_bytes(size_t ne0) { return (ne0 + 127) / 128 * 34; }

void or_decode_pq2_0_row(const uint8_t *raw, size_t ne0, float *out) {
  size_t k = 0;
  for (size_t block = 0; block < (ne0 + 127) / 128; ++block) {
    size_t base = block * 34;
    float scale = or_half_to_f32((uint16_t)(raw[base] | (raw[base + 1] << 8)));
    const uint8_t *qs = raw + base + 2;
    for (size_t j = 0; j < 128; ++j) {
      if (block * 128 + j >= ne0) break;
      uint8_t code = (uint8_t)((qs[j / 4] >> ((j % 4) * 2)) & 0x03);
      out[k++] = (float)((int32_t)code - 1) * scale;
    }
  }
}

int or_embed_gather(const uint8_t *payload, size_t ne0, size_t n_rows, const uint32_t *tokens,
                    size_t n_tok, const float *w, float eps, float *out, float *out_norm,
                    uint32_t *bad) {
  size_t rb = or_pq2_row_bytes(ne0);
  for (size_t k = 0; k < n_tok; ++k) {
    if (tokens[k] >= n_rows) {
      if (bad) *bad = tokens[k];
      return OR_ERR_RANGE;
    }
    or_decode_pq2_0_row(payload + (size_t)tokens[k] * rb, ne0, out + k * ne0);
    if (out_norm != NULL) or_rms_norm(out + k * ne0, ne0, w, eps, out_norm + k * ne0);
  }
  return OR_OK;
}

/* ---- causal conv1d + SiLU (src/forward.rs:508-533) ------------------------ */

/* Per token, per channel: win = [state[c][0..k-1), x[t][c]] (oldest first),
 * acc = sum_j w[c*k + j] * win[j] in f32, j ascending, out = silu(acc); then
 * the state drops its oldest sample and appends x[t][c] (:526-532).  state is
 * [ch][k-1] and is updated in place; k >= 1. */
void or_conv1d_silu(const float *x, float *state, const float *w, size_t n_tok, size_t ch,
                    size_t k, float *out) {
  size_t n_prev = k - 1;
  float win[64];
  for (size_t t = 0; t < n_tok; ++t) {
    for (size_t c = 0; c < ch; ++c) {
      for (size_t j = 0; j < n_prev; ++j) win[j] = state[c * n_prev + j];
      win[n_prev] = x[t * ch + c];
      float acc = 0.0f;
      for (size_t j = 0; j < k; ++j) acc += w[c * k + j] * win[j];
      out[t * ch + c] = or_silu(acc);
    }
    for (size_t c = 0; c < ch; ++c) {
      if (n_prev == 0) continue;
      for (size_t j = 0; j + 1 < n_prev; ++j) state[c * n_prev + j] = state[c * n_prev + j + 1];
      state[c * n_prev + n_prev - 1] = x[t * ch + c];
    }
  }
}

/* ---- gated delta-net recurrence (src/gdn.rs:17-77) ------------------------- */

/* gdn_step applied to n_tok tokens in order.  Per token t and v-head h (k/q
 * head h % h_k): M = state[h] (s x s, row j contiguous) *= expf(gate);
 * delta[j] = (v[j] - sum_i M[j][i] k[i]) * beta; M[j][i] += k[i] * delta[j];
 * attn[j] = (sum_i M[j][i] q[i]) * (1 / sqrtf(s)); sums in f32, i ascending.
 * q, k: [n_tok][h_k][s]; v, attn: [n_tok][h_v][s]; gate, beta: [n_tok][h_v];
 * state: [h_v][s][s], updated in place. */
void or_gdn_step(const float *q, const float *k, const float *v, const float *gate,
                 const float *beta, float *state, float *attn, size_t n_tok, size_t h_k,
                 size_t h_v, size_t s) {
  float scale = 1.0f / sqrtf((float)s);
  float *delta = (float *)malloc(s * sizeof(float));
  if (delta == NULL) return;
  for (size_t t = 0; t < n_tok; ++t) {
    for (size_t h = 0; h < h_v; ++h) {
      const float *qv = q + (t * h_k + h % h_k) * s;
      const float *kv = k + (t * h_k + h % h_k) * s;
      const float *vv = v + (t * h_v + h) * s;
      float *m = state + h * s * s;
      float eg = expf(gate[t * h_v + h]);
      for (size_t x = 0; x < s * s; ++x) m[x] *= eg;
      for (size_t j = 0; j < s; ++j) {
        float sum = 0.0f;
        for (size_t i = 0; i < s; ++i) sum += m[j * s + i] * kv[i];
        delta[j] = (vv[j] - sum) * beta[t * h_v + h];
      }
      for (size_t j = 0; j < s; ++j)
        for (size_t i = 0; i < s; ++i) m[j * s + i] += kv[i] * delta[j];
      float *out = attn + (t * h_v + h) * s;
      for (size_t j = 0; j < s; ++j) {
        float sum = 0.0f;
        for (size_t i = 0; i < s; ++i) sum += m[j * s + i] * qv[i];
        out[j] = sum * scale;
      }
    }
  }
  free(delta);
}

/* ---- attention over a KV cache (src/forward.rs:273-375) ------------------ */

/* AttnCache::append / append_f16, src/forward.rs:90-95, 120-125: the rows of
 * n_tok tokens (n_kv_elems floats each) land at positions pos0 .. of the
 * cache, f32 or converted by gguf::f32_to_half. */
void or_kv_store(const float *k, const float *v, size_t n_tok, size_t n_kv_elems, void *k_cache,
                 void *v_cache, size_t pos0, int kv_f16) {
  size_t n = n_tok * n_kv_elems, base = pos0 * n_kv_elems;
  for (size_t i = 0; i < n; ++i) {
    if (kv_f16) {
      ((uint16_t *)k_cache)[base + i] = or_f32_to_half(k[i]);
      ((uint16_t *)v_cache)[base + i] = or_f32_to_half(v[i]);
    } else {
      ((float *)k_cache)[base + i] = k[i];
      ((float *)v_cache)[base + i] = v[i];
    }
  }
}

static float kv_at(const void *cache, int kv_f16, size_t i) {
  return kv_f16 ? or_half_to_f32(((const uint16_t *)cache)[i]) : ((const float *)cache)[i];
}

/* The GQA block of full_attention_layer, src/forward.rs:282-375, for n_q
 * query tokens at positions pos0 .. pos0 + n_q - 1 (one call per token in
 * the reference; token i sees cache positions 0 .. pos0 + i).  Per q head
 * hq (kv head hq / (n_head / n_kv)): scores[j] = dot(q, k_j) * scale with
 * dot / dot_f16 (:181-191: f32 products summed in index order) and scale =
 * 1 / sqrtf(hd) (:282); probs = softmax_rows (:326); out[d] = sum_j p_j *
 * v_j[d] in position order, skipping p_j == 0 (:361-371, f16 :349-360). */
int or_attention(const float *q, size_t n_q, size_t pos0, const void *k_cache,
                 const void *v_cache, int kv_f16, size_t n_head, size_t n_kv, size_t hd,
                 float *out) {
  if (n_kv == 0 || hd == 0 || n_head % n_kv != 0) return OR_ERR_SHAPE;
  size_t n_rep = n_head / n_kv, n_kv_elems = n_kv * hd, n_max = pos0 + n_q;
  float scale = 1.0f / sqrtf((float)hd);
  float *scores = (float *)malloc((n_max ? n_max : 1) * sizeof(float));
  float *probs = (float *)malloc((n_max ? n_max : 1) * sizeof(float));
  if (scores == NULL || probs == NULL) {
    free(scores);
    free(probs);
    return OR_ERR_SHAPE;
  }
  for (size_t i = 0; i < n_q; ++i) {
    size_t n_pos = pos0 + i + 1;
    for (size_t hq = 0; hq < n_head; ++hq) {
      const float *qh = q + (i * n_head + hq) * hd;
      size_t kv_off = (hq / n_rep) * hd;
      for (size_t j = 0; j < n_pos; ++j) {
        float sum = 0.0f;
        size_t row = j * n_kv_elems + kv_off;
        for (size_t d = 0; d < hd; ++d) sum += qh[d] * kv_at(k_cache, kv_f16, row + d);
        scores[j] = sum * scale;
      }
      or_softmax_rows(scores, n_pos, n_pos, 1.0f, probs);
      float *o = out + (i * n_head + hq) * hd;
      for (size_t d = 0; d < hd; ++d) o[d] = 0.0f;
      for (size_t j = 0; j < n_pos; ++j) {
        float pj = probs[j];
        if (pj == 0.0f) continue;
        size_t row = j * n_kv_elems + kv_off;
        for (size_t d = 0; d < hd; ++d) o[d] += pj * kv_at(v_cache, kv_f16, row + d);
      }
    }
  }
  free(scores);
  free(probs);
  return OR_OK;
}

/* ---- PQ2_0 products (src/kernels.rs:233-423) ------------------------------ */

/* row_dot_scalar, src/kernels.rs:633-653: per 128-block an f32 sum of
 * x[j] * (code - 1) in column order, then acc += scale * block_acc. */
float or_pq2_row_dot(const uint8_t *raw, size_t ne0, const float *x) {
  size_t n_blocks = (ne0 + 127) / 128;
  float acc = 0.0f;
  for (size_t block = 0; block < n_blocks; ++block) {
    size_t b = block * 34;
    float scale = or_half_to_f32((uint16_t)(raw[b] | (raw[b + 1] << 8)));
    const uint8_t *qs = raw + b + 2;
    size_t start = block * 128, end = start + 128 < ne0 ? start + 128 : ne0;
    float block_acc = 0.0f;
    for (size_t j = start; j < end; ++j) {
      uint8_t code = (uint8_t)((qs[(j - start) / 4] >> (((j - start) % 4) * 2)) & 0x03);
      block_acc += x[j] * (float)((int32_t)code - 1);
    }
    acc += scale * block_acc;
  }
  return acc;
}

/* pq2_matmul_n, src/kernels.rs:340-423 (and pq2_matvec_range when n_tok is
 * 1): y[t][r] = row_dot(W[base_row + r], x[t]); y is [n_tok][n_rows].  The
 * caller has checked the payload length. */
void or_pq2_matmul_n(const uint8_t *payload, size_t ne0, uint64_t base_row, size_t n_rows,
                     const float *x, size_t n_tok, float *y) {
  size_t rb = or_pq2_row_bytes(ne0);
  for (size_t r = 0; r < n_rows; ++r)
    for (size_t t = 0; t < n_tok; ++t)
      y[t * n_rows + r] = or_pq2_row_dot(payload + ((size_t)base_row + r) * rb, ne0, x + t * ne0);
}

/* ---- GDN gate prep (src/forward.rs:497-507, 524, 539-540) ---------------- */

void or_gdn_gate_prep(const float *alpha_raw, const float *dt_bias, const float *ssm_a,
                      const float *beta_raw, size_t n_tok, size_t n_head, float *gate_out,
                      float *beta_out) {
  for (size_t t = 0; t < n_tok; ++t) {
    for (size_t h = 0; h < n_head; ++h) {
      size_t i = t * n_head + h;
      float beta = or_sigmoid(beta_raw[i]);
      float alpha = or_softplus(alpha_raw[i] + dt_bias[h]);
      if (beta_out) beta_out[i] = beta;
      if (gate_out) gate_out[i] = alpha * ssm_a[h];
    }
  }
}

int or_silu_l2_part(const float *conv, size_t n_tok, size_t conv_dim, size_t l2_dim,
                    size_t head_dim, float eps, float *conv_out) {
  if (head_dim == 0 || l2_dim % head_dim != 0 || l2_dim > conv_dim) return OR_ERR_SHAPE;
  for (size_t t = 0; t < n_tok; ++t) {
    const float *c = conv + t * conv_dim;
    float *o = conv_out + t * conv_dim;
    for (size_t i = 0; i < conv_dim; ++i) o[i] = or_silu(c[i]);
    if (l2_dim > 0) {
      int st = or_l2_norm_rows(o, l2_dim, head_dim, eps, o);
      if (st != OR_OK) return st;
    }
  }
  return OR_OK;
}
