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

/* ---- planar-quantized KV cache (src/kvquant.rs) -------------------------- */

/* erf by Abramowitz & Stegun 7.1.26, src/kvquant.rs:34-44 */
static double pq_erf(double x) {
  double sign = x < 0.0 ? -1.0 : 1.0;
  x = fabs(x);
  double t = 1.0 / (1.0 + 0.3275911 * x);
  double y = 1.0 - (((((1.061405429 * t - 1.453152027) * t) + 1.421413741) * t - 0.284496736) * t +
                    0.254829592) *
                       t * exp(-x * x);
  return sign * y;
}
static double pq_cdf(double x, double sigma) {
  return 0.5 * (1.0 + pq_erf(x / (sigma * 1.4142135623730951)));
}
static double pq_pdf(double x, double sigma) {
  return exp(-(x * x) / (2.0 * sigma * sigma)) / (sigma * sqrt(2.0 * 3.141592653589793));
}
static double pq_m1(double a, double b, double sigma) {
  return sigma * sigma * (pq_pdf(a, sigma) - pq_pdf(b, sigma));
}

/* solve_lloyd_max + codebook, src/kvquant.rs:58-118: sigma = 1/sqrt(d),
 * 2^bits centroids started evenly over +-3.5 sigma, edges at midpoints and
 * +-12 sigma, up to 300 updates c_i = E[X | edge_i < X < edge_i+1] (kept
 * when the cell's mass is <= 1e-15), stopping when no centroid moves by
 * 1e-12; then rounded to f32. */
void or_planar_codebook(size_t d, unsigned bits, float *out) {
  size_t n = (size_t)1 << bits;
  double sigma = 1.0 / sqrt((double)d);
  double lo = -3.5 * sigma, hi = 3.5 * sigma, outer = 12.0 * sigma;
  double c[256], nx[256], e[257];
  for (size_t i = 0; i < n; ++i) c[i] = lo + (hi - lo) * ((double)i + 0.5) / (double)n;
  for (int it = 0; it < 300; ++it) {
    e[0] = -outer;
    for (size_t i = 0; i + 1 < n; ++i) e[i + 1] = (c[i] + c[i + 1]) / 2.0;
    e[n] = outer;
    double shift = 0.0;
    for (size_t i = 0; i < n; ++i) {
      double mass = pq_cdf(e[i + 1], sigma) - pq_cdf(e[i], sigma);
      nx[i] = mass > 1e-15 ? pq_m1(e[i], e[i + 1], sigma) / mass : c[i];
    }
    for (size_t i = 0; i < n; ++i) {
      double dlt = fabs(nx[i] - c[i]);
      if (dlt > shift) shift = dlt;
      c[i] = nx[i];
    }
    if (shift < 1e-12) break;
  }
  for (size_t i = 0; i < n; ++i) out[i] = (float)c[i];
}

/* kvquant_expected_distortion, src/kvquant.rs:854-880 */
double or_planar_distortion(size_t d, unsigned bits) {
  size_t n = (size_t)1 << bits;
  double sigma = 1.0 / sqrt((double)d), outer = 12.0 * sigma;
  float c[256];
  double e[257], dist = 0.0;
  or_planar_codebook(d, bits, c);
  e[0] = -outer;
  for (size_t i = 0; i + 1 < n; ++i) e[i + 1] = ((double)c[i] + (double)c[i + 1]) / 2.0;
  e[n] = outer;
  for (size_t i = 0; i < n; ++i) {
    double a = e[i], b = e[i + 1], c0 = (double)c[i];
    double mass = pq_cdf(b, sigma) - pq_cdf(a, sigma);
    double m1 = pq_m1(a, b, sigma);
    double m2 = sigma * sigma * (mass + a * pq_pdf(a, sigma) - b * pq_pdf(b, sigma));
    dist += m2 - 2.0 * c0 * m1 + c0 * c0 * mass;
  }
  return (double)(float)dist;
}

/* givens_table, src/kvquant.rs:124-146: splitmix64 from state 42, u =
 * (r >> 11) / 2^53, t = 2 pi u in f64, (cos t, sin t) rounded to f32. */
void or_planar_givens(size_t d, float *c, float *s) {
  uint64_t st = 42;
  for (size_t i = 0; i < (d + 1) / 2; ++i) {
    uint64_t z = (st += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    double u = (double)(z >> 11) / 9007199254740992.0;
    double t = u * 6.283185307179586;
    c[i] = (float)cos(t);
    s[i] = (float)sin(t);
  }
}

/* packed_bytes(hd_padded, bits), src/kvquant.rs:182-184, 332-334 */
size_t or_planar_packed_len(size_t hd, unsigned bits) {
  size_t hp = (hd + 1) / 2 * 2;
  return (hp * bits + 7) / 8;
}

/* pack_idx / unpack_idx, src/kvquant.rs:150-330.  For the rows here (an
 * even count, and a multiple of 8 for 3 bits) every layout the reference
 * picks -- 8-coordinate groups in 3 bytes for 3 bits, single planes for 1,
 * 2 and 4 bits, the LSB-first bitstream otherwise -- places coordinate i at
 * bits [i bits, (i + 1) bits) of the little-endian byte string; the
 * bitstream is written directly (the equivalence is a test). */
void or_planar_pack(const uint8_t *idx, size_t n, unsigned bits, uint8_t *out) {
  size_t nb = (n * bits + 7) / 8;
  memset(out, 0, nb);
  size_t bitpos = 0;
  for (size_t i = 0; i < n; ++i) {
    size_t byte = bitpos >> 3;
    unsigned off = (unsigned)(bitpos & 7);
    unsigned v = idx[i] & ((1u << bits) - 1u);
    out[byte] |= (uint8_t)((v << off) & 0xffu);
    if (off + bits > 8) out[byte + 1] |= (uint8_t)(v >> (8 - off));
    bitpos += bits;
  }
}
void or_planar_unpack(const uint8_t *packed, size_t n, unsigned bits, uint8_t *out) {
  unsigned mask = (1u << bits) - 1u;
  size_t bitpos = 0;
  for (size_t i = 0; i < n; ++i) {
    size_t byte = bitpos >> 3;
    unsigned off = (unsigned)(bitpos & 7);
    unsigned v = (unsigned)packed[byte] >> off;
    if (off + bits > 8) v |= (unsigned)packed[byte + 1] << (8 - off);
    out[i] = (uint8_t)(v & mask);
    bitpos += bits;
  }
}

/* PlanarQuant::rotate, src/kvquant.rs:356-366: pair i (2i, 2i+1) by
 * (c_i, s_i): [c a - s b, s a + c b] */
void or_planar_rotate(const float *x, size_t hd, const float *c, const float *s, float *out) {
  for (size_t i = 0; i < (hd + 1) / 2; ++i) {
    float a = 2 * i < hd ? x[2 * i] : 0.0f, b = 2 * i + 1 < hd ? x[2 * i + 1] : 0.0f;
    out[2 * i] = c[i] * a - s[i] * b;
    out[2 * i + 1] = s[i] * a + c[i] * b;
  }
}

/* PlanarQuant::quantize, src/kvquant.rs:381-396 (nearest :341-353: the
 * first centroid of least |v - c|) */
void or_planar_quantize(const float *x, size_t hd, unsigned bits, uint8_t *packed, float *norm) {
  size_t hp = (hd + 1) / 2 * 2, nc = (size_t)1 << bits;
  float cb[256], gc[128], gs[128], unit[256], rot[256];
  uint8_t idx[256];
  or_planar_codebook(hd, bits, cb);
  or_planar_givens(hd, gc, gs);
  float ss = 0.0f;
  for (size_t i = 0; i < hd; ++i) ss += x[i] * x[i];
  float n = sqrtf(ss);
  *norm = n;
  float inv = n > 1e-12f ? 1.0f / n : 0.0f;
  for (size_t i = 0; i < hp; ++i) unit[i] = i < hd ? x[i] * inv : 0.0f;
  or_planar_rotate(unit, hp, gc, gs, rot);
  for (size_t i = 0; i < hp; ++i) {
    size_t best = 0;
    float bd = fabsf(rot[i] - cb[0]);
    for (size_t k = 1; k < nc; ++k) {
      float dk = fabsf(rot[i] - cb[k]);
      if (dk < bd) {
        bd = dk;
        best = k;
      }
    }
    idx[i] = (uint8_t)best;
  }
  or_planar_pack(idx, hp, bits, packed);
}

/* PlanarQuant::dequantize, src/kvquant.rs:399-413 (rotate_inv :369-378) */
void or_planar_dequantize(const uint8_t *packed, float norm, size_t hd, unsigned bits, float *out) {
  size_t hp = (hd + 1) / 2 * 2;
  float cb[256], gc[128], gs[128], rot[256];
  uint8_t idx[256];
  or_planar_codebook(hd, bits, cb);
  or_planar_givens(hd, gc, gs);
  or_planar_unpack(packed, hp, bits, idx);
  for (size_t i = 0; i < hp; ++i) rot[i] = cb[idx[i]];
  for (size_t i = 0; i < hp / 2; ++i) {
    float a = rot[2 * i], b = rot[2 * i + 1];
    float u0 = gc[i] * a + gs[i] * b, u1 = -gs[i] * a + gc[i] * b;
    if (2 * i < hd) out[2 * i] = u0 * norm;
    if (2 * i + 1 < hd) out[2 * i + 1] = u1 * norm;
  }
}

/* PlanarQuant::dot_rotated_scratch, src/kvquant.rs:444-460: f32 sum in
 * index order of q_rot[i] * c[idx_i] over i < hd, times the norm */
/* the dot against a given codebook (the attention loop builds it once) */
static float planar_dot_cb(const float *q_rot, const uint8_t *packed, float norm, size_t hd,
                           unsigned bits, const float *cb) {
  size_t hp = (hd + 1) / 2 * 2;
  uint8_t idx[256];
  or_planar_unpack(packed, hp, bits, idx);
  float acc = 0.0f;
  for (size_t i = 0; i < hd; ++i) acc += q_rot[i] * cb[idx[i]];
  return acc * norm;
}

float or_planar_dot_rotated(const float *q_rot, const uint8_t *packed, float norm, size_t hd,
                            unsigned bits) {
  float cb[256];
  or_planar_codebook(hd, bits, cb);
  return planar_dot_cb(q_rot, packed, norm, hd, bits, cb);
}

/* AttnCache::append_k_quantized / append_v_quantized / append_v,
 * src/forward.rs:99-118, 128-140: per token and kv head, packed indices at
 * kq[(pos * n_kv + kv) * packed_len] and the norm at kn[pos * n_kv + kv];
 * v likewise into vq / vn, or (vq == NULL) as f32 rows into v_f32. */
void or_kv_store_planar(const float *k, const float *v, size_t n_tok, size_t n_kv, size_t hd,
                        unsigned bits, uint8_t *kq, float *kn, uint8_t *vq, float *vn,
                        float *v_f32, size_t pos0) {
  size_t plen = or_planar_packed_len(hd, bits);
  for (size_t t = 0; t < n_tok; ++t)
    for (size_t h = 0; h < n_kv; ++h) {
      size_t r = (pos0 + t) * n_kv + h;
      or_planar_quantize(k + (t * n_kv + h) * hd, hd, bits, kq + r * plen, kn + r);
      if (vq != NULL)
        or_planar_quantize(v + (t * n_kv + h) * hd, hd, bits, vq + r * plen, vn + r);
      else
        memcpy(v_f32 + r * hd, v + (t * n_kv + h) * hd, hd * sizeof(float));
    }
}

/* The quantized branches of full_attention_layer, src/forward.rs:296-349:
 * per q head, q rotated once; score_j = dot_rotated(q_rot, k_j, |k_j|) *
 * scale; probs = softmax_rows; V quantized: head_out[d] += (p_j |v_j|) *
 * c[idx_jd] over positions with p_j != 0, then the inverse rotation in
 * place; V in f32: head_out[d] += p_j * v_j[d].  Token i of n_q sees
 * positions 0 .. pos0 + i. */
int or_attention_planar(const float *q, size_t n_q, size_t pos0, const uint8_t *kq,
                        const float *kn, const uint8_t *vq, const float *vn, const float *v_f32,
                        unsigned bits, size_t n_head, size_t n_kv, size_t hd, float *out) {
  if (n_kv == 0 || hd == 0 || hd % 2 != 0 || hd > 256 || n_head % n_kv != 0 || bits < 1 ||
      bits > 8)
    return OR_ERR_SHAPE;
  size_t n_rep = n_head / n_kv, n_max = pos0 + n_q, plen = or_planar_packed_len(hd, bits);
  float scale = 1.0f / sqrtf((float)hd);
  float cb[256], gc[128], gs[128], qrot[256], vrot[256];
  uint8_t idx[256];
  or_planar_codebook(hd, bits, cb);
  or_planar_givens(hd, gc, gs);
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
      size_t kv = hq / n_rep;
      or_planar_rotate(q + (i * n_head + hq) * hd, hd, gc, gs, qrot);
      for (size_t j = 0; j < n_pos; ++j) {
        size_t r = j * n_kv + kv;
        scores[j] = planar_dot_cb(qrot, kq + r * plen, kn[r], hd, bits, cb) * scale;
      }
      or_softmax_rows(scores, n_pos, n_pos, 1.0f, probs);
      float *o = out + (i * n_head + hq) * hd;
      for (size_t d = 0; d < hd; ++d) o[d] = 0.0f;
      for (size_t j = 0; j < n_pos; ++j) {
        float pj = probs[j];
        if (pj == 0.0f) continue;
        size_t r = j * n_kv + kv;
        if (vq != NULL) {
          or_planar_unpack(vq + r * plen, hd, bits, idx);
          for (size_t d = 0; d < hd; ++d) vrot[d] = cb[idx[d]];
          float w = pj * vn[r];
          for (size_t d = 0; d < hd; ++d) o[d] += w * vrot[d];
        } else {
          for (size_t d = 0; d < hd; ++d) o[d] += pj * v_f32[r * hd + d];
        }
      }
      if (vq != NULL)
        for (size_t p2 = 0; p2 < hd / 2; ++p2) {
          float a = o[2 * p2], b = o[2 * p2 + 1];
          o[2 * p2] = gc[p2] * a + gs[p2] * b;
          o[2 * p2 + 1] = -gs[p2] * a + gc[p2] * b;
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
