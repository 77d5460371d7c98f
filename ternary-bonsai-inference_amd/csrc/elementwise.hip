// Activations and the gated-delta-net gate prep for gfx950.
//
//   bh_unary            kernels::map_inplace(silu|sigmoid|softplus)
//                       (src/kernels.rs:148-171) and the gated products of
//                       shaders/elem.comp modes 3/4 (src/forward.rs:574, 549-551, 379-382)
//   bh_gdn_gate_prep    beta = sigmoid, gate = softplus(alpha + dt_bias) * ssm_a
//                       (src/forward.rs:497-507)
//   bh_gdn_prep_fused   every small op of a recurrent layer for a batch of
//                       tokens, one launch (src/forward.rs:497-551)
//
// All of these are streaming, HBM-bound maps, written in the shape that
// streams best on this GPU: one 16-byte vector per lane, many short blocks.
// The fused gate prep covers a token with a few such blocks: its conv row
// (silu, then L2 per head of head_dim/4-lane groups reduced with shuffles in
// f64, as src/kernels.rs:134-140), its z/y gate row and its n_v_head scalar
// gates, so a recurrent layer's prep is one pass over its inputs.
#include <hip/hip_runtime.h>

#include <string>

#include "common.hpp"
#include "conv.hpp"

namespace bh {
namespace {

constexpr int kBlock = 256;
constexpr int kUnroll = 1;  // float4 per lane: one streams best here

template <int MODE>
__device__ __forceinline__ float unary_op(float a, float b) {
  if constexpr (MODE == BH_SILU) return silu(a);
  if constexpr (MODE == BH_SIGMOID) return sigmoid(a);
  if constexpr (MODE == BH_SOFTPLUS) return softplus(a);
  // src/forward.rs:549-551 `normed[i] *= silu(z[i])` and :574 silu(g) * u;
  // the product is commutative, so b * act(a) has the reference's bits.
  if constexpr (MODE == BH_SILU_MUL) return b * silu(a);
  if constexpr (MODE == BH_SIGMOID_MUL) return b * sigmoid(a);
  return a;
}

template <int MODE>
__device__ __forceinline__ float4 unary_op4(float4 a, float4 b) {
  return make_float4(unary_op<MODE>(a.x, b.x), unary_op<MODE>(a.y, b.y),
                     unary_op<MODE>(a.z, b.z), unary_op<MODE>(a.w, b.w));
}

template <int MODE>
__global__ __launch_bounds__(kBlock) void unary_vec_kernel(const float *a, const float *b,
                                                           float *out, size_t n) {
  constexpr bool BIN = MODE == BH_SILU_MUL || MODE == BH_SIGMOID_MUL;
  const size_t n4 = n >> 2;
  const size_t base = static_cast<size_t>(blockIdx.x) * (kBlock * kUnroll) + threadIdx.x;
  const float4 *a4 = reinterpret_cast<const float4 *>(a);
  const float4 *b4 = reinterpret_cast<const float4 *>(b);
  float4 *o4 = reinterpret_cast<float4 *>(out);
  float4 va[kUnroll], vb[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const size_t i = base + u * kBlock;
    va[u] = i < n4 ? load_stream(a4 + i) : make_float4(0, 0, 0, 0);
    if constexpr (BIN) vb[u] = i < n4 ? load_stream(b4 + i) : make_float4(0, 0, 0, 0);
    else vb[u] = va[u];
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const size_t i = base + u * kBlock;
    if (i < n4) store_stream(o4 + i, unary_op4<MODE>(va[u], vb[u]));
  }
  // scalar tail (n % 4 elements), done by the first lanes of block 0
  if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
    const size_t i = n4 * 4 + threadIdx.x;
    out[i] = unary_op<MODE>(a[i], BIN ? b[i] : 0.0f);
  }
}

template <int MODE>
__global__ __launch_bounds__(kBlock) void unary_scalar_kernel(const float *a, const float *b,
                                                              float *out, size_t n) {
  constexpr bool BIN = MODE == BH_SILU_MUL || MODE == BH_SIGMOID_MUL;
  const size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i < n) out[i] = unary_op<MODE>(a[i], BIN ? b[i] : 0.0f);
}

template <int MODE>
int unary_launch(const float *a, const float *b, float *out, size_t n, hipStream_t st) {
  constexpr bool BIN = MODE == BH_SILU_MUL || MODE == BH_SIGMOID_MUL;
  const bool vec = aligned16(a) && aligned16(out) && (!BIN || aligned16(b));
  if (vec) {
    const size_t per_block = static_cast<size_t>(kBlock) * kUnroll;
    size_t blocks = ((n >> 2) + per_block - 1) / per_block;
    if (blocks == 0) blocks = 1;  // tail only
    if (blocks > 0x7fffffffu) return fail(BH_ERR_SHAPE, "unary: n too large");
    BH_LAUNCH((unary_vec_kernel<MODE>), static_cast<unsigned>(blocks), kBlock, 0, st, a, b, out,
              n);
  } else {
    const size_t blocks = (n + kBlock - 1) / kBlock;
    if (blocks > 0x7fffffffu) return fail(BH_ERR_SHAPE, "unary: n too large");
    BH_LAUNCH((unary_scalar_kernel<MODE>), static_cast<unsigned>(blocks), kBlock, 0, st, a, b,
              out, n);
  }
  return ok();
}

// ---------------------------------------------------------------------------
// GDN gate prep
// ---------------------------------------------------------------------------

struct GdnParams {
  const float *conv;
  float *conv_out;
  const float *z;
  const float *y;
  float *gated_out;
  const float *alpha_raw;
  const float *dt_bias;
  const float *ssm_a;
  const float *beta_raw;
  float *gate_out;
  float *beta_out;
  int conv_dim, l2_dim, head_dim, inner_dim, n_v_head;
  int sigmoid_gate;  // 1: y * sigmoid(z), 0: y * silu(z)
  float eps;
  ConvIn cv;         // cv.k > 0: `conv` holds the raw qkv, convolved here first
  int conv_state_out;  // the conv-mode kernel advances cv.state itself
};

// src/forward.rs:501-507: beta = sigmoid(beta_raw); gate = softplus(alpha_raw
// + dt_bias) * ssm_a, one (token, head) per call.
__device__ __forceinline__ void small_gates(const GdnParams &a, size_t idx, int h) {
  if (a.beta_out != nullptr) a.beta_out[idx] = sigmoid(a.beta_raw[idx]);
  if (a.gate_out != nullptr) a.gate_out[idx] = softplus(a.alpha_raw[idx] + a.dt_bias[h]) * a.ssm_a[h];
}

__global__ __launch_bounds__(kBlock) void gdn_gate_prep_kernel(GdnParams a, size_t total) {
  const size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i < total) small_gates(a, i, static_cast<int>(i % a.n_v_head));
}

// The fused prep kernels' activations: the hardware exponential and
// reciprocal (silu_fast / sigmoid_fast, a few ulps from the reference's
// expf-based forms; these outputs carry the 1e-5 tolerance).  Measured on
// the standalone conv: 65.5 -> 62.5 us.
__device__ __forceinline__ float4 silu4(float4 v) {
  return make_float4(silu_fast(v.x), silu_fast(v.y), silu_fast(v.z), silu_fast(v.w));
}
// src/forward.rs:549-551 / :379-382: y * silu(z) or y * sigmoid(z)
__device__ __forceinline__ float4 gate4(float4 z, float4 y, bool sig) {
  return sig ? make_float4(y.x * sigmoid_fast(z.x), y.y * sigmoid_fast(z.y), y.z * sigmoid_fast(z.z),
                           y.w * sigmoid_fast(z.w))
             : make_float4(y.x * silu_fast(z.x), y.y * silu_fast(z.y), y.z * silu_fast(z.z),
                           y.w * silu_fast(z.w));
}

// kU = 2 float4 per lane (measured on [4096 tokens, 6144]: 92 us vs 100 us
// at one and 97 us at six per lane).  A token's work is split over bc conv blocks (256*kU
// float4 = 8*kU L2 heads of 128) and bg gate blocks (256*kU float4 of z/y);
// the first conv block of a token also computes its n_v_head scalar gates.
// G = head_dim / 4 lanes per L2 head (a divisor of 256, so heads never
// straddle a 256-float4 slice).
constexpr int kU = 2;
template <int G>
__global__ __launch_bounds__(kBlock) void gdn_prep_fused_kernel(GdnParams a, int bc, int bg) {
  const int per_tok = bc + bg;
  const size_t t = blockIdx.x / per_tok;
  const int part = blockIdx.x % per_tok;
  const int tid = threadIdx.x;

  if (part < bc) {
    const int n4 = a.conv_dim >> 2;
    const int l2_4 = a.l2_dim >> 2;
    const float4 *c4 = reinterpret_cast<const float4 *>(a.conv) + t * n4;
    float4 v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int i = (part * kU + u) * kBlock + tid;
      v[u] = i < n4 ? load_stream(c4 + i) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (part == 0)
      for (int h = tid; h < a.n_v_head; h += kBlock) small_gates(a, t * a.n_v_head + h, h);
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int i = (part * kU + u) * kBlock + tid;
      // conv output: silu, then L2 per head over the first l2_dim channels
      float4 s = silu4(v[u]);
      double ss = static_cast<double>(s.x) * static_cast<double>(s.x);
      ss += static_cast<double>(s.y) * static_cast<double>(s.y);
      ss += static_cast<double>(s.z) * static_cast<double>(s.z);
      ss += static_cast<double>(s.w) * static_cast<double>(s.w);
      ss = lane_group_reduce<G>(ss, SumOp{});
      if (i < l2_4) {
        const float scale = 1.0f / fmaxf(sqrtf(static_cast<float>(ss)), a.eps);
        s = make_float4(s.x * scale, s.y * scale, s.z * scale, s.w * scale);
      }
      if (i < n4) store_stream(reinterpret_cast<float4 *>(a.conv_out) + t * n4 + i, s);
    }
  } else {
    // output gate row: y * act(z)
    const int n4 = a.inner_dim >> 2;
    float4 z[kU], y[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int i = ((part - bc) * kU + u) * kBlock + tid;
      if (i < n4) {
        z[u] = load_stream(reinterpret_cast<const float4 *>(a.z) + t * n4 + i);
        y[u] = load_stream(reinterpret_cast<const float4 *>(a.y) + t * n4 + i);
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int i = ((part - bc) * kU + u) * kBlock + tid;
      if (i < n4) {
        store_stream(reinterpret_cast<float4 *>(a.gated_out) + t * n4 + i,
                     gate4(z[u], y[u], a.sigmoid_gate != 0));
      }
    }
  }
}

// Conv mode of the fused prep: a conv block runs kConvTok consecutive tokens
// over its channels, with the taps loaded once and the 4-row input window
// kept in registers (one new input row per token); per token it applies the
// SiLU, the head L2 norm and the store as gdn_prep_fused_kernel does.  The
// gated-output blocks stay one token each.  Grid: per group of kConvTok
// tokens, bc conv blocks then kConvTok * bg gated-output blocks.
constexpr int kConvTok = 4;

template <int G>
__global__ __launch_bounds__(kBlock) void gdn_prep_conv_kernel(GdnParams a, int bc, int bg,
                                                               size_t n_tok, int gpx) {
  const int per_grp = bc + kConvTok * bg;
  // XCD-aware order: workgroups are dealt to the 8 XCDs in turn, so XCD
  // b % 8 takes groups [x gpx, (x + 1) gpx) in token order, and a conv
  // block's three window rows (the previous group's last inputs, read by
  // the same part of that group just before) are still in that XCD's L2
  const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
  const size_t grp = static_cast<size_t>(xcd) * gpx + slot / per_grp;
  const int part = slot % per_grp;
  if (grp * kConvTok >= n_tok) return;
  const int tid = threadIdx.x;
  const size_t t0 = grp * kConvTok;
  const int nt = n_tok - t0 < static_cast<size_t>(kConvTok) ? static_cast<int>(n_tok - t0) : kConvTok;

  if (part < bc) {
    const int n4 = a.conv_dim >> 2;
    const int l2_4 = a.l2_dim >> 2;
    if (part == 0)
      for (int e = tid; e < nt * a.n_v_head; e += kBlock) {
        const int tt = e / a.n_v_head, h = e - tt * a.n_v_head;
        small_gates(a, (t0 + tt) * a.n_v_head + h, h);
      }
    float wv[kU][4][4];  // [u][channel q][tap j]
    float4 win[kU][4];   // [u][tap j]: inputs of the current token's window
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int i = (part * kU + u) * kBlock + tid;
      const int c = 4 * (i < n4 ? i : 0);
      const float4 *w4 = reinterpret_cast<const float4 *>(a.cv.w + static_cast<size_t>(c) * 4);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 f = w4[q];
        wv[u][q][0] = f.x;
        wv[u][q][1] = f.y;
        wv[u][q][2] = f.z;
        wv[u][q][3] = f.w;
      }
      if (t0 != 0) {  // groups start at 0 or at kConvTok >= 3: three input rows
#pragma unroll
        for (int j = 0; j < 3; ++j)
          win[u][j] = reinterpret_cast<const float4 *>(a.cv.x + (t0 - 3 + j) * a.conv_dim)[c / 4];
      } else {  // the first group: the cache (oldest first)
        const float *st = a.cv.state + static_cast<size_t>(c) * 3;
#pragma unroll
        for (int j = 0; j < 3; ++j) win[u][j] = make_float4(st[j], st[3 + j], st[6 + j], st[9 + j]);
      }
    }
    // every input row of the group, loaded before the first use
    float4 xin[kConvTok][kU];
#pragma unroll
    for (int tt = 0; tt < kConvTok; ++tt) {
      const size_t t = t0 + (tt < nt ? tt : nt - 1);
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int i = (part * kU + u) * kBlock + tid;
        const int c = 4 * (i < n4 ? i : 0);
        xin[tt][u] = load_stream(reinterpret_cast<const float4 *>(a.cv.x + t * a.conv_dim) + c / 4);
      }
    }
    if (t0 == 0 && a.conv_state_out) {
      // The first group's lanes, the only readers of the cache, write its new
      // contents for their channels after reading them: entry e = s_{n_tok-3+e},
      // an input row, or for fewer than 3 tokens an old entry held in win.
      // Selects per component on values (see conv.hip).
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int i = (part * kU + u) * kBlock + tid;
        if (i >= n4) continue;
        const float4 *x4 = reinterpret_cast<const float4 *>(a.cv.x) + i;
        const size_t row4 = static_cast<size_t>(a.conv_dim) / 4;
        auto entry = [&](int e) {
          const long p = static_cast<long>(n_tok) - 3 + e;
          const float4 xv = x4[static_cast<size_t>(p >= 0 ? p : 0) * row4];
          const float4 ov = sel4(p == -2, win[u][1], win[u][2]);
          return sel4(p >= 0, xv, ov);
        };
        const float4 n0 = entry(0), n1 = entry(1), n2 = entry(2);
        float *nst = const_cast<float *>(a.cv.state) + static_cast<size_t>(4 * i) * 3;
        nst[0] = n0.x; nst[1] = n1.x; nst[2] = n2.x;
        nst[3] = n0.y; nst[4] = n1.y; nst[5] = n2.y;
        nst[6] = n0.z; nst[7] = n1.z; nst[8] = n2.z;
        nst[9] = n0.w; nst[10] = n1.w; nst[11] = n2.w;
      }
    }
#pragma unroll
    for (int tt = 0; tt < kConvTok; ++tt) {
      if (tt >= nt) break;
      const size_t t = t0 + tt;
#pragma unroll
      for (int u = 0; u < kU; ++u) win[u][3] = xin[tt][u];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int i = (part * kU + u) * kBlock + tid;
        // src/forward.rs:518-522: acc = sum_j w[c][j] * win[j], j ascending
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc.x += wv[u][0][j] * win[u][j].x;
          acc.y += wv[u][1][j] * win[u][j].y;
          acc.z += wv[u][2][j] * win[u][j].z;
          acc.w += wv[u][3][j] * win[u][j].w;
        }
        float4 s = silu4(acc);
        double ss = static_cast<double>(s.x) * static_cast<double>(s.x);
        ss += static_cast<double>(s.y) * static_cast<double>(s.y);
        ss += static_cast<double>(s.z) * static_cast<double>(s.z);
        ss += static_cast<double>(s.w) * static_cast<double>(s.w);
        ss = lane_group_reduce<G>(ss, SumOp{});
        if (i < l2_4) {
          const float scale = 1.0f / fmaxf(sqrtf(static_cast<float>(ss)), a.eps);
          s = make_float4(s.x * scale, s.y * scale, s.z * scale, s.w * scale);
        }
        if (i < n4) store_stream(reinterpret_cast<float4 *>(a.conv_out) + t * n4 + i, s);
#pragma unroll
        for (int j = 0; j < 3; ++j) win[u][j] = win[u][j + 1];  // slide the window
      }
    }
  } else {
    const int gp = part - bc;
    const size_t t = t0 + gp / bg;
    if (t >= n_tok) return;
    const int n4 = a.inner_dim >> 2;
    const int gb = gp % bg;
    float4 z[kU], y[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int i = (gb * kU + u) * kBlock + tid;
      if (i < n4) {
        z[u] = load_stream(reinterpret_cast<const float4 *>(a.z) + t * n4 + i);
        y[u] = load_stream(reinterpret_cast<const float4 *>(a.y) + t * n4 + i);
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int i = (gb * kU + u) * kBlock + tid;
      if (i < n4)
        store_stream(reinterpret_cast<float4 *>(a.gated_out) + t * n4 + i,
                     gate4(z[u], y[u], a.sigmoid_gate != 0));
    }
  }
}

template <int G>
int launch_fused(const GdnParams &p, bool conv, size_t n_tok, int bc, int bg, hipStream_t st) {
  if (conv) {
    const size_t groups = (n_tok + kConvTok - 1) / kConvTok;
    const size_t gpx = (groups + 7) / 8;  // token groups per XCD
    const size_t blocks = 8 * gpx * static_cast<size_t>(bc + kConvTok * bg);
    if (blocks > 0x7fffffffu) return fail(BH_ERR_SHAPE, "gdn_prep_fused: too many blocks");
    BH_LAUNCH(gdn_prep_conv_kernel<G>, static_cast<unsigned>(blocks), kBlock, 0, st, p, bc, bg,
              n_tok, static_cast<int>(gpx));
  } else {
    const size_t blocks = n_tok * static_cast<size_t>(bc + bg);
    if (blocks > 0x7fffffffu) return fail(BH_ERR_SHAPE, "gdn_prep_fused: too many blocks");
    BH_LAUNCH(gdn_prep_fused_kernel<G>, static_cast<unsigned>(blocks), kBlock, 0, st, p, bc, bg);
  }
  return ok();
}

// Scalar gates only (no conv / gated rows requested).
__global__ __launch_bounds__(kBlock) void gdn_small_gates_kernel(GdnParams a, size_t total) {
  const size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i < total) small_gates(a, i, static_cast<int>(i % a.n_v_head));
}

// Looped version for layouts the fast kernel does not cover (odd widths,
// unaligned pointers): one block per token, one L2 head at a time.
__global__ __launch_bounds__(kBlock) void gdn_prep_loop_kernel(GdnParams a) {
  __shared__ double lds[kBlock / 64];
  const size_t t = blockIdx.x;
  const int tid = threadIdx.x;
  for (int h = tid; h < a.n_v_head; h += kBlock) small_gates(a, t * a.n_v_head + h, h);
  if (a.conv_out != nullptr) {
    const float *c = a.conv + t * a.conv_dim;
    float *o = a.conv_out + t * a.conv_dim;
    // channel value before the SiLU: the input, or its causal conv
    auto pre = [&](int ch) { return a.cv.k > 0 ? conv_at(a.cv, t, ch) : c[ch]; };
    const int n_heads = a.l2_dim / a.head_dim;
    for (int hh = 0; hh < n_heads; ++hh) {
      double ss = 0.0;
      for (int d = tid; d < a.head_dim; d += kBlock) {
        const float s = silu(pre(hh * a.head_dim + d));
        ss += static_cast<double>(s) * static_cast<double>(s);
      }
      ss = group_reduce<kBlock>(ss, SumOp{}, lds);
      const float scale = 1.0f / fmaxf(sqrtf(static_cast<float>(ss)), a.eps);
      for (int d = tid; d < a.head_dim; d += kBlock)
        o[hh * a.head_dim + d] = silu(pre(hh * a.head_dim + d)) * scale;
      __syncthreads();  // lds reuse by the next head
    }
    for (int i = a.l2_dim + tid; i < a.conv_dim; i += kBlock) o[i] = silu(pre(i));
  }
  if (a.gated_out != nullptr) {
    const size_t off = t * a.inner_dim;
    for (int i = tid; i < a.inner_dim; i += kBlock) {
      const float z = a.z[off + i], y = a.y[off + i];
      a.gated_out[off + i] = a.sigmoid_gate ? y * sigmoid(z) : y * silu(z);
    }
  }
}

}  // namespace
}  // namespace bh

using namespace bh;

extern "C" int bh_unary(int mode, const float *a, const float *b, size_t n, float *out,
                        bh_stream stream) {
  if (mode < BH_SILU || mode > BH_SIGMOID_MUL)
    return fail(BH_ERR_ARG, "unary: unknown mode " + std::to_string(mode));
  if (n == 0) return ok();
  if (!a || !out || ((mode == BH_SILU_MUL || mode == BH_SIGMOID_MUL) && !b))
    return fail(BH_ERR_ARG, "unary: null pointer");
  hipStream_t st = as_stream(stream);
  switch (mode) {
    case BH_SILU: return unary_launch<BH_SILU>(a, b, out, n, st);
    case BH_SIGMOID: return unary_launch<BH_SIGMOID>(a, b, out, n, st);
    case BH_SOFTPLUS: return unary_launch<BH_SOFTPLUS>(a, b, out, n, st);
    case BH_SILU_MUL: return unary_launch<BH_SILU_MUL>(a, b, out, n, st);
    default: return unary_launch<BH_SIGMOID_MUL>(a, b, out, n, st);
  }
}

extern "C" int bh_gdn_gate_prep(const float *alpha_raw, const float *dt_bias, const float *ssm_a,
                                const float *beta_raw, size_t n_tok, size_t n_head,
                                float *gate_out, float *beta_out, bh_stream stream) {
  const size_t total = n_tok * n_head;
  if (total == 0) return ok();
  if ((gate_out && (!alpha_raw || !dt_bias || !ssm_a)) || (beta_out && !beta_raw))
    return fail(BH_ERR_ARG, "gdn_gate_prep: null pointer");
  if (n_head > 0x7fffffffu) return fail(BH_ERR_SHAPE, "gdn_gate_prep: n_head too large");
  GdnParams p{};
  p.alpha_raw = alpha_raw;
  p.dt_bias = dt_bias;
  p.ssm_a = ssm_a;
  p.beta_raw = beta_raw;
  p.gate_out = gate_out;
  p.beta_out = beta_out;
  p.n_v_head = static_cast<int>(n_head);
  const size_t blocks = (total + kBlock - 1) / kBlock;
  if (blocks > 0x7fffffffu) return fail(BH_ERR_SHAPE, "gdn_gate_prep: too many elements");
  BH_LAUNCH(gdn_gate_prep_kernel, static_cast<unsigned>(blocks), kBlock, 0, as_stream(stream), p,
            total);
  return ok();
}

extern "C" int bh_gdn_prep_fused(const bh_gdn_prep_args *args, bh_stream stream) {
  if (args == nullptr) return fail(BH_ERR_ARG, "gdn_prep_fused: null args");
  const bh_gdn_prep_args &g = *args;
  if (g.gate_mode != BH_SILU_MUL && g.gate_mode != BH_SIGMOID_MUL)
    return fail(BH_ERR_ARG, "gdn_prep_fused: gate_mode must be BH_SILU_MUL or BH_SIGMOID_MUL");
  if (g.conv_out != nullptr) {
    if (g.head_dim == 0 || g.l2_dim % g.head_dim != 0 || g.l2_dim > g.conv_dim)
      return fail(BH_ERR_SHAPE, "gdn_prep_fused: l2_dim " + std::to_string(g.l2_dim) +
                                    " must be a multiple of head_dim " +
                                    std::to_string(g.head_dim) + " and <= conv_dim " +
                                    std::to_string(g.conv_dim));
    if (!g.conv) return fail(BH_ERR_ARG, "gdn_prep_fused: null conv");
  }
  const bool conv_in = g.conv_w != nullptr;
  if (conv_in) {
    if (g.conv_out == nullptr)
      return fail(BH_ERR_ARG, "gdn_prep_fused: conv_w needs conv_out (the convolved channels)");
    if (g.conv_k < 1 || g.conv_k > static_cast<size_t>(kMaxConvK))
      return fail(BH_ERR_SHAPE, "gdn_prep_fused: conv kernel size " + std::to_string(g.conv_k) +
                                    " must be in 1.." + std::to_string(kMaxConvK));
    const ConvIn cv{g.conv, g.conv_state, g.conv_w, static_cast<int>(g.conv_dim),
                    static_cast<int>(g.conv_k)};
    if (g.n_tok > 0)
      if (int e = conv_check(cv, g.conv_out, "gdn_prep_fused")) return e;
  }
  if (g.gated_out != nullptr && (!g.z || !g.y)) return fail(BH_ERR_ARG, "gdn_prep_fused: null z/y");
  if ((g.gate_out && (!g.alpha_raw || !g.dt_bias || !g.ssm_a)) || (g.beta_out && !g.beta_raw))
    return fail(BH_ERR_ARG, "gdn_prep_fused: null gate input");
  if (g.conv_dim > 0x7fffffffu || g.inner_dim > 0x7fffffffu || g.n_v_head > 0x7fffffffu)
    return fail(BH_ERR_SHAPE, "gdn_prep_fused: dimension exceeds 2^31-1");
  if (g.n_tok == 0) return ok();
  if (g.n_tok > 0x7fffffffu) return fail(BH_ERR_SHAPE, "gdn_prep_fused: n_tok too large");
  GdnParams p{};
  p.conv = g.conv;
  p.conv_out = g.conv_out;
  p.z = g.z;
  p.y = g.y;
  p.gated_out = g.gated_out;
  p.alpha_raw = g.alpha_raw;
  p.dt_bias = g.dt_bias;
  p.ssm_a = g.ssm_a;
  p.beta_raw = g.beta_raw;
  p.gate_out = g.gate_out;
  p.beta_out = g.beta_out;
  p.conv_dim = static_cast<int>(g.conv_dim);
  p.l2_dim = static_cast<int>(g.l2_dim);
  p.head_dim = static_cast<int>(g.head_dim);
  p.inner_dim = static_cast<int>(g.inner_dim);
  p.n_v_head = (g.gate_out || g.beta_out) ? static_cast<int>(g.n_v_head) : 0;
  p.sigmoid_gate = g.gate_mode == BH_SIGMOID_MUL ? 1 : 0;
  p.eps = g.eps;
  if (conv_in)
    p.cv = ConvIn{g.conv, g.conv_state, g.conv_w, static_cast<int>(g.conv_dim),
                  static_cast<int>(g.conv_k)};
  const unsigned grid = static_cast<unsigned>(g.n_tok);
  hipStream_t st = as_stream(stream);
  const size_t hq = g.head_dim / 4;
  const bool conv_fast = g.conv_out == nullptr ||
                         (g.conv_dim % 4 == 0 && g.head_dim % 4 == 0 && hq >= 1 && hq <= 64 &&
                          (hq & (hq - 1)) == 0 && aligned16(g.conv) && aligned16(g.conv_out) &&
                          (!conv_in || (g.conv_k == 4 && aligned16(g.conv_w))));
  const bool gate_fast = g.gated_out == nullptr ||
                         (g.inner_dim % 4 == 0 && aligned16(g.z) && aligned16(g.y) &&
                          aligned16(g.gated_out));
  if (conv_fast && gate_fast) {
    if (g.conv_out == nullptr && g.gated_out == nullptr) {
      const size_t total = g.n_tok * static_cast<size_t>(p.n_v_head);
      if (total == 0) return ok();
      const size_t blocks = (total + kBlock - 1) / kBlock;
      if (blocks > 0x7fffffffu) return fail(BH_ERR_SHAPE, "gdn_prep_fused: too many gates");
      BH_LAUNCH(gdn_small_gates_kernel, static_cast<unsigned>(blocks), kBlock, 0, st, p, total);
      return ok();
    }
    // conv blocks (at least one per token: it also carries the scalar gates)
    const int per_block = kBlock * kU;  // float4 per block
    const int bc = g.conv_out ? static_cast<int>((g.conv_dim / 4 + per_block - 1) / per_block) : 1;
    const int bg = g.gated_out ? static_cast<int>((g.inner_dim / 4 + per_block - 1) / per_block) : 0;
    if (g.conv_out == nullptr) {
      // conv part disabled: its block only computes the scalar gates
      p.conv_dim = 0;
      p.l2_dim = 0;
    }
    // with conv outputs the conv-mode kernel's first token group advances
    // the cache itself (no second launch)
    p.conv_state_out = conv_in && g.conv_out != nullptr ? 1 : 0;
    int e = -999;
    switch (g.conv_out == nullptr ? 64 : hq) {
      case 1: e = launch_fused<1>(p, conv_in, g.n_tok, bc, bg, st); break;
      case 2: e = launch_fused<2>(p, conv_in, g.n_tok, bc, bg, st); break;
      case 4: e = launch_fused<4>(p, conv_in, g.n_tok, bc, bg, st); break;
      case 8: e = launch_fused<8>(p, conv_in, g.n_tok, bc, bg, st); break;
      case 16: e = launch_fused<16>(p, conv_in, g.n_tok, bc, bg, st); break;
      case 32: e = launch_fused<32>(p, conv_in, g.n_tok, bc, bg, st); break;
      case 64: e = launch_fused<64>(p, conv_in, g.n_tok, bc, bg, st); break;
      default: break;
    }
    if (e != -999) {
      if (e != BH_OK) return e;
      // otherwise the conv cache shifts after every token has read it
      return conv_in && !p.conv_state_out ? conv_state_update(p.cv, g.n_tok, st) : ok();
    }
  }
  BH_LAUNCH(gdn_prep_loop_kernel, grid, kBlock, 0, st, p);
  return conv_in ? conv_state_update(p.cv, g.n_tok, st) : ok();
}
