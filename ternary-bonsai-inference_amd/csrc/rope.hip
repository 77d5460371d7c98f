// Attention pre-block for gfx950: per-head q/k RMSNorm fused with IMROPE.
//
//   bh_qk_norm_rope   src/forward.rs:237-270 (split [q|gate], rms_norm_rows on
//                     q and k heads, rope_imrope per head) + the sigmoid of
//                     the gate half (src/forward.rs:379)
//   bh_rope_imrope    rope::rope_imrope (src/rope.rs:9-70) over a batch of heads
//
// Design.  A head row is held by G = head_dim/8 lanes, two float4 each (the
// first half-row slice and the second), so the RMSNorm sum is a G-lane
// shuffle reduction and the rotation partner of dim j (j + n_dims/2, always
// in the first slice) sits in lane gl + n_dims/8 of the same group: one
// cross-lane read per component (a DPP row rotation for n_dims 64), no LDS
// traffic for the data.  A block of 256 lanes holds 16 head rows of one
// token (2 per lane group, all loads issued together); the token's cos/sin
// table (n_dims/2 pairs) is built into LDS by the first n_dims/2 lanes while
// the rows' loads are in flight, and shared by all 16 rows.
//
// Angles.  The reference computes theta for pair j by multiplying the
// position by theta_scale once per pair (src/rope.rs:54-57), so theta_j is a
// chain of j rounded f32 products.  Lane j repeats that exact chain (there is
// no closed form with the same bits), with theta_scale = powf(base, -2/n_dims)
// computed on the host by the C library as the reference does (src/rope.rs:23).
// cosf/sinf are the full-range-reduction device versions.
#include <hip/hip_runtime.h>

#include <cmath>
#include <string>

#include "common.hpp"

namespace bh {
namespace {

constexpr int kBlock = 256;
constexpr int kMaxHalf = 128;  // n_dims/2 for head_dim <= 256

struct RopeParams {
  const float *q;
  float *q_out;
  float *gate_out;
  const float *k;
  float *k_out;
  const float *wq;
  const float *wk;
  const int32_t *pos;
  int n_q, n_k, head_dim, q_stride, n_dims;
  int s0, s1, s2, sect;
  float theta_scale;
  float eps;
};

// theta of pair j at the given positions, band selection of src/rope.rs:37-49.
__device__ __forceinline__ float imrope_theta(int j, const int32_t *p, const RopeParams &a) {
  const int sector = j % a.sect;
  int band;
  if (sector % 3 == 1 && sector < 3 * a.s1)
    band = 1;
  else if (sector % 3 == 2 && sector < 3 * a.s2)
    band = 2;
  else if (sector % 3 == 0 && sector < 3 * a.s0)
    band = 0;
  else
    band = 3;
  float th = static_cast<float>(p[band]);
  for (int i = 0; i < j; ++i) th *= a.theta_scale;
  return th;
}

// rotated value of one component: role 0 holds x0 = head[j], role 1 holds
// x1 = head[j + half] (src/rope.rs:61-69).
__device__ __forceinline__ float rot(float own, float other, float c, float s, bool role1) {
  return role1 ? (other * s + own * c) : (own * c - other * s);
}


// Fills the cos/sin table of `half` pairs for the token at `p` into LDS.
__device__ __forceinline__ void fill_table(const RopeParams &a, const int32_t *p, int half,
                                           float *cs_cos, float *cs_sin) {
  if (threadIdx.x < half) {
    const float th = imrope_theta(threadIdx.x, p, a);
    float sn, cn;
    sincosf(th, &sn, &cn);
    cs_cos[threadIdx.x] = cn;
    cs_sin[threadIdx.x] = sn;
  }
}

// A block holds rows of ONE token: blockDim.x/G row slots, R rows per slot
// (the loads of all R rows go out first), V float4 per lane per row (lane gl
// holds float4 gl, gl+G, ...: G*V*4 = head_dim).  A token's rows (q heads,
// then k heads) are spread over blocks_per_tok consecutive blocks.  The
// token's cos/sin table is built in LDS by the first n_dims/2 lanes while the
// loads are in flight.  Rotated dims all live in the first float4 slice
// (n_dims <= 4G).  DPP8: the rotation partner is 8 lanes away (n_dims 64), a
// DPP row rotation inside each 16-lane row instead of an LDS-crossbar permute.
template <int G, int V, bool NORM, int R, bool DPP8>
__global__ __launch_bounds__(kBlock) void qk_norm_rope_kernel(RopeParams a, int blocks_per_tok) {
  const int slots = blockDim.x / G;
  __shared__ float cs_cos[kMaxHalf];
  __shared__ float cs_sin[kMaxHalf];

  const size_t t = blockIdx.x / blocks_per_tok;
  const int row0 = (blockIdx.x % blocks_per_tok) * slots * R + threadIdx.x / G;
  const int gl = threadIdx.x % G;
  const int lane = threadIdx.x & 63;
  const int n_rows = a.n_q + a.n_k;
  const int half = a.n_dims >> 1;

  float4 x[R][V], g[R][V];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int r = row0 + k * slots;
#pragma unroll
    for (int v = 0; v < V; ++v) {
      x[k][v] = make_float4(0.f, 0.f, 0.f, 0.f);
      g[k][v] = x[k][v];
    }
    if (r < a.n_q) {
      const float4 *src = reinterpret_cast<const float4 *>(a.q + (t * a.n_q + r) * a.q_stride);
#pragma unroll
      for (int v = 0; v < V; ++v) x[k][v] = load_stream(src + gl + v * G);
      if (a.gate_out != nullptr) {
        const float4 *gs = reinterpret_cast<const float4 *>(a.q + (t * a.n_q + r) * a.q_stride + a.head_dim);
#pragma unroll
        for (int v = 0; v < V; ++v) g[k][v] = load_stream(gs + gl + v * G);
      }
    } else if (r < n_rows) {
      const float4 *src = reinterpret_cast<const float4 *>(a.k + (t * a.n_k + (r - a.n_q)) * a.head_dim);
#pragma unroll
      for (int v = 0; v < V; ++v) x[k][v] = load_stream(src + gl + v * G);
    }
  }
  float4 wq[V], wk[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    wq[v] = make_float4(1.f, 1.f, 1.f, 1.f);
    wk[v] = wq[v];
    if (NORM) {
      if (a.n_q > 0) wq[v] = reinterpret_cast<const float4 *>(a.wq)[gl + v * G];
      if (a.n_k > 0) wk[v] = reinterpret_cast<const float4 *>(a.wk)[gl + v * G];
    }
  }

  fill_table(a, a.pos + 4 * t, half, cs_cos, cs_sin);

  // rotation partner (first slice): dim j <-> j + n_dims/2, lane gl <-> gl +- n_dims/8
  const int d0 = 4 * gl;
  const bool rotates = d0 < a.n_dims;
  const bool role1 = d0 >= half;
  const int partner = rotates ? (role1 ? gl - half / 4 : gl + half / 4) : gl;
  const int src_lane = lane - gl + partner;
  const int j0 = role1 ? d0 - half : d0;

  __syncthreads();  // table ready
  float4 cv = make_float4(1.f, 1.f, 1.f, 1.f), sv = make_float4(0.f, 0.f, 0.f, 0.f);
  if (rotates) {
    cv = make_float4(cs_cos[j0], cs_cos[j0 + 1], cs_cos[j0 + 2], cs_cos[j0 + 3]);
    sv = make_float4(cs_sin[j0], cs_sin[j0 + 1], cs_sin[j0 + 2], cs_sin[j0 + 3]);
  }

#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int r = row0 + k * slots;
    const bool is_q = r < a.n_q;
    float4 vv[V];
#pragma unroll
    for (int v = 0; v < V; ++v) vv[v] = x[k][v];
    if constexpr (NORM) {
      // src/kernels.rs:112-120: (x * scale) * w, scale = 1/sqrt(sum(x^2)/n + eps)
      float ss = 0.0f;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        ss += vv[v].x * vv[v].x;
        ss += vv[v].y * vv[v].y;
        ss += vv[v].z * vv[v].z;
        ss += vv[v].w * vv[v].w;
      }
#pragma unroll
      for (int off = G / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
      const float scale = 1.0f / sqrtf(ss / static_cast<float>(a.head_dim) + a.eps);
#pragma unroll
      for (int v = 0; v < V; ++v) {
        const float4 w = is_q ? wq[v] : wk[v];
        vv[v].x = (vv[v].x * scale) * w.x;
        vv[v].y = (vv[v].y * scale) * w.y;
        vv[v].z = (vv[v].z * scale) * w.z;
        vv[v].w = (vv[v].w * scale) * w.w;
      }
    }
    float px, py, pz, pw;
    const float4 &u = vv[0];
    if constexpr (DPP8) {
      // lane i <- lane i^8 inside each 16-lane row: DPP row_ror:8 (0x128)
      px = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(u.x), 0x128, 0xf, 0xf, false));
      py = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(u.y), 0x128, 0xf, 0xf, false));
      pz = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(u.z), 0x128, 0xf, 0xf, false));
      pw = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(u.w), 0x128, 0xf, 0xf, false));
    } else {
      px = __shfl(u.x, src_lane, 64);
      py = __shfl(u.y, src_lane, 64);
      pz = __shfl(u.z, src_lane, 64);
      pw = __shfl(u.w, src_lane, 64);
    }
    if (rotates) {
      vv[0].x = rot(u.x, px, cv.x, sv.x, role1);
      vv[0].y = rot(u.y, py, cv.y, sv.y, role1);
      vv[0].z = rot(u.z, pz, cv.z, sv.z, role1);
      vv[0].w = rot(u.w, pw, cv.w, sv.w, role1);
    }
    if (is_q) {
      float4 *dst = reinterpret_cast<float4 *>(a.q_out + (t * a.n_q + r) * a.head_dim);
#pragma unroll
      for (int v = 0; v < V; ++v) store_stream(dst + gl + v * G, vv[v]);
      if (a.gate_out != nullptr) {
        float4 *gd = reinterpret_cast<float4 *>(a.gate_out + (t * a.n_q + r) * a.head_dim);
#pragma unroll
        for (int v = 0; v < V; ++v)
          gd[gl + v * G] = make_float4(sigmoid(g[k][v].x), sigmoid(g[k][v].y),
                                       sigmoid(g[k][v].z), sigmoid(g[k][v].w));
      }
    } else if (r < n_rows) {
      float4 *dst = reinterpret_cast<float4 *>(a.k_out + (t * a.n_k + (r - a.n_q)) * a.head_dim);
#pragma unroll
      for (int v = 0; v < V; ++v) store_stream(dst + gl + v * G, vv[v]);
    }
  }
}

// Looped fallback for shapes outside the lane mapping above (odd head_dim,
// n_dims not a multiple of 8, unaligned pointers): one block per head row.
template <bool NORM>
__global__ __launch_bounds__(64) void qk_norm_rope_loop_kernel(RopeParams a) {
  extern __shared__ float rowbuf[];
  __shared__ float lds[1];
  const int n_rows = a.n_q + a.n_k;
  const size_t t = blockIdx.x / n_rows;
  const int r = blockIdx.x % n_rows;
  const bool is_q = r < a.n_q;
  const float *src = is_q ? a.q + (t * a.n_q + r) * a.q_stride
                          : a.k + (t * a.n_k + (r - a.n_q)) * a.head_dim;
  float *dst = is_q ? a.q_out + (t * a.n_q + r) * a.head_dim
                    : a.k_out + (t * a.n_k + (r - a.n_q)) * a.head_dim;
  const float *w = is_q ? a.wq : a.wk;
  float scale = 1.0f;
  if constexpr (NORM) {
    float ss = 0.0f;
    for (int d = threadIdx.x; d < a.head_dim; d += 64) ss += src[d] * src[d];
    ss = group_reduce<64>(ss, SumOp{}, lds);
    scale = 1.0f / sqrtf(ss / static_cast<float>(a.head_dim) + a.eps);
  }
  for (int d = threadIdx.x; d < a.head_dim; d += 64)
    rowbuf[d] = NORM ? (src[d] * scale) * w[d] : src[d];
  __syncthreads();
  const int half = a.n_dims >> 1;
  for (int d = threadIdx.x; d < a.head_dim; d += 64) {
    float o = rowbuf[d];
    if (d < a.n_dims) {
      const int j = d < half ? d : d - half;
      float s, c;
      sincosf(imrope_theta(j, a.pos + 4 * t, a), &s, &c);
      const float x0 = rowbuf[j], x1 = rowbuf[j + half];
      o = d < half ? (x0 * c - x1 * s) : (x0 * s + x1 * c);
    }
    dst[d] = o;
  }
  if (is_q && a.gate_out != nullptr) {
    for (int d = threadIdx.x; d < a.head_dim; d += 64)
      a.gate_out[(t * a.n_q + r) * a.head_dim + d] = sigmoid(src[a.head_dim + d]);
  }
}

// Launches the register kernel with V float4 per lane and R rows per lane
// group; returns -999 when the shape does not fit that geometry.
template <int V, int R, bool NORM>
int launch_rope_v(const RopeParams &p, size_t n_tok, hipStream_t st) {
  if (p.head_dim % (4 * V) != 0) return -999;
  const int G = p.head_dim / 4 / V;
  if (G < 8 || G > 64 || (G & (G - 1)) != 0 || p.n_dims > 4 * G) return -999;
  const int n_rows = p.n_q + p.n_k;
  const int rows_per_block = (kBlock / G) * R;
  const int bpt = (n_rows + rows_per_block - 1) / rows_per_block;  // blocks per token
  const size_t blocks = n_tok * static_cast<size_t>(bpt);
  if (blocks > 0x7fffffffu) return fail(BH_ERR_SHAPE, "rope: too many head rows");
  const unsigned grid = static_cast<unsigned>(blocks);
  if (p.n_dims == 64 && G >= 16) {  // partner 8 lanes away: DPP
    switch (G) {
      case 16: BH_LAUNCH((qk_norm_rope_kernel<16, V, NORM, R, true>), grid, kBlock, 0, st, p, bpt); return ok();
      case 32: BH_LAUNCH((qk_norm_rope_kernel<32, V, NORM, R, true>), grid, kBlock, 0, st, p, bpt); return ok();
      case 64: BH_LAUNCH((qk_norm_rope_kernel<64, V, NORM, R, true>), grid, kBlock, 0, st, p, bpt); return ok();
      default: return -999;
    }
  }
  switch (G) {
    case 8: BH_LAUNCH((qk_norm_rope_kernel<8, V, NORM, R, false>), grid, kBlock, 0, st, p, bpt); return ok();
    case 16: BH_LAUNCH((qk_norm_rope_kernel<16, V, NORM, R, false>), grid, kBlock, 0, st, p, bpt); return ok();
    case 32: BH_LAUNCH((qk_norm_rope_kernel<32, V, NORM, R, false>), grid, kBlock, 0, st, p, bpt); return ok();
    case 64: BH_LAUNCH((qk_norm_rope_kernel<64, V, NORM, R, false>), grid, kBlock, 0, st, p, bpt); return ok();
    default: return -999;
  }
}

template <bool NORM>
int launch_rope(const RopeParams &p, size_t n_tok, hipStream_t st) {
  const bool fast = (p.head_dim % 4 == 0) && (p.n_dims % 8 == 0) && (p.q_stride % 4 == 0) &&
                    p.head_dim <= 512 && p.head_dim >= 32 && aligned16(p.q) &&
                    aligned16(p.q_out) && (p.gate_out == nullptr || aligned16(p.gate_out)) &&
                    (p.n_k == 0 || (aligned16(p.k) && aligned16(p.k_out))) &&
                    (!NORM || (aligned16(p.wq) && (p.n_k == 0 || aligned16(p.wk))));
  if (fast) {
    // 2 float4 per lane, 2 rows per lane group (measured on config 2: 25.2 us
    // vs 26.5-28.6 us at one float4 and 4 rows); shapes whose rotated dims
    // do not fit the first half-row slice take one float4 per lane
    if (int e = launch_rope_v<2, 2, NORM>(p, n_tok, st); e != -999) return e;
    if (int e = launch_rope_v<1, 4, NORM>(p, n_tok, st); e != -999) return e;
  }
  const size_t blocks = n_tok * static_cast<size_t>(p.n_q + p.n_k);
  if (blocks > 0x7fffffffu) return fail(BH_ERR_SHAPE, "rope: too many head rows");
  const size_t shmem = static_cast<size_t>(p.head_dim) * sizeof(float);
  if (shmem > 65536) return fail(BH_ERR_SHAPE, "rope: head_dim too large");
  BH_LAUNCH((qk_norm_rope_loop_kernel<NORM>), static_cast<unsigned>(blocks), 64, shmem, st, p);
  return ok();
}

int check_rope_common(size_t head_dim, size_t n_dims, const int32_t *sections, RopeParams &p,
                      float freq_base) {
  if (sections == nullptr) return fail(BH_ERR_ARG, "rope_imrope: null sections");
  if (n_dims % 2 != 0 || n_dims > head_dim)
    return fail(BH_ERR_SHAPE, "rope_imrope: n_dims " + std::to_string(n_dims) +
                                  " must be even and <= head len " + std::to_string(head_dim));
  if (head_dim > 16384) return fail(BH_ERR_SHAPE, "rope_imrope: head_dim too large");
  const long sect = static_cast<long>(sections[0]) + sections[1] + sections[2] + sections[3];
  if (sect <= 0 || sections[0] < 0 || sections[1] < 0 || sections[2] < 0 || sections[3] < 0)
    return fail(BH_ERR_ARG, "rope_imrope: sections must be >= 0 with a positive sum");
  p.s0 = sections[0];
  p.s1 = sections[1];
  p.s2 = sections[2];
  p.sect = static_cast<int>(sect);
  p.head_dim = static_cast<int>(head_dim);
  p.n_dims = static_cast<int>(n_dims);
  // src/rope.rs:23 -- the C library's powf, as Rust's f32::powf calls it
  p.theta_scale = powf(freq_base, -2.0f / static_cast<float>(n_dims));
  return BH_OK;
}

}  // namespace
}  // namespace bh

using namespace bh;

extern "C" int bh_qk_norm_rope(const bh_qk_norm_rope_args *args, bh_stream stream) {
  if (args == nullptr) return fail(BH_ERR_ARG, "qk_norm_rope: null args");
  const bh_qk_norm_rope_args &g = *args;
  RopeParams p{};
  if (int e = check_rope_common(g.head_dim, g.n_dims, g.sections, p, g.freq_base)) return e;
  if (g.q_head_stride < g.head_dim)
    return fail(BH_ERR_SHAPE, "qk_norm_rope: q_head_stride < head_dim");
  if (g.gate_out != nullptr && g.q_head_stride != 2 * g.head_dim)
    return fail(BH_ERR_SHAPE, "qk_norm_rope: gate_out needs q_head_stride == 2*head_dim");
  if (g.n_q_head + g.n_k_head > 4096) return fail(BH_ERR_SHAPE, "qk_norm_rope: too many heads");
  if (g.n_tok == 0 || g.n_q_head + g.n_k_head == 0 || g.head_dim == 0) return ok();
  if (!g.pos || (g.n_q_head && (!g.q || !g.q_out || !g.wq)) ||
      (g.n_k_head && (!g.k || !g.k_out || !g.wk)))
    return fail(BH_ERR_ARG, "qk_norm_rope: null pointer");
  p.q = g.q;
  p.q_out = g.q_out;
  p.gate_out = g.gate_out;
  p.k = g.k;
  p.k_out = g.k_out;
  p.wq = g.wq;
  p.wk = g.wk;
  p.pos = g.pos;
  p.n_q = static_cast<int>(g.n_q_head);
  p.n_k = static_cast<int>(g.n_k_head);
  p.q_stride = static_cast<int>(g.q_head_stride);
  p.eps = g.eps;
  return launch_rope<true>(p, g.n_tok, as_stream(stream));
}

extern "C" int bh_rope_imrope(float *heads, size_t n_tok, size_t n_head, size_t head_dim,
                              const int32_t *pos, size_t n_dims, const int32_t sections[4],
                              float freq_base, bh_stream stream) {
  RopeParams p{};
  if (int e = check_rope_common(head_dim, n_dims, sections, p, freq_base)) return e;
  if (n_head > 4096) return fail(BH_ERR_SHAPE, "rope_imrope: too many heads");
  if (n_tok == 0 || n_head == 0 || head_dim == 0) return ok();
  if (!heads || !pos) return fail(BH_ERR_ARG, "rope_imrope: null pointer");
  p.q = heads;
  p.q_out = heads;
  p.n_q = static_cast<int>(n_head);
  p.n_k = 0;
  p.q_stride = static_cast<int>(head_dim);
  p.pos = pos;
  return launch_rope<false>(p, n_tok, as_stream(stream));
}
