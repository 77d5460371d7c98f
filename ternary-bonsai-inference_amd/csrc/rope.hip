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

constexpr int kMaxHalf = 128;  // n_dims/2 for head_dim <= 256
constexpr int kMaxBlock = 512;  // lanes of the register kernel's largest block

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
  float inv_hd;  // 1 / head_dim
};

// theta of pair j at the given positions, band selection of src/rope.rs:37-49,
// then the reference's chain of j rounded f32 products (src/rope.rs:54-57).
__device__ __forceinline__ float imrope_theta(int j, int32_t p_t, int32_t p_h, int32_t p_w,
                                              int32_t p_e, const RopeParams &a) {
  const int sector = j % a.sect;
  int32_t p;
  if (sector % 3 == 1 && sector < 3 * a.s1)
    p = p_h;
  else if (sector % 3 == 2 && sector < 3 * a.s2)
    p = p_w;
  else if (sector % 3 == 0 && sector < 3 * a.s0)
    p = p_t;
  else
    p = p_e;
  float th = static_cast<float>(p);
  for (int i = 0; i < j; ++i) th *= a.theta_scale;
  return th;
}
__device__ __forceinline__ float imrope_theta(int j, const int32_t *p, const RopeParams &a) {
  return imrope_theta(j, p[0], p[1], p[2], p[3], a);
}

// rotated value of one component: role 0 holds x0 = head[j], role 1 holds
// x1 = head[j + half] (src/rope.rs:61-69).
__device__ __forceinline__ float rot(float own, float other, float c, float s, bool role1) {
  return role1 ? (other * s + own * c) : (own * c - other * s);
}


// A block holds rows of ONE token: blockDim.x/G row slots (at most 8 waves),
// R rows per slot, V float4 per lane per row (lane gl holds float4 gl, gl+G,
// ...: G*V*4 = head_dim).  A token's rows (q heads, then k heads) are spread
// evenly over blocks_per_tok consecutive blocks.  Order of work, chosen so that nothing
// waits on the row data except the arithmetic that needs it:
//   1. every row load is issued, branch-free (rows past the token's last
//      head re-read a valid row and are not stored);
//   2. the token's positions come in through the scalar cache (a separate
//      counter from the vector loads, so the angle chain starts while the
//      rows are in flight);
//   3. the first n_dims/2 lanes build the token's cos/sin table in LDS;
//   4. per row: sum of squares reduced with DPP/permlane swaps, scale,
//      weight, rotation (the partner of dim j < n_dims/2 is 8 lanes away for
//      n_dims 64: a DPP row rotation), non-temporal store.
// Rotated dims all live in the first float4 slice (n_dims <= 4G).
template <int G, int V, int R, bool NORM, bool GATE, bool DPP8>
__global__ __launch_bounds__(kMaxBlock) void qk_norm_rope_kernel(RopeParams a, int blocks_per_tok) {
  const int kSlots = blockDim.x / G;
  __shared__ float cs_cos[kMaxHalf];
  __shared__ float cs_sin[kMaxHalf];

  const size_t t = blockIdx.x / blocks_per_tok;
  const int row0 = (blockIdx.x % blocks_per_tok) * kSlots * R + threadIdx.x / G;
  const int gl = threadIdx.x % G;
  const int lane = threadIdx.x & 63;
  const int n_rows = a.n_q + a.n_k;
  const int half = a.n_dims >> 1;

  // 1. row loads
  float4 x[R][V];
  float4 g[GATE ? R : 1][V];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int r0 = row0 + k * kSlots;
    const int r = r0 < n_rows ? r0 : n_rows - 1;
    const float *row = r < a.n_q ? a.q + (t * a.n_q + r) * a.q_stride
                                 : a.k + (t * a.n_k + (r - a.n_q)) * a.head_dim;
    const float4 *src = reinterpret_cast<const float4 *>(row);
#pragma unroll
    for (int v = 0; v < V; ++v) x[k][v] = load_stream(src + gl + v * G);
    if constexpr (GATE) {
      // the gate half of a q head row (k rows re-read their own row, unused)
      const float4 *gs = reinterpret_cast<const float4 *>(r < a.n_q ? row + a.head_dim : row);
#pragma unroll
      for (int v = 0; v < V; ++v) g[k][v] = load_stream(gs + gl + v * G);
    }
  }
  float4 wq[V], wk[V];
#pragma unroll
  for (int v = 0; v < V; ++v) {
    wq[v] = make_float4(1.f, 1.f, 1.f, 1.f);
    wk[v] = wq[v];
    if constexpr (NORM) {
      if (a.n_q > 0) wq[v] = reinterpret_cast<const float4 *>(a.wq)[gl + v * G];
      if (a.n_k > 0) wk[v] = reinterpret_cast<const float4 *>(a.wk)[gl + v * G];
    }
  }

  // 2. the token's positions (p_t, p_h, p_w, p_e): a uniform address, so a
  // scalar load, whose wait does not wait for the row loads above
  const int4 pos = *reinterpret_cast<const int4 *>(a.pos + 4 * t);

  // 3. the token's cos/sin table
  for (int j = threadIdx.x; j < half; j += blockDim.x) {  // one pass unless the block is small
    float sn, cn;
    sincosf(imrope_theta(j, pos.x, pos.y, pos.z, pos.w, a), &sn, &cn);
    cs_cos[j] = cn;
    cs_sin[j] = sn;
  }

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

  // 4. per row
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int r = row0 + k * kSlots;
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
      ss = lane_group_sum<G>(ss);
      const float scale = rms_scale(ss, a.inv_hd, a.eps);
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
      px = dpp_move<0x128>(u.x);
      py = dpp_move<0x128>(u.y);
      pz = dpp_move<0x128>(u.z);
      pw = dpp_move<0x128>(u.w);
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
      if constexpr (GATE) {
        float4 *gd = reinterpret_cast<float4 *>(a.gate_out + (t * a.n_q + r) * a.head_dim);
#pragma unroll
        for (int v = 0; v < V; ++v)
          store_stream(gd + gl + v * G, make_float4(sigmoid(g[k][v].x), sigmoid(g[k][v].y),
                                                    sigmoid(g[k][v].z), sigmoid(g[k][v].w)));
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
    scale = rms_scale(ss, a.inv_hd, a.eps);
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

// Launches the register kernel for lane-group size G; the gate and the DPP
// rotation partner are compile-time variants.
template <int G, int V, int R, bool NORM>
int launch_rope_g(const RopeParams &p, unsigned grid, unsigned block, int bpt, hipStream_t st) {
  const bool dpp8 = p.n_dims == 64 && G >= 16;  // partner 8 lanes away: DPP
  if constexpr (NORM) {
    if (p.gate_out != nullptr) {
      if (dpp8) BH_LAUNCH((qk_norm_rope_kernel<G, V, R, NORM, true, true>), grid, block, 0, st, p, bpt);
      else BH_LAUNCH((qk_norm_rope_kernel<G, V, R, NORM, true, false>), grid, block, 0, st, p, bpt);
      return ok();
    }
  }
  if (dpp8) BH_LAUNCH((qk_norm_rope_kernel<G, V, R, NORM, false, true>), grid, block, 0, st, p, bpt);
  else BH_LAUNCH((qk_norm_rope_kernel<G, V, R, NORM, false, false>), grid, block, 0, st, p, bpt);
  return ok();
}

// Launches the register kernel with V float4 per lane and R rows per lane
// group; returns -999 when the shape does not fit.  Block size: a token's
// rows need ceil(rows / rows-per-wave) waves; they are split evenly over the
// fewest blocks of at most 8 waves (config 2's 28 heads of 256: 14 waves,
// two blocks of 7 -- measured 20.7 us against 22.3 us for 16-row blocks of
// 4 waves, which leave 4 of 32 row slots idle per token).
template <int V, int R, bool NORM>
int launch_rope_v(const RopeParams &p, size_t n_tok, hipStream_t st) {
  if (p.head_dim % (4 * V) != 0) return -999;
  const int G = p.head_dim / 4 / V;
  if (G < 8 || G > 64 || (G & (G - 1)) != 0 || p.n_dims > 4 * G) return -999;
  const int n_rows = p.n_q + p.n_k;
  const int rows_per_wave = (64 / G) * R;
  const int waves = (n_rows + rows_per_wave - 1) / rows_per_wave;  // per token
  const int max_waves = kMaxBlock / 64;
  const int bpt = (waves + max_waves - 1) / max_waves;               // blocks per token
  const unsigned block = 64u * static_cast<unsigned>((waves + bpt - 1) / bpt);
  const size_t blocks = n_tok * static_cast<size_t>(bpt);
  if (blocks > 0x7fffffffu) return fail(BH_ERR_SHAPE, "rope: too many head rows");
  const unsigned grid = static_cast<unsigned>(blocks);
  switch (G) {
    case 8: return launch_rope_g<8, V, R, NORM>(p, grid, block, bpt, st);
    case 16: return launch_rope_g<16, V, R, NORM>(p, grid, block, bpt, st);
    case 32: return launch_rope_g<32, V, R, NORM>(p, grid, block, bpt, st);
    case 64: return launch_rope_g<64, V, R, NORM>(p, grid, block, bpt, st);
    default: return -999;
  }
}

template <bool NORM>
int launch_rope(const RopeParams &p, size_t n_tok, hipStream_t st) {
  const bool fast = (p.head_dim % 4 == 0) && (p.n_dims % 8 == 0) && (p.q_stride % 4 == 0) &&
                    p.head_dim <= 512 && p.head_dim >= 32 && aligned16(p.q) &&
                    aligned16(p.q_out) && (p.gate_out == nullptr || aligned16(p.gate_out)) &&
                    (p.n_k == 0 || (aligned16(p.k) && aligned16(p.k_out))) &&
                    (!NORM || (aligned16(p.wq) && (p.n_k == 0 || aligned16(p.wk)))) && aligned16(p.pos);
  if (fast) {
    // one float4 per lane, two rows per lane group (config 2: 20.7 us; two
    // float4 and one row per lane group: 20.7-21.2 us; 2 x 2: 21.5 us;
    // 1 x 1: 24.5 us); shapes whose head rows are wider than 64 float4 take
    // two float4 per lane
    if (int e = launch_rope_v<1, 2, NORM>(p, n_tok, st); e != -999) return e;
    if (int e = launch_rope_v<2, 1, NORM>(p, n_tok, st); e != -999) return e;
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
  p.inv_hd = head_dim ? 1.0f / static_cast<float>(head_dim) : 0.0f;
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
