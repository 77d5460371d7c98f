// Row-wise normalisation and softmax kernels for gfx950.
//
//   bh_rms_norm / bh_rms_norm_rows   kernels::rms_norm, rms_norm_rows
//                                    (src/kernels.rs:59-122)
//   bh_add_rms_norm_rows             residual add + RMSNorm (src/forward.rs:708-713)
//   bh_l2_norm_rows                  kernels::l2_norm_rows (src/kernels.rs:126-145)
//   bh_silu_l2_norm_rows             silu + l2_norm_rows (src/forward.rs:524, 539-540)
//   bh_softmax_rows                  kernels::softmax_rows (src/kernels.rs:175-202)
//                                    with the sampler temperature (src/sampler.rs:85,110)
//
// Design.  Every op here reads a row once from HBM and writes it once; the
// arithmetic is < 1 flop/byte, so the roofline is HBM bandwidth and the
// kernels are built around it.  Measured on MI355X, streaming runs fastest
// when every lane moves only one or two 16-byte vectors (a copy at one
// float4 per lane: 6.2 TB/s; at eight per lane: 5.3 TB/s), so rows are
// spread over as many lanes as that takes:
//   * rows of up to 256 floats are owned by a group of G = row_len/4 lanes
//     inside one wave (128-float L2 heads: 32 lanes, 256-float heads: 64),
//     one float4 per lane, several rows per 256-lane block;
//   * longer rows are owned by one block of NT <= 1024 lanes with VPT =
//     ceil(row_len/4/1024) float4 per lane (5120-float hidden rows: 640
//     lanes x 2; softmax takes at least 2 per lane: 2048-float attention rows
//     on 256 lanes x 2);
//   * the row stays in registers between the reduction and the write-back
//     (no second HBM pass); reductions are cross-lane shuffles inside the
//     wave plus an LDS combine across waves in wave order (deterministic);
//   * rows that do not fit this scheme (length not a multiple of 4, unaligned
//     pointers, > 32768 floats) go to a block-per-row looped kernel; softmax
//     rows that are both long and few (the 248320-wide vocabulary rows) are
//     split: pass 1 reduces 32 KB chunks to (max, f64 sum) partials, pass 2
//     (one float4 per lane) folds a row's partials and writes it.
#include <hip/hip_runtime.h>

#include <mutex>

#include <cmath>
#include <string>
#include <type_traits>

#include "common.hpp"

namespace bh {
namespace {

constexpr int kBlock = 256;

template <int N>
using IC = std::integral_constant<int, N>;

// Row geometry: G > 0 -> G lanes per row (power of two <= 64), 256-lane
// blocks, one float4 per lane; G == 0 -> one block of NT lanes per row, VPT
// float4 per lane.
struct RowGeom {
  int G = 0;
  int VPT = 0;
  int NT = 0;
};

// Returns false when the register scheme does not apply (the caller then
// uses the looped kernel).  min_vpt raises the float4 per lane of block rows
// (softmax: 2, measured 143 us vs 158 us for one wave per row and 193 us for
// one float4 per lane on [49152, 2048]).
bool pick_geom(size_t row_len, RowGeom &g, int min_vpt = 1) {
  if (row_len == 0 || (row_len & 3u) != 0) return false;
  const size_t r4 = row_len / 4;
  if (r4 <= 64) {
    g.G = pow2ceil(r4);
    g.VPT = 1;
    g.NT = kBlock;
    return true;
  }
  if (r4 > 8192) return false;
  int vpt = static_cast<int>((r4 + 1023) / 1024);
  if (vpt < min_vpt) vpt = min_vpt;
  const int lanes = static_cast<int>((r4 + vpt - 1) / vpt);
  g.G = 0;
  g.VPT = vpt;
  g.NT = (lanes + 63) / 64 * 64;
  return true;
}

// Calls f(IC<G>, IC<VPT>) for the instantiated geometries; -999 if none.
template <class F>
int with_geom(const RowGeom &g, F &&f) {
  if (g.G > 0) {
    switch (g.G) {
      case 1: return f(IC<1>{}, IC<1>{});
      case 2: return f(IC<2>{}, IC<1>{});
      case 4: return f(IC<4>{}, IC<1>{});
      case 8: return f(IC<8>{}, IC<1>{});
      case 16: return f(IC<16>{}, IC<1>{});
      case 32: return f(IC<32>{}, IC<1>{});
      case 64: return f(IC<64>{}, IC<1>{});
      default: return -999;
    }
  }
  switch (g.VPT) {
    case 1: return f(IC<0>{}, IC<1>{});
    case 2: return f(IC<0>{}, IC<2>{});
    case 3: return f(IC<0>{}, IC<3>{});
    case 4: return f(IC<0>{}, IC<4>{});
    case 5: return f(IC<0>{}, IC<5>{});
    case 6: return f(IC<0>{}, IC<6>{});
    case 7: return f(IC<0>{}, IC<7>{});
    case 8: return f(IC<0>{}, IC<8>{});
    default: return -999;
  }
}

// Lane <-> row mapping of a geometry.
template <int G>
struct RowLane {
  size_t row;  // row index
  int gl;      // lane within the row
  int stride;  // lanes per row
  bool live;   // row exists (group mode pads the last block)
  __device__ explicit RowLane(size_t rows) {
    if constexpr (G == 0) {
      row = blockIdx.x;
      gl = threadIdx.x;
      stride = blockDim.x;
      live = true;
    } else {
      row = static_cast<size_t>(blockIdx.x) * (kBlock / G) + threadIdx.x / G;
      gl = threadIdx.x % G;
      stride = G;
      live = row < rows;
    }
  }
};

// Reduction over the lanes of a row: G-lane DPP/permlane steps, or (G == 0) the whole
// block through `lds` (blockDim.x/64 entries), combined in wave order.
template <int G, class T, class Op>
__device__ __forceinline__ T row_reduce(T v, Op op, T *lds) {
  if constexpr (G > 0) {
    return lane_group_reduce<G>(v, op);
  } else {
    v = lane_group_reduce<64>(v, op);
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    T r = lds[0];
    const int nw = blockDim.x >> 6;
    for (int i = 1; i < nw; ++i) r = op(r, lds[i]);
    return r;
  }
}

constexpr int kMaxWaves = 1024 / 64;



int launch_grid(const RowGeom &g, size_t rows, unsigned *grid, unsigned *block) {
  const size_t rpb = g.G > 0 ? static_cast<size_t>(kBlock / g.G) : 1;
  const size_t n = (rows + rpb - 1) / rpb;
  if (n > 0x7fffffffu) return fail(BH_ERR_SHAPE, "row count exceeds the launch grid limit");
  *grid = static_cast<unsigned>(n);
  *block = static_cast<unsigned>(g.NT);
  return BH_OK;
}

__device__ __forceinline__ float4 f4_zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }

// ---------------------------------------------------------------------------
// RMSNorm rows (optionally with the residual add in front)
// ---------------------------------------------------------------------------

// out = (v * scale) * w, scale = 1 / sqrt(sum(v^2)/row_len + eps), with v = x
// or v = x + r (ADD, also stored to sum_out).  Matches src/kernels.rs:112-120
// operation for operation; only the order of the sum of squares differs
// (lane partials + tree instead of one sequential loop).
template <int G, int VPT, bool ADD>
__global__ __launch_bounds__(1024) void rms_rows_kernel(
    const float *x, const float *__restrict__ r, const float *__restrict__ w,
    float *sum_out, float *out, size_t rows, int row_len, float eps) {
  __shared__ float lds[kMaxWaves];
  const RowLane<G> L(rows);
  const int r4 = row_len >> 2;
  const size_t off = L.live ? L.row * r4 : 0;
  const float4 *x4 = reinterpret_cast<const float4 *>(x) + off;

  float4 v[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = L.gl + i * L.stride;
    v[i] = (L.live && c < r4) ? x4[c] : f4_zero();
  }
  if constexpr (ADD) {
    // the residual's loads go out with x's, before any use
    const float4 *r4p = reinterpret_cast<const float4 *>(r) + off;
    float4 *s4 = reinterpret_cast<float4 *>(sum_out) + off;
    float4 rv[VPT];
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int c = L.gl + i * L.stride;
      rv[i] = (L.live && c < r4) ? r4p[c] : f4_zero();
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int c = L.gl + i * L.stride;
      v[i].x += rv[i].x;
      v[i].y += rv[i].y;
      v[i].z += rv[i].z;
      v[i].w += rv[i].w;
      if (L.live && c < r4) store_stream(s4 + c, v[i]);
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    ss += v[i].x * v[i].x;
    ss += v[i].y * v[i].y;
    ss += v[i].z * v[i].z;
    ss += v[i].w * v[i].w;
  }
  ss = row_reduce<G>(ss, SumOp{}, lds);
  const float scale = rms_scale(ss, 1.0f / static_cast<float>(row_len), eps);
  const float4 *w4 = reinterpret_cast<const float4 *>(w);
  float4 *o4 = reinterpret_cast<float4 *>(out) + off;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = L.gl + i * L.stride;
    if (L.live && c < r4) {
      const float4 wv = w4[c];
      float4 o;
      o.x = (v[i].x * scale) * wv.x;
      o.y = (v[i].y * scale) * wv.y;
      o.z = (v[i].z * scale) * wv.z;
      o.w = (v[i].w * scale) * wv.w;
      store_stream(o4 + c, o);
    }
  }
}

// Looped fallback: one block per row, any length / alignment.  Reads x twice.
template <bool ADD>
__global__ __launch_bounds__(kBlock) void rms_rows_loop_kernel(
    const float *x, const float *__restrict__ r, const float *__restrict__ w,
    float *sum_out, float *out, int row_len, float eps) {
  __shared__ float lds[kBlock / 64];
  const size_t off = static_cast<size_t>(blockIdx.x) * row_len;
  float ss = 0.0f;
  for (int c = threadIdx.x; c < row_len; c += kBlock) {
    float v = x[off + c];
    if constexpr (ADD) {
      v += r[off + c];
      sum_out[off + c] = v;
    }
    ss += v * v;
  }
  ss = group_reduce<kBlock>(ss, SumOp{}, lds);
  const float scale = rms_scale(ss, 1.0f / static_cast<float>(row_len), eps);
  for (int c = threadIdx.x; c < row_len; c += kBlock) {
    // each thread re-reads exactly the elements it wrote, so sum_out == x is safe
    const float v = ADD ? sum_out[off + c] : x[off + c];
    out[off + c] = (v * scale) * w[c];
  }
}

// ---------------------------------------------------------------------------
// L2 rows (optionally SiLU first)
// ---------------------------------------------------------------------------

// out = v * (1 / max(sqrt((f32) sum_f64(v^2)), eps)), v = x or silu(x)
// (src/kernels.rs:136-143; silu src/kernels.rs:148-150).
template <int G, int VPT, bool SILU>
__global__ __launch_bounds__(1024) void l2_rows_kernel(const float *x, float *out, size_t rows,
                                                       int row_len, float eps) {
  __shared__ double lds[kMaxWaves];
  const RowLane<G> L(rows);
  const int r4 = row_len >> 2;
  const size_t off = L.live ? L.row * r4 : 0;
  const float4 *x4 = reinterpret_cast<const float4 *>(x) + off;

  float4 v[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = L.gl + i * L.stride;
    v[i] = (L.live && c < r4) ? x4[c] : f4_zero();
    if constexpr (SILU) {
      v[i].x = silu(v[i].x);
      v[i].y = silu(v[i].y);
      v[i].z = silu(v[i].z);
      v[i].w = silu(v[i].w);
    }
  }
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    ss += static_cast<double>(v[i].x) * static_cast<double>(v[i].x);
    ss += static_cast<double>(v[i].y) * static_cast<double>(v[i].y);
    ss += static_cast<double>(v[i].z) * static_cast<double>(v[i].z);
    ss += static_cast<double>(v[i].w) * static_cast<double>(v[i].w);
  }
  ss = row_reduce<G>(ss, SumOp{}, lds);
  const float scale = 1.0f / fmaxf(sqrtf(static_cast<float>(ss)), eps);
  float4 *o4 = reinterpret_cast<float4 *>(out) + off;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = L.gl + i * L.stride;
    if (L.live && c < r4) {
      store_stream(o4 + c, make_float4(v[i].x * scale, v[i].y * scale, v[i].z * scale, v[i].w * scale));
    }
  }
}

template <bool SILU>
__global__ __launch_bounds__(kBlock) void l2_rows_loop_kernel(const float *x, float *out,
                                                              int row_len, float eps) {
  __shared__ double lds[kBlock / 64];
  const size_t off = static_cast<size_t>(blockIdx.x) * row_len;
  double ss = 0.0;
  for (int c = threadIdx.x; c < row_len; c += kBlock) {
    float v = x[off + c];
    if constexpr (SILU) v = silu(v);
    ss += static_cast<double>(v) * static_cast<double>(v);
  }
  ss = group_reduce<kBlock>(ss, SumOp{}, lds);
  const float scale = 1.0f / fmaxf(sqrtf(static_cast<float>(ss)), eps);
  for (int c = threadIdx.x; c < row_len; c += kBlock) {
    float v = x[off + c];
    if constexpr (SILU) v = silu(v);
    out[off + c] = v * scale;
  }
}

// ---------------------------------------------------------------------------
// Softmax rows
// ---------------------------------------------------------------------------

// (f32)((f64)e * inv) per element: the sampler's normalisation
__device__ __forceinline__ float sampler_norm(float e, double inv) {
  return static_cast<float>(static_cast<double>(e) * inv);
}
__device__ __forceinline__ float4 sampler_norm4(float4 e, double inv) {
  return make_float4(sampler_norm(e.x, inv), sampler_norm(e.y, inv), sampler_norm(e.z, inv),
                     sampler_norm(e.w, inv));
}

// y = x * inv_t; m = max(y) (NaN never becomes the max, as `if v > max`);
// e = expf(y - m); s = sum_f64(e); out = e * (1 / (f32)s)
// (src/kernels.rs:184-200).  -inf entries give expf(-inf) = 0.  With SN
// (the sampler's normalisation, src/sampler.rs:118-126) out is instead
// (f32)((f64)e * (1 / s)), the division and the product in f64.
template <int G, int VPT, bool SN>
__global__ __launch_bounds__(1024) void softmax_rows_kernel(const float *x, float *out, size_t rows,
                                                            int row_len, float inv_t) {
  __shared__ float lds_m[kMaxWaves];
  __shared__ double lds_s[kMaxWaves];
  const RowLane<G> L(rows);
  const int r4 = row_len >> 2;
  const size_t off = L.live ? L.row * r4 : 0;
  const float4 *x4 = reinterpret_cast<const float4 *>(x) + off;
  const float ninf = -INFINITY;

  // loads first, all in flight together; scale after
  float4 v[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = L.gl + i * L.stride;
    v[i] = (L.live && c < r4) ? x4[c] : make_float4(ninf, ninf, ninf, ninf);
  }
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = L.gl + i * L.stride;
    if (L.live && c < r4) {
      v[i].x *= inv_t;
      v[i].y *= inv_t;
      v[i].z *= inv_t;
      v[i].w *= inv_t;
    }
  }
  float m = ninf;
  const MaxOp mx;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    m = mx(m, v[i].x);
    m = mx(m, v[i].y);
    m = mx(m, v[i].z);
    m = mx(m, v[i].w);
  }
  m = row_reduce<G>(m, mx, lds_m);
  double s = 0.0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int c = L.gl + i * L.stride;
    if (L.live && c < r4) {
      v[i].x = expf(v[i].x - m);
      v[i].y = expf(v[i].y - m);
      v[i].z = expf(v[i].z - m);
      v[i].w = expf(v[i].w - m);
      s += static_cast<double>(v[i].x);
      s += static_cast<double>(v[i].y);
      s += static_cast<double>(v[i].z);
      s += static_cast<double>(v[i].w);
    }
  }
  s = row_reduce<G>(s, SumOp{}, lds_s);
  float4 *o4 = reinterpret_cast<float4 *>(out) + off;
  if constexpr (SN) {
    const double inv = 1.0 / s;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int c = L.gl + i * L.stride;
      if (L.live && c < r4) store_stream(o4 + c, sampler_norm4(v[i], inv));
    }
  } else {
    const float inv = 1.0f / static_cast<float>(s);
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int c = L.gl + i * L.stride;
      if (L.live && c < r4) {
        store_stream(o4 + c, make_float4(v[i].x * inv, v[i].y * inv, v[i].z * inv, v[i].w * inv));
      }
    }
  }
}

// (max, f64 sum of expf(y - max)) of a part of a row.  Merging two parts
// rescales each sum by exp(part max - merged max) in f64.  A part with no
// value above -inf (m = -inf) adds its sum unscaled: 0, or NaN if it held a
// NaN, which the reference's sum carries through.  A row with no value above
// -inf ends with S = 0 and an output of expf(-inf - -inf) * inf = NaN, as
// the reference's.
struct MaxSum {
  float m;
  double s;
};

__device__ __forceinline__ double ms_scaled(const MaxSum &a, double M) {
  return a.m == -INFINITY ? a.s : a.s * exp(static_cast<double>(a.m) - M);
}

// Split-row pass 1: block (c, r) reduces chunk c of row r (kSplitVPT float4
// per lane, loaded up front) to (max, sum of e^(y - max)).  The chunk max
// comes first, so each element costs one exponential.  Both passes are
// bound by the exponentials as much as by HBM, so they use exp_hw (a few
// 1e-7 relative, inside the softmax tolerance) and each lane adds its 8
// values in f32 before the f64 sum (pass 1 of [64, 248320]: 14.1 us against
// 15.2 us with expf and f64 per element; 8 KB chunks make pass 1 faster
// still but double the chunk states every pass-2 block folds: slower overall).
// Pass 2 folds each row's chunk states (the kernel boundary orders the two
// launches; no block waits for another).
constexpr int kSplitVPT = 4;
constexpr size_t kMaxSplitRows = 65535;  // grid.y limit of both passes
constexpr size_t kSplitChunk4 = static_cast<size_t>(kBlock) * kSplitVPT;  // float4 per chunk

struct SplitScratch {
  double *part_s;  // [rows][nch]
  float *part_m;   // [rows][nch]
};

// Chunk c of row r to (max, sum of e^(y - max)) in every lane of the block;
// v keeps the chunk's y = x * inv_t (padding lanes -inf).  Every lane of the
// block must call it (two block reductions).
__device__ __forceinline__ void split_chunk_stats(const float4 *x, size_t r4, float inv_t, size_t r,
                                                  int c, float4 (&v)[kSplitVPT], float *lm,
                                                  double *ls, float &m_out, double &s_out) {
  const size_t base = r * r4 + static_cast<size_t>(c) * kSplitChunk4;
  const size_t end = (r + 1) * r4;
  const float ninf = -INFINITY;
  // all loads in flight before the first use (lanes past the row's end
  // re-read its last float4 and are masked below); a load whose value is
  // used inside its own branch gets a wait of its own
#pragma unroll
  for (int i = 0; i < kSplitVPT; ++i) {
    const size_t e = base + threadIdx.x + i * kBlock;
    v[i] = x[e < end ? e : end - 1];
  }
#pragma unroll
  for (int i = 0; i < kSplitVPT; ++i) {
    const size_t e = base + threadIdx.x + i * kBlock;
    if (e < end) {
      v[i].x *= inv_t;
      v[i].y *= inv_t;
      v[i].z *= inv_t;
      v[i].w *= inv_t;
    } else {
      v[i] = make_float4(ninf, ninf, ninf, ninf);
    }
  }
  const MaxOp mx;
  float m = ninf;
#pragma unroll
  for (int i = 0; i < kSplitVPT; ++i) {
    m = mx(m, v[i].x);
    m = mx(m, v[i].y);
    m = mx(m, v[i].z);
    m = mx(m, v[i].w);
  }
  m = group_reduce<kBlock>(m, mx, lm);
  double sum = 0.0;
  if (m != ninf) {
    // masked (-inf) and padding entries give exp_hw(-inf) = 0
    float q[kSplitVPT];
#pragma unroll
    for (int i = 0; i < kSplitVPT; ++i)
      q[i] = (exp_hw(v[i].x - m) + exp_hw(v[i].y - m)) + (exp_hw(v[i].z - m) + exp_hw(v[i].w - m));
#pragma unroll
    for (int i = 0; i < kSplitVPT; ++i) sum += static_cast<double>(q[i]);
  } else {
    // a chunk with no number above -inf adds 0, unless it holds a NaN
    // (which the reference's sum carries through)
#pragma unroll
    for (int i = 0; i < kSplitVPT; ++i)
      if (isnan(v[i].x) || isnan(v[i].y) || isnan(v[i].z) || isnan(v[i].w)) sum = NAN;
  }
  s_out = group_reduce<kBlock>(sum, SumOp{}, ls);
  m_out = m;
}

__global__ __launch_bounds__(kBlock) void softmax_split_stats_kernel(const float4 *x, size_t r4,
                                                                     float inv_t, SplitScratch sc) {
  __shared__ float lm[kBlock / 64];
  __shared__ double ls[kBlock / 64];
  const size_t r = blockIdx.y;
  const int nch = gridDim.x;
  float4 v[kSplitVPT];
  float m;
  double sum;
  split_chunk_stats(x, r4, inv_t, r, static_cast<int>(blockIdx.x), v, lm, ls, m, sum);
  if (threadIdx.x == 0) {
    sc.part_m[r * nch + blockIdx.x] = m;
    sc.part_s[r * nch + blockIdx.x] = sum;
  }
}

// The fold of a row's nch chunk states into (M, 1/(f32)S) (and 1/S in f64
// for SN) by one wave: lane i takes chunks i, i + 64, ..., then a fixed
// shuffle tree, so every block that folds a row gets the same bits.  m0/s0
// are chunk `lane`'s state (loaded early by the caller, -inf/0 past nch);
// load(i) returns the state of chunk i >= 64.
template <bool SN, class Load>
__device__ __forceinline__ void split_fold(int nch, float m0, double s0, Load load, float2 &stat,
                                           double &stat_inv) {
  const int lane = static_cast<int>(threadIdx.x & 63);
  const MaxOp mx;
  float M = mx(-INFINITY, m0);  // the reference's `if v > max` ignores a NaN state
  for (int i = lane + 64; i < nch; i += 64) M = mx(M, load(i).m);
  M = lane_group_reduce<64>(M, mx);
  double S = lane < nch ? ms_scaled(MaxSum{m0, s0}, M) : 0.0;
  for (int i = lane + 64; i < nch; i += 64) S += ms_scaled(load(i), M);
  S = lane_group_reduce<64>(S, SumOp{});
  if (lane == 0) {
    stat = make_float2(M, 1.0f / static_cast<float>(S));
    if constexpr (SN) stat_inv = 1.0 / S;
  }
}

// Split-row pass 2: the block's first wave folds the row's chunk states into
// (M, 1/(f32)S) while the block's x loads are in flight -- every block of a
// row folds the same states in the same fixed order (lane i takes chunks i,
// i+64, ..., then a fixed shuffle tree), so all of them agree bit for bit --
// then each lane writes e^(y - M) * (1 / (f32)S), the reference's output
// formula (the exponential by exp_hw), for its kSplitWV float4.
constexpr int kSplitWV = 4;  // measured: 17.6 us vs 20.2 (2) and 21.3 (8) on [64, 248320]
template <bool SN>
__global__ __launch_bounds__(kBlock) void softmax_split_write_kernel(const float4 *x, float4 *out,
                                                                     size_t r4, float inv_t,
                                                                     SplitScratch sc, int nch) {
  __shared__ float2 stat;
  __shared__ double stat_inv;  // 1 / S in f64 (SN)
  const size_t r = blockIdx.y;
  const size_t c0 = static_cast<size_t>(blockIdx.x) * (kBlock * kSplitWV) + threadIdx.x;
  // wave 0 requests the row's chunk states before its x loads: loads return
  // in order, so the fold does not wait for the x data
  float pm0 = -INFINITY;
  double ps0 = 0.0;
  const float *pm = sc.part_m + r * nch;
  const double *ps = sc.part_s + r * nch;
  if (threadIdx.x < 64 && static_cast<int>(threadIdx.x) < nch) {
    pm0 = pm[threadIdx.x];
    ps0 = ps[threadIdx.x];
  }
  float4 v[kSplitWV];
#pragma unroll
  for (int i = 0; i < kSplitWV; ++i) {
    const size_t c = c0 + static_cast<size_t>(i) * kBlock;
    if (c < r4) v[i] = load_stream(x + r * r4 + c);
  }
  if (threadIdx.x < 64)
    split_fold<SN>(nch, pm0, ps0, [&](int i) { return MaxSum{pm[i], ps[i]}; }, stat, stat_inv);
  __syncthreads();
  const float2 st = stat;
#pragma unroll
  for (int i = 0; i < kSplitWV; ++i) {
    const size_t c = c0 + static_cast<size_t>(i) * kBlock;
    if (c < r4) {
      const float4 e = make_float4(exp_hw(v[i].x * inv_t - st.x), exp_hw(v[i].y * inv_t - st.x),
                                   exp_hw(v[i].z * inv_t - st.x), exp_hw(v[i].w * inv_t - st.x));
      if constexpr (SN)
        store_stream(out + r * r4 + c, sampler_norm4(e, stat_inv));
      else
        store_stream(out + r * r4 + c, make_float4(e.x * st.y, e.y * st.y, e.z * st.y, e.w * st.y));
    }
  }
}

// Looped fallback for rows whose length is not a multiple of 4 or whose
// pointers are unaligned: one block per row, three sweeps (max, sum, write).
template <bool SN>
__global__ __launch_bounds__(kBlock) void softmax_loop_kernel(const float *x, float *out,
                                                              size_t row_len, float inv_t) {
  __shared__ float lm[kBlock / 64];
  __shared__ double ls[kBlock / 64];
  const float *xr = x + blockIdx.x * row_len;
  float *orow = out + blockIdx.x * row_len;
  const MaxOp mx;
  float m = -INFINITY;
  for (size_t c = threadIdx.x; c < row_len; c += kBlock) m = mx(m, xr[c] * inv_t);
  m = group_reduce<kBlock>(m, mx, lm);
  double s = 0.0;
  for (size_t c = threadIdx.x; c < row_len; c += kBlock)
    s += static_cast<double>(expf(xr[c] * inv_t - m));
  s = group_reduce<kBlock>(s, SumOp{}, ls);
  const float inv = 1.0f / static_cast<float>(s);
  const double inv_d = 1.0 / s;
  // each element is read by the lane that writes it: in place is safe
  for (size_t c = threadIdx.x; c < row_len; c += kBlock) {
    const float e = expf(xr[c] * inv_t - m);
    orow[c] = SN ? sampler_norm(e, inv_d) : e * inv;
  }
}

// ---------------------------------------------------------------------------
// host dispatch
// ---------------------------------------------------------------------------

int grid_for(size_t rows, int rows_per_block, unsigned *grid) {
  const size_t g = (rows + rows_per_block - 1) / rows_per_block;
  if (g > 0x7fffffffu) return fail(BH_ERR_SHAPE, "row count exceeds the launch grid limit");
  *grid = static_cast<unsigned>(g);
  return BH_OK;
}

int rms_rows_impl(const float *x, const float *r, const float *w, float *sum_out,
                  float *out, size_t rows, size_t row_len, float eps, hipStream_t st,
                  bool add) {
  if (rows == 0) return ok();
  if (row_len > 0x7fffffffu) return fail(BH_ERR_SHAPE, "row_len exceeds 2^31-1");
  RowGeom g;
  const bool vec = pick_geom(row_len, g) && aligned16(x) && aligned16(w) && aligned16(out) &&
                   (!add || (aligned16(r) && aligned16(sum_out)));
  // 5120-wide rows, 2048..4095 of them: one wave per row (20 float4 per lane,
  // four rows per 256-lane block) measured 8-10% faster than the 640-lane
  // block-per-row form (T=2048: 15.1 vs 16.6 us, T=3072: 22.1 vs 24.1 us);
  // below and above that range the block form is as fast or faster.  The
  // residual-add form stays on the block form: with two inputs per lane it
  // needs more than the 128 registers per lane the kernel's 1024-lane bound
  // allows, and spilled.
  if (vec && !add && row_len == 5120 && rows >= 2048 && rows < 4096) {
    const unsigned grid = static_cast<unsigned>((rows + 3) / 4);
    BH_LAUNCH((rms_rows_kernel<64, 20, false>), grid, 256, 0, st, x, r, w, sum_out, out, rows,
              5120, eps);
    return ok();
  }
  if (vec) {
    int st_code = with_geom(g, [&](auto GC, auto VC) -> int {
      constexpr int G_ = decltype(GC)::value;
      constexpr int V_ = decltype(VC)::value;
      unsigned grid, block;
      if (int e = launch_grid(g, rows, &grid, &block)) return e;
      if (add) {
        BH_LAUNCH((rms_rows_kernel<G_, V_, true>), grid, block, 0, st, x, r, w, sum_out, out,
                  rows, static_cast<int>(row_len), eps);
      } else {
        BH_LAUNCH((rms_rows_kernel<G_, V_, false>), grid, block, 0, st, x, r, w, sum_out, out,
                  rows, static_cast<int>(row_len), eps);
      }
      return ok();
    });
    if (st_code != -999) return st_code;
  }
  unsigned grid;
  if (int e = grid_for(rows, 1, &grid)) return e;
  if (add) {
    BH_LAUNCH((rms_rows_loop_kernel<true>), grid, kBlock, 0, st, x, r, w, sum_out, out,
              static_cast<int>(row_len), eps);
  } else {
    BH_LAUNCH((rms_rows_loop_kernel<false>), grid, kBlock, 0, st, x, r, w, sum_out, out,
              static_cast<int>(row_len), eps);
  }
  return ok();
}

template <bool SILU>
int l2_rows_impl(const float *x, float *out, size_t rows, size_t row_len, float eps,
                 hipStream_t st) {
  if (rows == 0) return ok();
  if (row_len > 0x7fffffffu) return fail(BH_ERR_SHAPE, "row_len exceeds 2^31-1");
  RowGeom g;
  if (pick_geom(row_len, g) && aligned16(x) && aligned16(out)) {
    int st_code = with_geom(g, [&](auto GC, auto VC) -> int {
      constexpr int G_ = decltype(GC)::value;
      constexpr int V_ = decltype(VC)::value;
      unsigned grid, block;
      if (int e = launch_grid(g, rows, &grid, &block)) return e;
      BH_LAUNCH((l2_rows_kernel<G_, V_, SILU>), grid, block, 0, st, x, out, rows,
                static_cast<int>(row_len), eps);
      return ok();
    });
    if (st_code != -999) return st_code;
  }
  unsigned grid;
  if (int e = grid_for(rows, 1, &grid)) return e;
  BH_LAUNCH((l2_rows_loop_kernel<SILU>), grid, kBlock, 0, st, x, out, static_cast<int>(row_len),
            eps);
  return ok();
}

// Scratch of bh_softmax_rows_noalloc: a fixed device array instead of the
// library's growable buffer, so that entry point never allocates.  Host code
// must not pass `scratch` itself to a kernel (in host code the name is a
// stand-in, not a device address): it uses the address hipGetSymbolAddress
// returns for the current device, looked up once per device.
constexpr size_t kNoAllocScratchBytes = size_t{1} << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
char *g_noalloc_ptr[kMaxDevices] = {};

// This device's address of `scratch`, or nullptr with the status recorded.
char *noalloc_scratch() {
  int dev = 0;
  if (check_hip(hipGetDevice(&dev), "hipGetDevice") != BH_OK) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    fail(BH_ERR_HIP, "softmax_rows_noalloc: device ordinal out of range");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (g_noalloc_ptr[dev] == nullptr) {
    void *p = nullptr;
    if (check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                  "softmax_rows_noalloc: hipGetSymbolAddress") != BH_OK)
      return nullptr;
    g_noalloc_ptr[dev] = static_cast<char *>(p);
  }
  return g_noalloc_ptr[dev];
}

// Wide-row softmax: stats pass then write pass.  `fixed` (with `fixed_cap`
// bytes) is the no-allocation entry point's scratch; nullptr takes the
// library's growable per-device buffer.
template <bool SN>
int softmax_split(const float *x, float *out, size_t rows, size_t row_len, float inv_t,
                  hipStream_t st, char *fixed, size_t fixed_cap) {
  if (rows > kMaxSplitRows)
    return fail(BH_ERR_SHAPE, "softmax_rows: too many wide rows for one launch");
  const bool vec = (row_len % 4 == 0) && aligned16(x) && aligned16(out);
  if (!vec) {
    if (rows > 0x7fffffffu) return fail(BH_ERR_SHAPE, "softmax_rows: too many rows");
    BH_LAUNCH(softmax_loop_kernel<SN>, static_cast<unsigned>(rows), kBlock, 0, st, x, out, row_len,
              inv_t);
    return ok();
  }
  const size_t r4 = row_len / 4;
  const size_t nch = (r4 + kSplitChunk4 - 1) / kSplitChunk4;
  if (nch > 65535) return fail(BH_ERR_SHAPE, "softmax_rows: row too long");
  const size_t nparts = rows * nch;
  // scratch: f64 partial sums, then f32 partial maxima
  const size_t off_m = nparts * sizeof(double);
  const size_t need = off_m + nparts * sizeof(float);
  char *buf;
  if (fixed != nullptr) {
    if (need > fixed_cap)
      return fail(BH_ERR_SHAPE, "softmax_rows_noalloc: " + std::to_string(rows) + " rows of " +
                                    std::to_string(row_len) + " need " + std::to_string(need) +
                                    " scratch bytes, above the fixed " +
                                    std::to_string(fixed_cap));
    buf = fixed;
  } else {
    buf = static_cast<char *>(device_scratch(need, kScratchSoftmax, st));
    if (buf == nullptr) return BH_ERR_HIP;
  }
  SplitScratch sc;
  sc.part_s = reinterpret_cast<double *>(buf);
  sc.part_m = reinterpret_cast<float *>(buf + off_m);
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  BH_LAUNCH(softmax_split_stats_kernel, dim3(static_cast<unsigned>(nch), static_cast<unsigned>(rows)),
            kBlock, 0, st, x4, r4, inv_t, sc);
  const size_t wblocks = (r4 + kBlock * kSplitWV - 1) / (kBlock * kSplitWV);
  if (wblocks > 0x7fffffffu) return fail(BH_ERR_SHAPE, "softmax_rows: row too long");
  BH_LAUNCH(softmax_split_write_kernel<SN>,
            dim3(static_cast<unsigned>(wblocks), static_cast<unsigned>(rows)), kBlock, 0, st, x4,
            reinterpret_cast<float4 *>(out), r4, inv_t, sc, static_cast<int>(nch));
  return ok();
}

}  // namespace
}  // namespace bh

using namespace bh;

extern "C" int bh_rms_norm(const float *x, const float *w, size_t n, float eps, float *out,
                           bh_stream stream) {
  if (n == 0) return ok();
  if (!x || !w || !out) return fail(BH_ERR_ARG, "rms_norm: null pointer");
  return rms_rows_impl(x, nullptr, w, nullptr, out, 1, n, eps, as_stream(stream), false);
}

extern "C" int bh_rms_norm_rows(const float *x, size_t x_len, const float *w, size_t w_len,
                                size_t row_len, float eps, float *out, bh_stream stream) {
  if (w_len != row_len)
    return fail(BH_ERR_SHAPE, "rms_norm_rows: weight len " + std::to_string(w_len) +
                                  " != row_len " + std::to_string(row_len));
  if (row_len == 0 || x_len % row_len != 0)
    return fail(BH_ERR_SHAPE, "rms_norm_rows: x len " + std::to_string(x_len) +
                                  " not divisible by row_len " + std::to_string(row_len));
  if (x_len == 0) return ok();
  if (!x || !w || !out) return fail(BH_ERR_ARG, "rms_norm_rows: null pointer");
  return rms_rows_impl(x, nullptr, w, nullptr, out, x_len / row_len, row_len, eps,
                       as_stream(stream), false);
}

extern "C" int bh_add_rms_norm_rows(const float *x, const float *residual, size_t x_len,
                                    const float *w, size_t w_len, size_t row_len, float eps,
                                    float *sum_out, float *out, bh_stream stream) {
  if (w_len != row_len)
    return fail(BH_ERR_SHAPE, "add_rms_norm_rows: weight len " + std::to_string(w_len) +
                                  " != row_len " + std::to_string(row_len));
  if (row_len == 0 || x_len % row_len != 0)
    return fail(BH_ERR_SHAPE, "add_rms_norm_rows: x len " + std::to_string(x_len) +
                                  " not divisible by row_len " + std::to_string(row_len));
  if (x_len == 0) return ok();
  if (!x || !residual || !w || !sum_out || !out)
    return fail(BH_ERR_ARG, "add_rms_norm_rows: null pointer");
  return rms_rows_impl(x, residual, w, sum_out, out, x_len / row_len, row_len, eps,
                       as_stream(stream), true);
}

extern "C" int bh_l2_norm_rows(const float *x, size_t x_len, size_t row_len, float eps,
                               float *out, bh_stream stream) {
  if (row_len == 0 || x_len % row_len != 0)
    return fail(BH_ERR_SHAPE, "l2_norm_rows: x len " + std::to_string(x_len) +
                                  " not divisible by row_len " + std::to_string(row_len));
  if (x_len == 0) return ok();
  if (!x || !out) return fail(BH_ERR_ARG, "l2_norm_rows: null pointer");
  return l2_rows_impl<false>(x, out, x_len / row_len, row_len, eps, as_stream(stream));
}

extern "C" int bh_silu_l2_norm_rows(const float *x, size_t x_len, size_t row_len, float eps,
                                    float *out, bh_stream stream) {
  if (row_len == 0 || x_len % row_len != 0)
    return fail(BH_ERR_SHAPE, "silu_l2_norm_rows: x len " + std::to_string(x_len) +
                                  " not divisible by row_len " + std::to_string(row_len));
  if (x_len == 0) return ok();
  if (!x || !out) return fail(BH_ERR_ARG, "silu_l2_norm_rows: null pointer");
  return l2_rows_impl<true>(x, out, x_len / row_len, row_len, eps, as_stream(stream));
}

namespace bh {
namespace {
template <bool SN>
int softmax_impl(const float *x, size_t x_len, size_t row_len, float inv_temp, float *out,
                 hipStream_t st, bool noalloc) {
  const char *name = noalloc ? "softmax_rows_noalloc" : "softmax_rows";
  if (row_len == 0 || x_len % row_len != 0)
    return fail(BH_ERR_SHAPE, std::string(name) + ": x len " + std::to_string(x_len) +
                                  " not divisible by row_len " + std::to_string(row_len));
  if (x_len == 0) return ok();
  if (!x || !out) return fail(BH_ERR_ARG, std::string(name) + ": null pointer");
  const size_t rows = x_len / row_len;
  RowGeom g;
  const bool fits = pick_geom(row_len, g, 2) && aligned16(x) && aligned16(out);
  const bool few_long_rows = rows < 1024 && row_len >= 16384;
  if (fits && !few_long_rows) {
    int st_code = with_geom(g, [&](auto GC, auto VC) -> int {
      constexpr int G_ = decltype(GC)::value;
      constexpr int V_ = decltype(VC)::value;
      unsigned grid, block;
      if (int e = launch_grid(g, rows, &grid, &block)) return e;
      BH_LAUNCH((softmax_rows_kernel<G_, V_, SN>), grid, block, 0, st, x, out, rows,
                static_cast<int>(row_len), inv_temp);
      return ok();
    });
    if (st_code != -999) return st_code;
  }
  // The split path reads x again in pass 2; each element is read by the same
  // thread just before it writes it, so out == x (in place) is safe there too.
  char *fixed = nullptr;
  if (noalloc) {
    fixed = noalloc_scratch();
    if (fixed == nullptr) return BH_ERR_HIP;
  }
  return softmax_split<SN>(x, out, rows, row_len, inv_temp, st, fixed, kNoAllocScratchBytes);
}
}  // namespace
}  // namespace bh

extern "C" int bh_softmax_rows(const float *x, size_t x_len, size_t row_len, float inv_temp,
                               float *out, bh_stream stream) {
  return softmax_impl<false>(x, x_len, row_len, inv_temp, out, as_stream(stream), false);
}

extern "C" int bh_softmax_rows_ex(const float *x, size_t x_len, size_t row_len, float inv_temp,
                                  int flags, float *out, bh_stream stream) {
  if ((flags & ~BH_SOFTMAX_SAMPLER_NORM) != 0)
    return fail(BH_ERR_ARG, "softmax_rows_ex: unknown flags " + std::to_string(flags));
  if (flags & BH_SOFTMAX_SAMPLER_NORM)
    return softmax_impl<true>(x, x_len, row_len, inv_temp, out, as_stream(stream), false);
  return softmax_impl<false>(x, x_len, row_len, inv_temp, out, as_stream(stream), false);
}

extern "C" int bh_softmax_rows_noalloc(const float *x, size_t x_len, size_t row_len,
                                       float inv_temp, float *out, bh_stream stream) {
  return softmax_impl<false>(x, x_len, row_len, inv_temp, out, as_stream(stream), true);
}
