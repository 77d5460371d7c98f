// Planar-quantized KV cache append (reference: src/kvquant.rs, PlanarQuant;
// AttnCache::append_k_quantized / append_v_quantized / append_v,
// src/forward.rs:99-140).  The attention over such a cache is in
// attention.hip.
//
// Tables (host, once per (hd, bits)): the Lloyd-Max centroids of a unit
// hd-vector coordinate (N(0, 1/hd)) by the reference's float64 iteration
// (src/kvquant.rs:58-118, erf by Abramowitz & Stegun 7.1.26), and the Givens
// table from splitmix64 seeded 42 (src/kvquant.rs:124-146).  Both are the
// reference's steps in the same order and precision (no contraction), so the
// f32 values are the reference's and every stored index matches it.
//
// Store kernel: one wave per (token, kv head) vector of 256 floats, lane l
// holding coordinates 4l .. 4l+3 (the two Givens pairs 2l, 2l+1).  The norm
// is the reference's sequential f32 sum of the squares (one lane adds the 256
// squares from LDS in index order); then the unit vector x * (1/n) (0 for
// n <= 1e-12), the rotation [c a - s b, s a + c b], the first nearest
// centroid by |v - c| (a linear scan, as the reference), and the LSB-first
// packing (each output byte assembled by one lane from the indices in LDS).
// The indices and the norm are the reference's bit for bit.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <string>

#include "common.hpp"
#include "kvquant.hpp"

namespace bh {

namespace {

// src/kvquant.rs:34-44
double as_erf(double x) {
  const double sign = x < 0.0 ? -1.0 : 1.0;
  x = std::fabs(x);
  const double t = 1.0 / (1.0 + 0.3275911 * x);
  const double y =
      1.0 - (((((1.061405429 * t - 1.453152027) * t) + 1.421413741) * t - 0.284496736) * t +
             0.254829592) *
                t * std::exp(-x * x);
  return sign * y;
}
double g_cdf(double x, double sigma) { return 0.5 * (1.0 + as_erf(x / (sigma * 1.4142135623730951))); }
double g_pdf(double x, double sigma) {
  return std::exp(-(x * x) / (2.0 * sigma * sigma)) / (sigma * std::sqrt(2.0 * 3.141592653589793));
}

// solve_lloyd_max, src/kvquant.rs:58-99
void lloyd_max(size_t d, unsigned bits, float *out) {
  const size_t n = size_t{1} << bits;
  const double sigma = 1.0 / std::sqrt(static_cast<double>(d));
  const double lo = -3.5 * sigma, hi = 3.5 * sigma, outer = 12.0 * sigma;
  double c[256], nx[256], e[257];
  for (size_t i = 0; i < n; ++i) c[i] = lo + (hi - lo) * (static_cast<double>(i) + 0.5) / static_cast<double>(n);
  for (int it = 0; it < 300; ++it) {
    e[0] = -outer;
    for (size_t i = 0; i + 1 < n; ++i) e[i + 1] = (c[i] + c[i + 1]) / 2.0;
    e[n] = outer;
    for (size_t i = 0; i < n; ++i) {
      const double mass = g_cdf(e[i + 1], sigma) - g_cdf(e[i], sigma);
      nx[i] = mass > 1e-15 ? sigma * sigma * (g_pdf(e[i], sigma) - g_pdf(e[i + 1], sigma)) / mass : c[i];
    }
    double shift = 0.0;
    for (size_t i = 0; i < n; ++i) {
      const double dl = std::fabs(nx[i] - c[i]);
      if (dl > shift) shift = dl;
      c[i] = nx[i];
    }
    if (shift < 1e-12) break;
  }
  for (size_t i = 0; i < n; ++i) out[i] = static_cast<float>(c[i]);
}

// givens_table, src/kvquant.rs:124-146
void givens(size_t d, float *gc, float *gs) {
  uint64_t st = 42;
  for (size_t i = 0; i < (d + 1) / 2; ++i) {
    uint64_t z = (st += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    const double u = static_cast<double>(z >> 11) / 9007199254740992.0;
    const double t = u * 6.283185307179586;
    gc[i] = static_cast<float>(std::cos(t));
    gs[i] = static_cast<float>(std::sin(t));
  }
}

}  // namespace

bool planar_tables(size_t hd, unsigned bits, PlanarTables *out) {
  if (hd != static_cast<size_t>(kPlanarHd) || bits < 1 || bits > 8) return false;
  static std::mutex mu;
  static PlanarTables cache[9];
  static bool ready[9] = {};
  std::lock_guard<std::mutex> lock(mu);
  if (!ready[bits]) {
    PlanarTables t{};
    lloyd_max(hd, bits, t.cent);
    givens(hd, t.gc, t.gs);
    cache[bits] = t;
    ready[bits] = true;
  }
  *out = cache[bits];
  return true;
}

namespace {

constexpr int kRowsPerBlock = 4;  // one wave per vector

// Quantizes the vector this wave holds (lane: coordinates 4 lane .. +3)
// into packed[32 * bits] and *norm (lane 0 writes it).
__device__ __forceinline__ void planar_quantize_wave(float4 x, int bits, const float *s_c,
                                                     const float *s_gc, const float *s_gs,
                                                     float *s_sq, uint8_t *s_idx, uint8_t *packed,
                                                     float *norm) {
  const int lane = threadIdx.x & 63;
  s_sq[4 * lane] = x.x * x.x;
  s_sq[4 * lane + 1] = x.y * x.y;
  s_sq[4 * lane + 2] = x.z * x.z;
  s_sq[4 * lane + 3] = x.w * x.w;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float ss = 0.0f;
  if (lane == 0) {
    // src/kvquant.rs:382: x.iter().map(|v| v * v).sum(), in index order
    for (int i = 0; i < kPlanarHd; ++i) ss += s_sq[i];
  }
  ss = __shfl(ss, 0, 64);
  const float n = sqrtf(ss);
  const float inv = n > 1e-12f ? 1.0f / n : 0.0f;
  const float u[4] = {x.x * inv, x.y * inv, x.z * inv, x.w * inv};
  float r[4];
#pragma unroll
  for (int p = 0; p < 2; ++p) {  // pairs 2 lane + p: coordinates 4 lane + 2p, +1
    const float c = s_gc[2 * lane + p], s = s_gs[2 * lane + p];
    const float a = u[2 * p], b = u[2 * p + 1];
    r[2 * p] = c * a - s * b;
    r[2 * p + 1] = s * a + c * b;
  }
  const int nc = 1 << bits;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int best = 0;
    float bd = fabsf(r[i] - s_c[0]);
    for (int k = 1; k < nc; ++k) {
      const float dk = fabsf(r[i] - s_c[k]);
      if (dk < bd) {
        bd = dk;
        best = k;
      }
    }
    s_idx[4 * lane + i] = static_cast<uint8_t>(best);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // LSB-first packing: byte j holds bits [8 j, 8 j + 8) of the index string
  const int nbytes = 32 * bits;
  for (int j = lane; j < nbytes; j += 64) {
    uint32_t v = 0;
    const int b0 = 8 * j;
    for (int i = b0 / bits; i * bits < b0 + 8; ++i) {
      const int sh = i * bits - b0;
      const uint32_t ix = s_idx[i];
      v |= sh >= 0 ? ix << sh : ix >> (-sh);
    }
    packed[j] = static_cast<uint8_t>(v & 0xffu);
  }
  if (lane == 0) *norm = n;
}

__global__ __launch_bounds__(64 * kRowsPerBlock) void kv_planar_store_kernel(
    const float *k, const float *v, size_t rows, int bits, uint8_t *kq, float *kn, uint8_t *vq,
    float *vn, float *v_f32, size_t row0, PlanarTables tb) {
  __shared__ float s_c[256], s_gc[kPlanarHd / 2], s_gs[kPlanarHd / 2];
  __shared__ float s_sq[kRowsPerBlock][kPlanarHd];
  __shared__ uint8_t s_idx[kRowsPerBlock][kPlanarHd];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  s_c[tid] = tb.cent[tid];
  if (tid < kPlanarHd / 2) {
    s_gc[tid] = tb.gc[tid];
    s_gs[tid] = tb.gs[tid];
  }
  __syncthreads();
  const size_t row = static_cast<size_t>(blockIdx.x) * kRowsPerBlock + w;
  if (row >= rows) return;
  const size_t plen = static_cast<size_t>(32 * bits);
  const size_t dst = row0 + row;
  const float4 xk = reinterpret_cast<const float4 *>(k + row * kPlanarHd)[lane];
  const float4 xv = reinterpret_cast<const float4 *>(v + row * kPlanarHd)[lane];
  planar_quantize_wave(xk, bits, s_c, s_gc, s_gs, s_sq[w], s_idx[w], kq + dst * plen, kn + dst);
  if (vq != nullptr) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // the K pass's LDS reads are done
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    planar_quantize_wave(xv, bits, s_c, s_gc, s_gs, s_sq[w], s_idx[w], vq + dst * plen, vn + dst);
  } else {
    reinterpret_cast<float4 *>(v_f32 + dst * kPlanarHd)[lane] = xv;  // append_v: f32 rows
  }
}

}  // namespace
}  // namespace bh

using namespace bh;

extern "C" size_t bh_planar_packed_len(size_t hd, unsigned bits) { return planar_packed_len(hd, bits); }

extern "C" int bh_kv_store_planar(const float *k, const float *v, size_t n_tok, size_t n_kv,
                                  size_t hd, unsigned bits, uint8_t *kq, float *kn, uint8_t *vq,
                                  float *vn, float *v_f32, size_t pos0, bh_stream stream) {
  if (bits < 1 || bits > 8) return fail(BH_ERR_ARG, "kv_store_planar: bits must be 1..8");
  if (hd != static_cast<size_t>(kPlanarHd))
    return fail(BH_ERR_SHAPE, "kv_store_planar: head_dim must be 256 (got " + std::to_string(hd) + ")");
  if ((vq == nullptr) != (vn == nullptr))
    return fail(BH_ERR_ARG, "kv_store_planar: vq and vn go together (quantized V) or are both null");
  size_t rows = 0;
  if (!mul_size(n_tok, n_kv, &rows) || rows > 0x7fffffffu * size_t{kRowsPerBlock})
    return fail(BH_ERR_SHAPE, "kv_store_planar: too many rows");
  if (rows == 0) return ok();
  if (!k || !v || !kq || !kn || (vq == nullptr && v_f32 == nullptr))
    return fail(BH_ERR_ARG, "kv_store_planar: null pointer");
  if (!aligned16(k) || !aligned16(v) || (vq == nullptr && !aligned16(v_f32)))
    return fail(BH_ERR_ARG, "kv_store_planar: k, v and v_f32 must be 16-byte aligned");
  size_t row0 = 0;
  if (!mul_size(pos0, n_kv, &row0)) return fail(BH_ERR_SHAPE, "kv_store_planar: position overflows");
  PlanarTables tb;
  if (!planar_tables(hd, bits, &tb)) return fail(BH_ERR_ARG, "kv_store_planar: no tables");
  const unsigned grid = static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock);
  BH_LAUNCH(kv_planar_store_kernel, grid, 64 * kRowsPerBlock, 0, as_stream(stream), k, v, rows,
            static_cast<int>(bits), kq, kn, vq, vn, v_f32, row0, tb);
  return ok();
}
