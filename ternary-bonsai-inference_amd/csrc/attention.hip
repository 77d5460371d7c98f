// Grouped-query attention over a KV cache, and the cache append.
//
// Reference: full_attention_layer, src/forward.rs:273-375 (one token per
// call): the token's k/v rows are appended at position pos (:273-287,
// AttnCache::append / append_f16 :90-95, 120-125); then for every q head hq
// (kv head hq / (n_head / n_kv)): scores[j] = dot(q, k_j) * (1 / sqrtf(hd))
// over the pos + 1 cached positions (dot / dot_f16 :181-191), probs =
// softmax_rows(scores) (:326), out[d] = sum_j probs[j] * v_j[d], skipping
// probs[j] == 0 (:361-371, f16 cache :349-360).
//
// bh_attention takes n_q query tokens at positions pos0 .. pos0 + n_q - 1
// (query i sees positions 0 .. pos0 + i, as the reference's token loop).
//
// Decode path (hd = 256, n_head / n_kv in {1, 2, 3, 4, 6, 8}): the
// positions of one (query, kv head) are split into chunks, one block each.
// A block keeps the q slices of the kv head's REP q heads in registers and
// runs 64-position tiles: scores with 16 lanes per position (16 dims per
// lane, DPP row sums) into LDS, the tile's max and exponentials once per
// tile (running max and sum per head, the accumulators rescaled once per
// tile), then P.V with each lane owning 4 output dims of every head and the
// four waves taking every fourth position, so K and V are each read once.
// A second launch merges the chunks' (max, sum, acc) triples.  Results are
// the reference's up to rounding (sums in another order); a non-finite v at
// a position whose probability underflows to 0 is not skipped here.
//
// Many queries per kv head (prefill, verification; hd = 256): the
// matrix-core path (mq_body: f16 hi / lo products with power-of-two
// scaling, one block per (position chunk, 128-row tile, kv head)); over an
// f32 cache read by 8 or more row tiles per kv head the cache is first
// split into f16 hi / lo once (attn_kv_split_kernel) instead of per block.
//
// Generic path (any hd and grouping, any alignment): one block per (query,
// head) computes the scores, the reference's softmax (f32 max, expf, f64
// sum, inv = 1 / (f32)sum, p = e * inv) into scratch; a second launch forms
// P.V in position order, skipping p == 0 -- the reference's sequence, with
// only the f64 sum reduced as a tree.
#include <hip/hip_runtime.h>

#include <cmath>
#include <mutex>
#include <string>
#include <type_traits>

#include "common.hpp"
#include "kvquant.hpp"

namespace bh {
namespace {

constexpr int kBlock = 256;
constexpr int kHd = 256;        // head size of the decode path
constexpr int kTile = 64;       // positions per tile
constexpr int kQkLanes = 16;    // lanes per position in the score pass
constexpr int kQkPer = kHd / kQkLanes;  // 16 dims per lane

// gguf::f32_to_half (src/gguf.rs:914-944) in integer arithmetic: NaN keeps
// only a quiet bit, overflow goes to inf, the subnormal range shifts the
// mantissa before rounding to nearest even on the 13 dropped bits.
__device__ __forceinline__ uint32_t f32_to_half_bits(float v) {
  const uint32_t b = __float_as_uint(v);
  const uint32_t sign = (b >> 16) & 0x8000u;
  const int exp = static_cast<int>((b >> 23) & 0xffu);
  const uint32_t man = b & 0x7fffffu;
  if (exp == 0xff) return sign | 0x7c00u | (man != 0u ? 0x200u : 0u);
  const int e = exp - 127 + 15;
  if (e >= 0x1f) return sign | 0x7c00u;
  uint32_t half, rem;
  if (e <= 0) {
    if (e < -10) return sign;
    const uint32_t m = (man | 0x800000u) >> (1 - e);
    half = m >> 13;
    rem = m & 0x1fffu;
  } else {
    half = (static_cast<uint32_t>(e) << 10) | (man >> 13);
    rem = man & 0x1fffu;
  }
  const uint32_t up = (rem > 0x1000u || (rem == 0x1000u && (half & 1u) != 0u)) ? 1u : 0u;
  return sign | ((half + up) & 0xffffu);
}

__device__ __forceinline__ float half_to_float(uint32_t h) {
  return __uint_as_float(half_bits_to_f32_bits(h));
}

// Cache element access for the two storage types.
template <class T>
struct Kv;

template <>
struct Kv<float> {
  static __device__ __forceinline__ float at(const float *c, size_t e) { return c[e]; }
  // 4 values at e (a multiple of 4)
  static __device__ __forceinline__ f32x4 load4(const float *c, size_t e) {
    return *reinterpret_cast<const f32x4 *>(c + e);
  }
};

template <>
struct Kv<uint16_t> {
  static __device__ __forceinline__ float at(const uint16_t *c, size_t e) {
    return half_to_float(c[e]);
  }
  // the hardware widening (v_cvt_f32_f16): exact for every finite f16 and
  // the infinities, as the reference's half_to_f32; only a NaN's payload may
  // differ, and a NaN score or value propagates as NaN either way
  static __device__ __forceinline__ f32x4 load4(const uint16_t *c, size_t e) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 h = *reinterpret_cast<const h4 *>(c + e);
    return f32x4{static_cast<float>(h.x), static_cast<float>(h.y), static_cast<float>(h.z),
                 static_cast<float>(h.w)};
  }
};

// ---- KV append -------------------------------------------------------------

template <class T>
__global__ __launch_bounds__(kBlock) void kv_store_kernel(const float *k, const float *v,
                                                          size_t n, T *kc, T *vc) {
  const size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= n) return;
  if constexpr (sizeof(T) == 2) {
    kc[i] = static_cast<T>(f32_to_half_bits(k[i]));
    vc[i] = static_cast<T>(f32_to_half_bits(v[i]));
  } else {
    kc[i] = k[i];
    vc[i] = v[i];
  }
}

// ---- decode path -----------------------------------------------------------

struct DecodeArgs {
  const float *q;
  const void *kc, *vc;
  float *pm, *pl, *pacc;  // chunk partials [n_q][n_head][n_chunks] (+ [hd])
  size_t pos0, kv_stride, chunk;
  int n_head, n_chunks;
  float scale;
  int tile;  // positions per tile: 64, or 32 when 64-position tiles leave the chip short of blocks
};

template <int L>
__device__ __forceinline__ float dpp_row(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), L, 0xF, 0xF, false));
}

// Sum over the 16 lanes of a DPP row; every lane gets the same bits.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp_row<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp_row<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp_row<0x141>(x);  // row_half_mirror
  x += dpp_row<0x140>(x);  // row_mirror
  return x;
}

// max over the four lanes l % 16 + 16 g (one row): permlane swaps
__device__ __forceinline__ float rows4_max(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float rows4_sum(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

struct FMaxOp {
  __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
__device__ __forceinline__ float wave_max(float x) { return lane_group_reduce<64>(x, FMaxOp{}); }
__device__ __forceinline__ float wave_sum(float x) { return lane_group_sum<64>(x); }

template <int REP, class T, int TILE>
__global__ __launch_bounds__(kBlock) void attn_decode_kernel(DecodeArgs a) {
  static_assert(TILE == 32 || TILE == 64, "tiles of 32 or 64 positions");
  constexpr int kPasses = TILE / 16;
  constexpr int kWj = kPasses * 4;  // positions of a wave per tile
  static_assert(REP <= 16, "one head per lane of a 16-lane group");
  __shared__ float s_e[4][kWj][REP];  // per wave: P.V weights of its positions
  __shared__ float s_wm[4][REP], s_wl[4][REP], s_ww[4][REP];
  __shared__ float s_acc[4][REP][kHd];
  __shared__ f32x4 s_q[REP * kHd / 4];
  const T *kc = static_cast<const T *>(a.kc);
  const T *vc = static_cast<const T *>(a.vc);
  const int c = blockIdx.x, g = blockIdx.y, i = blockIdx.z;
  const int tid = threadIdx.x, w = tid / 64, lane = tid % 64;
  const size_t n_pos = a.pos0 + i + 1;
  const size_t beg = static_cast<size_t>(c) * a.chunk;
  const size_t end = beg + a.chunk < n_pos ? beg + a.chunk : n_pos;
  const size_t part0 = (static_cast<size_t>(i) * a.n_head + static_cast<size_t>(g) * REP) *
                       a.n_chunks + c;  // + r * n_chunks
  if (beg >= end) {  // this query has no positions in the chunk
    if (tid < REP) {
      a.pm[part0 + static_cast<size_t>(tid) * a.n_chunks] = -INFINITY;
      a.pl[part0 + static_cast<size_t>(tid) * a.n_chunks] = 0.0f;
    }
    for (int o = tid; o < REP * kHd; o += kBlock)
      a.pacc[(part0 + static_cast<size_t>(o / kHd) * a.n_chunks) * kHd + o % kHd] = 0.0f;
    return;
  }
  const int grp = tid / kQkLanes, sub = tid % kQkLanes;
  const int grp4 = lane / kQkLanes;  // the lane's group within its wave
  // the group's q rows go to LDS (REP x 256 floats, the kv head's q heads
  // are consecutive), so registers go to the K and V tiles.  They are loaded
  // here and stored to LDS only after the first tile's K (and V) loads are
  // issued: the tile's loads do not wait for q's round trip.
  constexpr int kQ4 = REP * kHd / 4;
  constexpr int kQPer = (kQ4 + kBlock - 1) / kBlock;
  f32x4 qreg[kQPer];
  {
    const f32x4 *qg = reinterpret_cast<const f32x4 *>(
        a.q + (static_cast<size_t>(i) * a.n_head + g * REP) * kHd);
#pragma unroll
    for (int u = 0; u < kQPer; ++u) {
      const int o = tid + u * kBlock;
      qreg[u] = qg[o < kQ4 ? o : kQ4 - 1];
    }
  }
  // Each wave runs its own online softmax over the positions it scores
  // (pass * 16 + 4 w + g, g its lane group): after a pass's DPP row sums
  // every lane of a group holds the group's REP scores, lane sub keeps head
  // sub's, the wave's per-head max is two permlane swaps away, and head
  // sub's running max and sum live in lane sub.  No block barrier inside the
  // chunk loop but the q stage's; the four waves merge once per chunk.
  float run_m = -INFINITY, run_l = 0.0f;
  float acc[REP][4];
#pragma unroll
  for (int r = 0; r < REP; ++r)
#pragma unroll
    for (int x = 0; x < 4; ++x) acc[r][x] = 0.0f;
  const size_t head_off = static_cast<size_t>(g) * kHd;

  for (size_t t0 = beg; t0 < end; t0 += TILE) {
    // scores: 16 lanes per position, 4 passes of 16 positions
    f32x4 kr[kPasses][kQkPer / 4];
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
      const size_t p = t0 + pass * 16 + grp;
      const size_t e0 = (p < end ? p : end - 1) * a.kv_stride + head_off + kQkPer * sub;
#pragma unroll
      for (int x = 0; x < kQkPer / 4; ++x) kr[pass][x] = Kv<T>::load4(kc, e0 + 4 * x);
    }
    if (t0 == beg) {
#pragma unroll
      for (int u = 0; u < kQPer; ++u) {
        const int o = tid + u * kBlock;
        if (o < kQ4) s_q[o] = qreg[u];
      }
    }
    if (t0 == beg) __syncthreads();  // s_q written, while the K rows are in flight
    float sc[kPasses];  // head sub's score of the group's position, per pass
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) sc[pass] = -INFINITY;
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      f32x4 qv[kQkPer / 4];  // head r's 16 dims of this lane, read once per tile
#pragma unroll
      for (int x = 0; x < kQkPer / 4; ++x) qv[x] = s_q[(r * kHd + kQkPer * sub) / 4 + x];
#pragma unroll
      for (int pass = 0; pass < kPasses; ++pass) {
        const size_t p = t0 + pass * 16 + grp;
        // fused multiply-adds, two chains of 8 dims (the library builds
        // with contraction off, so a * b + c would cost two instructions)
        float part[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const f32x4 k0 = kr[pass][2 * h], k1 = kr[pass][2 * h + 1];
          const f32x4 q0 = qv[2 * h], q1 = qv[2 * h + 1];
          float s = q0.x * k0.x;
          s = fmaf(q0.y, k0.y, s);
          s = fmaf(q0.z, k0.z, s);
          s = fmaf(q0.w, k0.w, s);
          s = fmaf(q1.x, k1.x, s);
          s = fmaf(q1.y, k1.y, s);
          s = fmaf(q1.z, k1.z, s);
          part[h] = fmaf(q1.w, k1.w, s);
        }
        const float d = row16_sum(part[0] + part[1]);
        if (sub == r) sc[pass] = p < end ? d * a.scale : -INFINITY;
      }
    }
    // the wave's V rows of the tile: issued now (the K registers are free) so
    // their latency overlaps the softmax step and its barriers (issued with
    // the K rows instead, one round trip per tile, they measured slower:
    // ctx 4096 14.0 -> 15.7 us, ctx 32768 55 -> 60 us)
    const int nt = static_cast<int>(end - t0 < static_cast<size_t>(TILE) ? end - t0 : TILE);
    f32x4 vr[kWj];  // the wave's positions (jl >> 2) * 16 + 4 w + (jl & 3)
#pragma unroll
    for (int jl = 0; jl < kWj; ++jl) {
      const int j = min((jl >> 2) * 16 + 4 * w + (jl & 3), nt - 1);
      vr[jl] = Kv<T>::load4(vc, (t0 + j) * a.kv_stride + head_off + 4 * lane);
    }
    // head sub's max over the wave's positions (the four groups)
    float tm = sc[0];
#pragma unroll
    for (int pass = 1; pass < kPasses; ++pass) tm = fmaxf(tm, sc[pass]);
    const float hm = fmaxf(run_m, rows4_max(tm));
    const float corr_mine = hm == -INFINITY ? 1.0f : expf(run_m - hm);
    run_m = hm;
    float ps = 0.0f;
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
      const float e = hm == -INFINITY ? 0.0f : expf(sc[pass] - hm);
      ps += e;
      if (sub < REP) s_e[w][4 * pass + grp4][sub] = e;
    }
    run_l = run_l * corr_mine + rows4_sum(ps);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // P.V: lane owns dims 4*lane .. +3 of the wave's positions
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      const float cr = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(corr_mine), r));
#pragma unroll
      for (int x = 0; x < 4; ++x) acc[r][x] *= cr;
    }
#pragma unroll
    for (int jl = 0; jl < kWj; ++jl) {
      if ((jl >> 2) * 16 + 4 * w + (jl & 3) < nt) {
        const f32x4 v = vr[jl];
#pragma unroll
        for (int r = 0; r < REP; ++r) {
          const float e = s_e[w][jl][r];
          acc[r][0] = fmaf(e, v.x, acc[r][0]);
          acc[r][1] = fmaf(e, v.y, acc[r][1]);
          acc[r][2] = fmaf(e, v.z, acc[r][2]);
          acc[r][3] = fmaf(e, v.w, acc[r][3]);
        }
      }
    }
    // the weights are consumed before the next tile writes them
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // merge the four waves: weights e^(m_w - M) per head
#pragma unroll
  for (int r = 0; r < REP; ++r)
#pragma unroll
    for (int x = 0; x < 4; ++x) s_acc[w][r][4 * lane + x] = acc[r][x];
  if (lane < REP) {
    s_wm[w][lane] = run_m;
    s_wl[w][lane] = run_l;
  }
  __syncthreads();
  if (tid < REP) {
    const int r = tid;
    const float big = fmaxf(fmaxf(s_wm[0][r], s_wm[1][r]), fmaxf(s_wm[2][r], s_wm[3][r]));
    float l = 0.0f;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const float wt = s_wm[ww][r] == -INFINITY ? 0.0f : expf(s_wm[ww][r] - big);
      s_ww[ww][r] = wt;
      l += s_wl[ww][r] * wt;
    }
    a.pm[part0 + static_cast<size_t>(r) * a.n_chunks] = big;
    a.pl[part0 + static_cast<size_t>(r) * a.n_chunks] = l;
  }
  __syncthreads();
  for (int o = tid; o < REP * kHd; o += kBlock) {
    const int r = o / kHd, d = o % kHd;
    const float sum = (s_acc[0][r][d] * s_ww[0][r] + s_acc[1][r][d] * s_ww[1][r]) +
                      (s_acc[2][r][d] * s_ww[2][r] + s_acc[3][r][d] * s_ww[3][r]);
    a.pacc[(part0 + static_cast<size_t>(r) * a.n_chunks) * kHd + d] = sum;
  }
}

// out[i][h][d] = sum_c acc_c[d] e^(m_c - M) / sum_c l_c e^(m_c - M), chunks
// with m_c = -inf left out.  Block (h, i, z) of kCombWaves waves (16; more than 128
// chunks, the single-round-trip form below takes fewer) writes dims
// 64z .. 64z + 63 of row (i, h): the chunk weights e^(m_c - M) are computed
// once per block into LDS (in tiles of kCombTile chunks), wave w takes
// chunks w, w + kCombWaves, ... with one lane per dim (loads unconditional,
// so eight are in flight per lane), and the waves' sums are added in wave
// order.  Every block of a row computes M and the denominator the same way.
constexpr int kCombDims = 64;
constexpr int kCombTile = 2048;
template <int kCombWaves>
__global__ __launch_bounds__(64 * kCombWaves) void attn_combine_kernel(const float *pm,
                                                                    const float *pl,
                                                                    const float *pacc,
                                                                    int n_chunks, int hd,
                                                                    float *out) {
  __shared__ float s_w[kCombTile];
  __shared__ float s_red[kCombWaves][kCombDims];
  __shared__ float s_m[kCombWaves];
  __shared__ float s_l[kCombWaves];
  constexpr int kCombThreads = 64 * kCombWaves;
  const size_t row = static_cast<size_t>(blockIdx.y) * gridDim.x + blockIdx.x;  // i * n_head + h
  const int tid = threadIdx.x, w = tid / 64, lane = tid % 64;
  const float *m = pm + row * n_chunks;
  const float *l = pl + row * n_chunks;
  float big = -INFINITY;
  for (int c = tid; c < n_chunks; c += kCombThreads) big = fmaxf(big, m[c]);
  big = wave_max(big);
  if (lane == 0) s_m[w] = big;
  __syncthreads();
  big = s_m[0];
  for (int i = 1; i < kCombWaves; ++i) big = fmaxf(big, s_m[i]);
  float den = 0.0f;
  for (int c = tid; c < n_chunks; c += kCombThreads)
    if (m[c] != -INFINITY) den += l[c] * expf(m[c] - big);
  den = wave_sum(den);
  if (lane == 0) s_l[w] = den;
  const int d = static_cast<int>(blockIdx.z) * kCombDims + (lane < hd ? lane : 0);
  const float *acc = pacc + row * n_chunks * static_cast<size_t>(hd) + d;
  float num = 0.0f;
  for (int c0 = 0; c0 < n_chunks; c0 += kCombTile) {
    const int cn = n_chunks - c0 < kCombTile ? n_chunks - c0 : kCombTile;
    __syncthreads();  // previous tile's weights consumed (first pass: s_l visible)
    for (int c = tid; c < cn; c += kCombThreads)
      s_w[c] = m[c0 + c] != -INFINITY ? expf(m[c0 + c] - big) : -1.0f;  // -1: left out
    __syncthreads();
#pragma unroll 8
    for (int c = w; c < cn; c += kCombWaves) {
      const float a = acc[static_cast<size_t>(c0 + c) * hd];
      const float wc = s_w[c];
      num += wc != -1.0f ? a * wc : 0.0f;
    }
  }
  s_red[w][lane] = num;
  __syncthreads();
  const int dd = static_cast<int>(blockIdx.z) * kCombDims + lane;
  if (w == 0 && dd < hd) {
    float dsum = s_l[0], nsum = s_red[0][lane];
    for (int i = 1; i < kCombWaves; ++i) {
      dsum += s_l[i];
      nsum += s_red[i][lane];
    }
    out[row * hd + dd] = nsum * (1.0f / dsum);
  }
}

// The same merge for at most kCombWaves * kCombPer chunks in one round trip:
// every load of the block is issued first -- wave w's accumulators of chunks
// w, w + kCombWaves, ... (kCombPer per lane, one lane per dim) and thread c's
// (max, sum) of chunk c -- then the block's max, the chunk weights (LDS) and
// the weighted sum are formed from registers.  The general kernel above
// waits for the maxima, then the sums, then the accumulators.
// ROT (planar-quantized V, whose sums are formed in rotated space): the
// merged row is turned back by the inverse Givens rotation of each pair
// (2i, 2i+1) -- [c a + s b, -s a + c b] (src/kvquant.rs:425-436) -- the
// partner dimension coming from the neighbouring lane.
template <int kCombWaves, int kCombPer, bool ROT>
__device__ __forceinline__ void combine1_body(const float *pm, const float *pl, const float *pacc,
                                              int n_chunks, float *out, const float *gc,
                                              const float *gs) {
  constexpr int kMax = kCombWaves * kCombPer;
  static_assert(kMax <= 64 * kCombWaves, "one (max, sum) pair per thread");
  __shared__ float s_w[kMax];
  __shared__ float s_red[kCombWaves][kCombDims];
  __shared__ float s_m[kCombWaves];
  __shared__ float s_l[kCombWaves];
  const size_t row = static_cast<size_t>(blockIdx.y) * gridDim.x + blockIdx.x;  // i * n_head + h
  const int tid = threadIdx.x, w = tid / 64, lane = tid % 64;
  const float *acc = pacc + row * n_chunks * static_cast<size_t>(kHd) + blockIdx.z * kCombDims + lane;
  float av[kCombPer];
#pragma unroll
  for (int k = 0; k < kCombPer; ++k) {
    const int c = w + kCombWaves * k;
    av[k] = acc[static_cast<size_t>(c < n_chunks ? c : n_chunks - 1) * kHd];
  }
  const float mc = tid < n_chunks ? pm[row * n_chunks + tid] : -INFINITY;
  const float lc = tid < n_chunks ? pl[row * n_chunks + tid] : 0.0f;
  float big = wave_max(mc);
  if (lane == 0) s_m[w] = big;
  __syncthreads();
  big = s_m[0];
#pragma unroll
  for (int i = 1; i < kCombWaves; ++i) big = fmaxf(big, s_m[i]);
  const float wc = mc != -INFINITY ? expf(mc - big) : -1.0f;  // -1: left out
  if (tid < kMax) s_w[tid] = wc;
  const float den = wave_sum(wc != -1.0f ? lc * wc : 0.0f);
  if (lane == 0) s_l[w] = den;
  __syncthreads();
  float num = 0.0f;
#pragma unroll
  for (int k = 0; k < kCombPer; ++k) {
    const int c = w + kCombWaves * k;
    const float wk = c < n_chunks ? s_w[c] : -1.0f;
    num += wk != -1.0f ? av[k] * wk : 0.0f;
  }
  s_red[w][lane] = num;
  __syncthreads();
  if (w == 0) {
    float dsum = s_l[0], nsum = s_red[0][lane];
#pragma unroll
    for (int i = 1; i < kCombWaves; ++i) {
      dsum += s_l[i];
      nsum += s_red[i][lane];
    }
    const float val = nsum * (1.0f / dsum);
    const int d = static_cast<int>(blockIdx.z) * kCombDims + lane;
    if constexpr (ROT) {
      const float other = __shfl_xor(val, 1, 64);
      const float c = gc[d >> 1], sn = gs[d >> 1];
      out[row * kHd + d] = (d & 1) == 0 ? c * val + sn * other : -sn * other + c * val;
    } else {
      out[row * kHd + d] = val;
    }
  }
}

template <int kCombWaves, int kCombPer>
__global__ __launch_bounds__(64 * kCombWaves) void attn_combine1_kernel(const float *pm,
                                                                     const float *pl,
                                                                     const float *pacc,
                                                                     int n_chunks, float *out) {
  combine1_body<kCombWaves, kCombPer, false>(pm, pl, pacc, n_chunks, out, nullptr, nullptr);
}

template <int kCombWaves, int kCombPer>
__global__ __launch_bounds__(64 * kCombWaves) void attn_combine1_rot_kernel(
    const float *pm, const float *pl, const float *pacc, int n_chunks, float *out, PlanarTables tb) {
  combine1_body<kCombWaves, kCombPer, true>(pm, pl, pacc, n_chunks, out, tb.gc, tb.gs);
}

// ---- planar-quantized caches (src/forward.rs:296-349, src/kvquant.rs) -------
//
// K (and V, unless the cache keeps V in f32: BONSAI_KV=planarNk) hold per
// (position, kv head) a norm and 256 packed centroid indices of the rotated
// unit vector (kvquant.hip).  Block (chunk, kv head, query) of 256 lanes,
// the f32 decode kernel's layout: the REP q rows of the kv head are rotated
// once into LDS (the reference rotates q and dots it against centroids,
// src/kvquant.rs:444-460); per tile of 64 positions a score is 16 lanes x 16
// coordinates: each lane reads its 2 BITS bytes of the packed row straight
// from memory (16 lanes read a row's 32 BITS contiguous bytes), looks the 16
// centroids up in LDS and dots them with q_rot (DPP row sums), times the
// norm and 1/sqrt(hd).  The running (max, sum) per head and the P.V
// accumulation follow the f32 decode kernel, the quantized V term being
// (e_j |v_j|) * centroid: lane l owns dims 4l .. 4l+3, whose 4 BITS index
// bits it reads from one or two dwords.  Chunks merge in
// attn_combine1_rot_kernel, which also applies the inverse rotation (a V
// cache in f32 merges plainly).
constexpr int kPlTile = 64;

struct PlanarArgs {
  const float *q;
  const uint8_t *kq;
  const float *kn;
  const uint8_t *vq;  // null: V in f32 (vf)
  const float *vn;
  const float *vf;
  float *pm, *pl, *pacc;
  size_t pos0, chunk;
  int n_head, n_chunks, n_kv, bits;
  float scale;
};

// One tile's global data of a lane, held in registers: the K words and
// norms of the four positions its 16-lane group scores (one per pass), the
// V norms of the same positions, and the V index bits (one or two dwords)
// of the wave's 16 positions for the lane's 4 dims -- or, V in f32, the f32
// dims.  The wave's positions of a tile are pass * 16 + 4 w + g (g the
// lane's group, pass 0..3): local index jl = 4 pass + g.
template <int BITS, bool VQ>
struct PlanarTile {
  static constexpr int kPasses = kPlTile / 16;
  static constexpr bool kDw = BITS % 2 == 0;  // whole dwords (even BITS) or halfwords
  static constexpr int kWords = kDw ? BITS / 2 : BITS;
  static constexpr int kVj = kPlTile / 4;
  // 4 BITS index bits at bit 4 lane BITS straddle a dword boundary for
  // some lanes unless BITS divides 8
  static constexpr bool kTwo = 8 % BITS != 0;
  uint32_t kw[kPasses][kWords];
  float kn[kPasses];
  float vn[VQ ? kPasses : 1];
  uint32_t vlo[VQ ? kVj : 1], vhi[VQ && kTwo ? kVj : 1];
  float4 vr[VQ ? 1 : kVj];

  // addresses: the tile's first row once (uniform), then 32-bit offsets of
  // whole positions (64-bit products per row cost ~250 VALU per tile)
  // K words and norms (and V norms) of the group's positions
  __device__ __forceinline__ void load_k(const PlanarArgs &a, size_t t0, int nt, int g, int w,
                                         int grp4, int sub) {
    constexpr int kPlen = 32 * BITS;
    const uint32_t nkv = static_cast<uint32_t>(a.n_kv);
    const uint32_t pstride = nkv * kPlen;  // bytes from one position to the next
    const size_t r0 = t0 * a.n_kv + g;
    const uint8_t *kb = a.kq + r0 * kPlen + 2 * BITS * sub;
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
      const uint32_t p = static_cast<uint32_t>(min(pass * 16 + 4 * w + grp4, nt - 1));
      const uint8_t *src = kb + p * pstride;
#pragma unroll
      for (int h = 0; h < kWords; ++h)
        kw[pass][h] = kDw ? reinterpret_cast<const uint32_t *>(src)[h]
                          : static_cast<uint32_t>(reinterpret_cast<const uint16_t *>(src)[h]);
      kn[pass] = a.kn[r0 + p * nkv];
      if constexpr (VQ) vn[pass] = a.vn[r0 + p * nkv];
    }
  }
  // V index bits (or f32 dims) of the wave's 16 positions
  __device__ __forceinline__ void load_v(const PlanarArgs &a, size_t t0, int nt, int g, int w,
                                         int lane, int vdw, bool two) {
    constexpr int kPlen = 32 * BITS;
    const uint32_t nkv = static_cast<uint32_t>(a.n_kv);
    const uint32_t pstride = nkv * kPlen;
    const size_t r0 = t0 * a.n_kv + g;
    if constexpr (VQ) {
      const uint8_t *vb = a.vq + r0 * kPlen + 4 * vdw;
#pragma unroll
      for (int jl = 0; jl < kVj; ++jl) {
        const uint32_t j = static_cast<uint32_t>(min((jl >> 2) * 16 + 4 * w + (jl & 3), nt - 1));
        const uint32_t *src = reinterpret_cast<const uint32_t *>(vb + j * pstride);
        vlo[jl] = src[0];
        if constexpr (kTwo) vhi[jl] = two ? src[1] : 0u;
      }
    } else {
      const float *vfb = a.vf + r0 * kPlanarHd + 4 * lane;
      const uint32_t vstride = nkv * kPlanarHd;  // floats
#pragma unroll
      for (int jl = 0; jl < kVj; ++jl) {
        const uint32_t j = static_cast<uint32_t>(min((jl >> 2) * 16 + 4 * w + (jl & 3), nt - 1));
        vr[jl] = *reinterpret_cast<const float4 *>(vfb + j * vstride);
      }
    }
  }
};

// x[i] for a per-lane i as a chain of selects.  Each value goes through an
// empty asm statement first: otherwise the compiler turns the chain back
// into an indexed load and puts the array in scratch memory.
template <int N>
__device__ __forceinline__ float pick(const float (&x)[N], int i) {
  float v = x[0];
#pragma unroll
  for (int r = 1; r < N; ++r) {
    float xr = x[r];
    asm volatile("" : "+v"(xr));
    v = i == r ? xr : v;
  }
  return v;
}

// Each wave runs its own online softmax over the positions it scores (no
// block barrier inside the chunk loop): after a pass's DPP row sums every
// lane of a 16-lane group holds all REP scores of the group's position, so
// the wave's per-head tile max is two permlane swaps away; lane sub < REP
// forms head sub's weight of its position, writes it (times |v_j| for a
// quantized V) to the wave's own LDS slice and keeps head sub's running sum;
// P.V then reads the weights back as broadcasts.  The four waves' (max,
// sum, accumulator) states merge once per chunk.
template <int REP, int BITS, bool VQ>
__global__ __launch_bounds__(kBlock) void attn_planar_kernel(PlanarArgs a, PlanarTables tb) {
  using Tile = PlanarTile<BITS, VQ>;
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  constexpr int kPasses = Tile::kPasses;
  constexpr int kVj = Tile::kVj;
  static_assert(REP <= 16, "one head per lane of a 16-lane group");
  static_assert(kPasses == 4, "the tile max below reads four passes");
  // 2- and 4-bit indices are looked up a byte at a time: entry b of s_cb
  // holds the centroids of the kE indices packed in byte b, in bit order
  constexpr bool kByteTab = BITS == 2 || BITS == 4;
  constexpr int kE = kByteTab ? 8 / BITS : 1;
  using CVec = typename std::conditional<kE == 4, float4, float2>::type;
  __shared__ __attribute__((aligned(16))) CVec s_cb[kByteTab ? 256 : 1];
  __shared__ float s_c[256];
  __shared__ float s_q[REP][kPlanarHd];
  __shared__ float s_e[4][kVj][REP];  // per wave: weights of its 16 positions
  __shared__ float s_wm[4][REP], s_wl[4][REP], s_ww[4][REP];
  __shared__ float s_acc[4][REP][kPlanarHd];
  const int c = blockIdx.x, g = blockIdx.y, i = blockIdx.z;
  const int tid = threadIdx.x, w = tid / 64, lane = tid % 64;
  const size_t n_pos = a.pos0 + i + 1;
  const size_t beg = static_cast<size_t>(c) * a.chunk;
  const size_t end = beg + a.chunk < n_pos ? beg + a.chunk : n_pos;
  const size_t part0 = (static_cast<size_t>(i) * a.n_head + static_cast<size_t>(g) * REP) * a.n_chunks + c;
  if (beg >= end) {  // this query has no positions in the chunk
    if (tid < REP) {
      a.pm[part0 + static_cast<size_t>(tid) * a.n_chunks] = -INFINITY;
      a.pl[part0 + static_cast<size_t>(tid) * a.n_chunks] = 0.0f;
    }
    for (int o = tid; o < REP * kHd; o += kBlock)
      a.pacc[(part0 + static_cast<size_t>(o / kHd) * a.n_chunks) * kHd + o % kHd] = 0.0f;
    return;
  }
  const int grp4 = lane / kQkLanes, sub = lane % kQkLanes;  // group within the wave, lane in it
  const int vbit = 4 * lane * BITS, vdw = vbit >> 5, vsh = vbit & 31;
  const bool two = vsh + 4 * BITS > 32;
  auto tile_len = [&](size_t t0) {
    return static_cast<int>(end - t0 < static_cast<size_t>(kPlTile) ? end - t0 : kPlTile);
  };
  Tile nxt;
  nxt.load_k(a, beg, tile_len(beg), g, w, grp4, sub);
  nxt.load_v(a, beg, tile_len(beg), g, w, lane, vdw, two);
  s_c[tid] = tb.cent[tid];
  if constexpr (kByteTab) {
    float ce[kE];
#pragma unroll
    for (int e = 0; e < kE; ++e) ce[e] = tb.cent[(tid >> (e * BITS)) & kMask];
    if constexpr (kE == 4)
      s_cb[tid] = CVec{ce[0], ce[1], ce[2], ce[3]};
    else
      s_cb[tid] = CVec{ce[0], ce[kE - 1]};
  }
  // q rows of the kv head's REP heads, rotated: pair p of head r
  for (int o = tid; o < REP * kPlanarHd / 2; o += kBlock) {
    const int r = o / (kPlanarHd / 2), pp = o % (kPlanarHd / 2);
    const float2 qa = reinterpret_cast<const float2 *>(
        a.q + (static_cast<size_t>(i) * a.n_head + g * REP + r) * kPlanarHd)[pp];
    const float cc = tb.gc[pp], sn = tb.gs[pp];
    s_q[r][2 * pp] = cc * qa.x - sn * qa.y;  // src/kvquant.rs:356-366
    s_q[r][2 * pp + 1] = sn * qa.x + cc * qa.y;
  }
  __syncthreads();
  // the lane's 16 rotated coordinates of every head stay in registers for
  // the whole chunk (re-reading them from LDS per position is what bounds a
  // straightforward version: 16 lanes at a 64-byte stride share few banks)
  float qreg[REP][16];
#pragma unroll
  for (int r = 0; r < REP; ++r)
#pragma unroll
    for (int e = 0; e < 16; e += 4) {
      const float4 v4 = *reinterpret_cast<const float4 *>(&s_q[r][16 * sub + e]);
      qreg[r][e] = v4.x;
      qreg[r][e + 1] = v4.y;
      qreg[r][e + 2] = v4.z;
      qreg[r][e + 3] = v4.w;
    }
  // head sub's running max and sum over the wave's positions (lanes sub <
  // REP; the same in the four groups)
  float run_m = -INFINITY, run_l = 0.0f;
  float acc[REP][4];
#pragma unroll
  for (int r = 0; r < REP; ++r)
#pragma unroll
    for (int x = 0; x < 4; ++x) acc[r][x] = 0.0f;

  for (size_t t0 = beg; t0 < end; t0 += kPlTile) {
    const int nt = tile_len(t0);
    const Tile cur = nxt;
    const bool more = t0 + kPlTile < end;
    // the next tile's V words now, its K words once this tile's are used
    if (more) nxt.load_v(a, t0 + kPlTile, tile_len(t0 + kPlTile), g, w, lane, vdw, two);
    float sc[kPasses];  // head sub's score of the group's position, per pass
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
      const bool in = pass * 16 + 4 * w + grp4 < nt;
      unsigned __int128 win = 0;
#pragma unroll
      for (int h = 0; h < Tile::kWords; ++h)
        win |= static_cast<unsigned __int128>(cur.kw[pass][h]) << ((Tile::kDw ? 32 : 16) * h);
      float cv[16];
      if constexpr (kByteTab) {
#pragma unroll
        for (int b = 0; b < 16 / kE; ++b) {
          const CVec cb = s_cb[static_cast<uint32_t>(win >> (8 * b)) & 0xFFu];
          if constexpr (kE == 4) {
            cv[4 * b] = cb.x; cv[4 * b + 1] = cb.y; cv[4 * b + 2] = cb.z; cv[4 * b + 3] = cb.w;
          } else {
            cv[2 * b] = cb.x; cv[2 * b + 1] = cb.y;
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) cv[e] = s_c[static_cast<uint32_t>(win >> (e * BITS)) & kMask];
      }
      const float kscale = cur.kn[pass] * a.scale;
      float d[REP];
#pragma unroll
      for (int r = 0; r < REP; ++r) {
        float s0 = qreg[r][0] * cv[0], s1 = qreg[r][8] * cv[8];
#pragma unroll
        for (int e = 1; e < 8; ++e) {
          s0 = fmaf(qreg[r][e], cv[e], s0);
          s1 = fmaf(qreg[r][8 + e], cv[8 + e], s1);
        }
        d[r] = s0 + s1;
      }
      // the REP row sums step by step, so their DPP moves fill each other's
      // wait slots (every lane of the row ends with the sum)
#pragma unroll
      for (int r = 0; r < REP; ++r) d[r] += dpp_row<0xB1>(d[r]);
#pragma unroll
      for (int r = 0; r < REP; ++r) d[r] += dpp_row<0x4E>(d[r]);
#pragma unroll
      for (int r = 0; r < REP; ++r) d[r] += dpp_row<0x141>(d[r]);
#pragma unroll
      for (int r = 0; r < REP; ++r) d[r] += dpp_row<0x140>(d[r]);
      // src/forward.rs:307: dot_rotated (times the norm) * scale
      sc[pass] = in ? pick(d, sub) * kscale : -INFINITY;
    }
    if (more) nxt.load_k(a, t0 + kPlTile, tile_len(t0 + kPlTile), g, w, grp4, sub);
    // head sub's max over the wave's 16 positions (the four groups)
    const float hm = fmaxf(run_m, rows4_max(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]))));
    const float corr_mine = hm == -INFINITY ? 1.0f : expf(run_m - hm);
    run_m = hm;
    float ps = 0.0f;
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
      const float e = hm == -INFINITY ? 0.0f : expf(sc[pass] - hm);
      ps += e;
      // the P.V weight: p_j, or (p_j |v_j|) for a quantized V (src/forward.rs:344);
      // p_j == 0 adds nothing even for an infinite |v_j| (the reference skips
      // such positions, src/forward.rs:335)
      if (sub < REP) s_e[w][4 * pass + grp4][sub] = VQ ? (e != 0.0f ? e * cur.vn[pass] : 0.0f) : e;
    }
    run_l = run_l * corr_mine + rows4_sum(ps);
    float corr[REP];  // head r's correction, from lane r
#pragma unroll
    for (int r = 0; r < REP; ++r)
      corr[r] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(corr_mine), r));
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int r = 0; r < REP; ++r)
#pragma unroll
      for (int x = 0; x < 4; ++x) acc[r][x] *= corr[r];
    // P.V: lane owns dims 4 lane .. +3 of the wave's 16 positions
#pragma unroll
    for (int jl = 0; jl < kVj; ++jl) {
      if ((jl >> 2) * 16 + 4 * w + (jl & 3) < nt) {
        float4 v;
        if constexpr (VQ) {
          if constexpr (kE == 4) {  // 2 bits: the lane's 4 indices are one byte
            v = s_cb[(cur.vlo[jl] >> vsh) & 0xFFu];
          } else if constexpr (kE == 2) {  // 4 bits: two bytes
            const uint32_t bb = cur.vlo[jl] >> vsh;
            const CVec lo = s_cb[bb & 0xFFu], hi = s_cb[(bb >> 8) & 0xFFu];
            v = make_float4(lo.x, lo.y, hi.x, hi.y);
          } else {
            uint64_t bitsv = cur.vlo[jl];
            if constexpr (Tile::kTwo) bitsv |= static_cast<uint64_t>(cur.vhi[jl]) << 32;
            bitsv >>= vsh;
            v = make_float4(s_c[bitsv & kMask], s_c[(bitsv >> BITS) & kMask],
                            s_c[(bitsv >> (2 * BITS)) & kMask], s_c[(bitsv >> (3 * BITS)) & kMask]);
          }
        } else {
          v = cur.vr[jl];
        }
#pragma unroll
        for (int r = 0; r < REP; ++r) {
          const float e = s_e[w][jl][r];
          acc[r][0] = fmaf(e, v.x, acc[r][0]);
          acc[r][1] = fmaf(e, v.y, acc[r][1]);
          acc[r][2] = fmaf(e, v.z, acc[r][2]);
          acc[r][3] = fmaf(e, v.w, acc[r][3]);
        }
      }
    }
    // the weights are consumed before the next tile writes them
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // merge the four waves: weights e^(m_w - M) per head
#pragma unroll
  for (int r = 0; r < REP; ++r)
#pragma unroll
    for (int x = 0; x < 4; ++x) s_acc[w][r][4 * lane + x] = acc[r][x];
  if (lane < REP) {
    s_wm[w][lane] = run_m;
    s_wl[w][lane] = run_l;
  }
  __syncthreads();
  if (tid < REP) {
    const int r = tid;
    const float big = fmaxf(fmaxf(s_wm[0][r], s_wm[1][r]), fmaxf(s_wm[2][r], s_wm[3][r]));
    float l = 0.0f;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const float wt = s_wm[ww][r] == -INFINITY ? 0.0f : expf(s_wm[ww][r] - big);
      s_ww[ww][r] = wt;
      l += s_wl[ww][r] * wt;
    }
    a.pm[part0 + static_cast<size_t>(r) * a.n_chunks] = big;
    a.pl[part0 + static_cast<size_t>(r) * a.n_chunks] = l;
  }
  __syncthreads();
  for (int o = tid; o < REP * kHd; o += kBlock) {
    const int r = o / kHd, dd = o % kHd;
    const float sum = (s_acc[0][r][dd] * s_ww[0][r] + s_acc[1][r][dd] * s_ww[1][r]) +
                      (s_acc[2][r][dd] * s_ww[2][r] + s_acc[3][r][dd] * s_ww[3][r]);
    a.pacc[(part0 + static_cast<size_t>(r) * a.n_chunks) * kHd + dd] = sum;
  }
}

template <int REP, bool VQ>
int launch_planar_v(const PlanarArgs &a, dim3 grid, const PlanarTables &tb, hipStream_t st) {
  switch (a.bits) {
    case 1: BH_LAUNCH((attn_planar_kernel<REP, 1, VQ>), grid, kBlock, 0, st, a, tb); break;
    case 2: BH_LAUNCH((attn_planar_kernel<REP, 2, VQ>), grid, kBlock, 0, st, a, tb); break;
    case 3: BH_LAUNCH((attn_planar_kernel<REP, 3, VQ>), grid, kBlock, 0, st, a, tb); break;
    case 4: BH_LAUNCH((attn_planar_kernel<REP, 4, VQ>), grid, kBlock, 0, st, a, tb); break;
    case 5: BH_LAUNCH((attn_planar_kernel<REP, 5, VQ>), grid, kBlock, 0, st, a, tb); break;
    case 6: BH_LAUNCH((attn_planar_kernel<REP, 6, VQ>), grid, kBlock, 0, st, a, tb); break;
    case 7: BH_LAUNCH((attn_planar_kernel<REP, 7, VQ>), grid, kBlock, 0, st, a, tb); break;
    default: BH_LAUNCH((attn_planar_kernel<REP, 8, VQ>), grid, kBlock, 0, st, a, tb); break;
  }
  return ok();
}

template <int REP>
int launch_planar(const PlanarArgs &a, dim3 grid, const PlanarTables &tb, hipStream_t st) {
  return a.vq != nullptr ? launch_planar_v<REP, true>(a, grid, tb, st)
                         : launch_planar_v<REP, false>(a, grid, tb, st);
}

// ---- multi-query path (matrix cores) ---------------------------------------
//
// Many query tokens at once (prefill, verification): block (c, t, g) takes
// position chunk c, q-row tile t and kv head g; the tile's rows are
// (query i, head g*REP + r) for 128 consecutive row numbers i*REP + r, so one
// K/V tile staged in LDS serves every q head of the kv head and every query
// of the tile.  Both products run on v_mfma_f32_16x16x32_f16 in transposed
// form -- S^T = K Q^T (positions x rows), O^T = V^T P^T (dims x rows) -- so
// the lane that holds a row's scores (row l % 16, eight positions) holds
// exactly that row's P fragment for the next product and that row's output
// dims: no transposes, and the softmax state of a row sits in the four lanes
// l % 16 + 16 g, combined with two permlane swaps.
//
// f32 inputs need more than f16's 11 bits: every operand is split into
// hi = f16(x') and lo = f16(x' - hi) (22 significant bits) and a product is
// hi*hi + hi*lo + lo*hi, accumulated in f32 (an f16 cache is exact in f16:
// its lo parts are zero and skipped).  The splits are made safe by powers of
// two: a q row is scaled so its largest |q| lies in [2^13, 2^14), each
// staged K position row likewise, each staged V tile as a whole, and P by
// 2^14.  The scores are unscaled exactly before the softmax (then times
// 1/sqrtf(hd)); each tile's P.V product is formed from zero and added to the
// f32 output accumulators, unscaled, as they take the online-softmax
// correction.  Results match the reference's f32 arithmetic to ~1e-7
// relative (sums in another order).
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
constexpr int kMqThreads = 512; // 8 waves
constexpr int kMqRows = 128;    // q rows per block: 8 waves x 16
constexpr int kMqTile = 32;     // positions per tile
constexpr int kKStride = 264;   // halves per staged K row (256 + 8: no bank conflicts)
constexpr int kVStride = 40;    // halves per staged V^T row (32 + 8)
constexpr int kMqMinRows = 48;  // q rows per kv head from which this path is taken
constexpr size_t kMqPreTiles = 8;  // row tiles per kv head from which an f32 cache is pre-split

struct MqArgs {
  const float *q;
  const void *kc, *vc;
  float *pm, *pl, *pacc;  // chunk partials [n_q][n_head][n_chunks] (+ [hd])
  size_t pos0, kv_stride, chunk;
  int n_head, n_q, rep, n_chunks, n_kv;
  float scale;
  // planar-quantized caches: kc holds the packed K rows, vc the packed V rows
  // (or V's f32 rows), kn / vn the norms; unused otherwise
  const float *kn, *vn;
  // one chunk: the rows are final, written here as acc / l (what the merge
  // of a single chunk computes; only an exact zero's sign can differ)
  // instead of as partials; nullptr otherwise
  float *out;
  // f32 cache pre-split by attn_kv_split_kernel (PRE): K as f16 hi / lo
  // halves in the cache's layout with its per-position factors 2^-b; V per
  // (32-position tile, kv head) as [dim][32 halves in vcol order], hi then
  // lo, with the tile's shift; unused otherwise
  const uint16_t *kh, *kl, *vh;
  const float *ks;
  const int *vsh;
};

// 2^e as a float for e <= 127; 0 below the normal range
__device__ __forceinline__ float pow2f(int e) {
  return e < -126 ? 0.0f : __uint_as_float(static_cast<uint32_t>(e + 127) << 23);
}

// exponent that puts the largest magnitude m in [2^13, 2^14); 0 for 0 or non-finite m
__device__ __forceinline__ int split_shift(float m) {
  if (!(m > 0.0f) || !isfinite(m)) return 0;
  return 13 - ilogbf(m);
}

// scale exponent of a V tile: its largest |v| into [2^13, 2^14), kept
// where 2^(vs - 14) stays a normal float
__device__ __forceinline__ int v_shift(float m) {
  if (!(m > 0.0f) || !isfinite(m)) return 0;
  const int e = ilogbf(m) - 13;
  return e < -112 ? -112 : (e > 114 ? 114 : e);
}

__device__ __forceinline__ void split_hl(float x, _Float16 &h, _Float16 &l) {
  h = static_cast<_Float16>(x);
  l = static_cast<_Float16>(x - static_cast<float>(h));
}

// Column of position p (0..31) in a staged V^T row: the eight positions a
// lane group g feeds one P.V step -- 4g .. 4g+3 and 16+4g .. 16+4g+3, the
// positions its S^T fragment holds -- sit in columns 8g .. 8g+7, so the
// fragment is one 16-byte LDS read.
__device__ __forceinline__ int vcol(int p) { return p < 16 ? 8 * (p >> 2) + (p & 3) : 8 * ((p - 16) >> 2) + 4 + (p & 3); }

// PB > 0: a planar-quantized cache of PB-bit indices (src/kvquant.rs).  The
// tile's K and V values are the centroids of the packed indices, looked up
// while staging (V's times its row norm, or V's f32 rows when VQ is false),
// q is rotated as it is split, each score takes K's row norm with the
// position's scale (src/forward.rs:307), and the sums stay in rotated space
// for attn_merge_rows_rot_kernel to turn back.  The rest is the f32 path.
template <bool F16, int PB, bool VQ, bool PRE = false>
__device__ __forceinline__ void mq_body(const MqArgs &a, const float *cent, const float *gc,
                                        const float *gs) {
  constexpr bool PL = PB > 0;
  static_assert(!(PL && F16), "planar caches take the f32 staging");
  static_assert(!(PRE && (PL || F16)), "the pre-split form is for the f32 cache");
  __shared__ __attribute__((aligned(16))) _Float16 sKh[kMqTile * kKStride];
  __shared__ __attribute__((aligned(16))) _Float16 sKl[F16 ? 8 : kMqTile * kKStride];
  __shared__ __attribute__((aligned(16))) _Float16 sVh[kHd * kVStride];
  __shared__ __attribute__((aligned(16))) _Float16 sVl[F16 ? 8 : kHd * kVStride];
  __shared__ __attribute__((aligned(16))) _Float16 sQl[kMqRows * kKStride];  // q lo fragments
  __shared__ float sKs[kMqTile];  // 2^-b of each staged K row
  __shared__ unsigned sVmax[2];   // bits of a tile's largest |v| (non-negative floats order as ints), by tile parity
  __shared__ float sC[PL ? 256 : 1];  // the centroids
  // XCD-aware numbering: workgroups go to the 8 XCDs round robin by id, so
  // the row tiles of one (chunk, kv head) get ids 8 apart -- the same XCD,
  // dispatched together -- and share the K/V tiles in that XCD's L2.
  const int R = a.n_q * a.rep;
  const int tiles_r = (R + kMqRows - 1) / kMqRows;
  int c, t, g;
  {
    const int b = blockIdx.x;
    const int n_groups = a.n_chunks * a.n_kv;  // (chunk, kv head) pairs
    const int full = n_groups / 8 * 8;         // groups placed 8 at a time
    const int x = b % 8, jb = b / 8;
    int q;
    if (a.n_chunks == 1) {
      // one chunk (every position in one block, e.g. a causal prefill): the
      // row tiles longest-first, kv heads interleaved, so the tiles that see
      // the most positions start in the first round instead of the last
      t = tiles_r - 1 - b / a.n_kv;
      q = b % a.n_kv;
    } else if (jb < (full / 8) * tiles_r) {
      q = (jb / tiles_r) * 8 + x;
      t = jb % tiles_r;
    } else {  // the last n_groups % 8 groups, in plain order
      const int rest = b - full * tiles_r;
      q = full + rest / tiles_r;
      t = rest % tiles_r;
    }
    c = q % a.n_chunks;
    g = q / a.n_chunks;
  }
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, r16 = l & 15, grp = l >> 4;
  const int rho = t * kMqRows + w * 16 + r16;
  const bool valid = rho < R;
  const int qi = valid ? rho / a.rep : 0;
  const int head = g * a.rep + (valid ? rho % a.rep : 0);
  const size_t limit = valid ? a.pos0 + qi + 1 : 0;  // this row sees positions < limit
  const int last_row = (t + 1) * kMqRows - 1 < R - 1 ? (t + 1) * kMqRows - 1 : R - 1;
  const size_t lim_blk = a.pos0 + last_row / a.rep + 1;
  const size_t beg = static_cast<size_t>(c) * a.chunk;
  const size_t end = beg + a.chunk < lim_blk ? beg + a.chunk : lim_blk;
  const size_t part = (static_cast<size_t>(qi) * a.n_head + head) * a.n_chunks + c;
  if (beg >= end) {  // no position of this chunk is visible to the tile
    if (valid && a.out != nullptr) {
      // (not reached: a one-chunk tile sees position 0) the merge's 0 / 0
      f32x4 *dst = reinterpret_cast<f32x4 *>(a.out + (static_cast<size_t>(qi) * a.n_head + head) * kHd);
      const float nan = __builtin_nanf("");
#pragma unroll
      for (int dt = 0; dt < 16; ++dt) dst[4 * dt + grp] = f32x4{nan, nan, nan, nan};
    } else if (valid) {
      if (grp == 0) {
        a.pm[part] = -INFINITY;
        a.pl[part] = 0.0f;
      }
      f32x4 *acc = reinterpret_cast<f32x4 *>(a.pacc + part * kHd);
#pragma unroll
      for (int dt = 0; dt < 16; ++dt) acc[4 * dt + grp] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    return;
  }

  // q row fragments: dims 32 s + 8 grp .. +7 of row rho, scaled and split
  half8 qh[8];  // the lo parts go to LDS (registers hold the next tile's K/V)
  _Float16 *qlrow = sQl + (w * 16 + r16) * kKStride + 8 * grp;
  int qa = 0;
  {
    const f32x4 *qr = reinterpret_cast<const f32x4 *>(
        a.q + (static_cast<size_t>(qi) * a.n_head + head) * kHd + 8 * grp);
    f32x4 v[16];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      v[2 * s] = valid ? qr[8 * s] : f32x4{0.f, 0.f, 0.f, 0.f};
      v[2 * s + 1] = valid ? qr[8 * s + 1] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    if constexpr (PL) {
      // rotated q: pairs (2p, 2p + 1) of the lane's dims (src/kvquant.rs:356-366)
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int p0 = (32 * (k >> 1) + 8 * grp + 4 * (k & 1)) >> 1;
        const float c0 = gc[p0], s0 = gs[p0], c1 = gc[p0 + 1], s1 = gs[p0 + 1];
        const f32x4 x = v[k];
        v[k] = f32x4{c0 * x.x - s0 * x.y, s0 * x.x + c0 * x.y, c1 * x.z - s1 * x.w, s1 * x.z + c1 * x.w};
      }
    }
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k)
      m = fmaxf(m, fmaxf(fmaxf(fabsf(v[k].x), fabsf(v[k].y)), fmaxf(fabsf(v[k].z), fabsf(v[k].w))));
    qa = split_shift(rows4_max(m));
    const float f = ldexpf(1.0f, qa);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const f32x4 x = v[2 * s + h];
        _Float16 a0, a1, a2, a3, b0, b1, b2, b3;
        split_hl(x.x * f, a0, b0);
        split_hl(x.y * f, a1, b1);
        split_hl(x.z * f, a2, b2);
        split_hl(x.w * f, a3, b3);
        qh[s][4 * h + 0] = a0; qh[s][4 * h + 1] = a1; qh[s][4 * h + 2] = a2; qh[s][4 * h + 3] = a3;
        half4v lo4;
        lo4[0] = b0; lo4[1] = b1; lo4[2] = b2; lo4[3] = b3;
        *reinterpret_cast<half4v *>(qlrow + 32 * s + 4 * h) = lo4;
      }
    }
  }
  const float qunscale = ldexpf(a.scale, -qa);  // scores: S' * 2^-a * 2^-b * (1/sqrtf(hd))

  f32x4 o[16];
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float run_m = -INFINITY, run_l = 0.0f;
  // the accumulators are in units of 2^(14 - vs_cur); vs_cur only grows
  // within a block, so changing the unit never scales a value up
  int vs_cur = -112;
  if (tid == 0) {
    sVmax[0] = 0u;
    sVmax[1] = 0u;
  }
  if constexpr (PL) {
    if (tid < 256) sC[tid] = cent[tid];
  }
  __syncthreads();
  int parity = 0;

  const size_t head_off = static_cast<size_t>(g) * kHd;
  // staging: K position sp, dims 16 kpart .. +15 (16 lanes per position);
  // V dims vd, vd + 64, vd + 128, vd + 192 of positions 4 vpg .. +3 (a
  // wave's lanes read 256 consecutive bytes per load, and their V^T stores
  // go to consecutive rows: no LDS bank conflicts)
  const int sp = tid >> 4, kpart = tid & 15;
  const int vd = tid & 63, vpg = tid >> 6;
  // this lane's share of a tile: K position sp, dims 16 kpart .. +15; V
  // positions 4 vpg .. +3 at dims vd + 64 i.  Registers hold the next
  // tile's share while the current one is multiplied.
  using KReg = typename std::conditional<F16, uint4[2], f32x4[4]>::type;
  using VElt = typename std::conditional<F16, uint16_t, float>::type;
  KReg kr;
  VElt vr[4][4];
  // planar: the lane's 2 PB bytes of K row sp (16 indices) as PB / 2 dwords
  // or PB halfwords, and of its V positions the index bits of dims vd + 64 i
  // (one or two dwords), with the rows' norms
  constexpr int kPlen = 32 * (PL ? PB : 1);
  constexpr bool kKDw = PB % 2 == 0;
  constexpr int kKWords = !PL ? 1 : (kKDw ? PB / 2 : PB);
  constexpr bool kVTwo = PL && 8 % PB != 0;
  uint32_t kw[kKWords];
  float knr = 0.0f;
  // pre-split f32 cache: K row sp's 16 hi then 16 lo halves, its factor, the
  // V halves of the lane's positions and dims, the tile's V shift
  // (ext_vector_type arrays: HIP's uint4 struct arrays carried across the
  // tile loop are kept in scratch memory)
  u32x4v kph[PRE ? 4 : 1];
  u32x4v vpq[PRE ? 4 : 1];  // 16-byte pieces tid, tid + 512 of the tile's V hi, then of its lo
  float ksr = 0.0f;
  int vsr = 0, cur_vst = 0;
  uint32_t vlo[PL && VQ ? 4 : 1][PL && VQ ? 4 : 1], vhi[kVTwo && VQ ? 4 : 1][kVTwo && VQ ? 4 : 1];
  float vnr[PL && VQ ? 4 : 1];
  auto fetch = [&](size_t t0) {
    const int nt = static_cast<int>(end - t0 < kMqTile ? end - t0 : kMqTile);
    const size_t krow = (t0 + (sp < nt ? sp : nt - 1)) * a.kv_stride + head_off + 16 * kpart;
    const VElt *vcp = static_cast<const VElt *>(a.vc);
    if constexpr (PRE) {
      kph[0] = *reinterpret_cast<const u32x4v *>(a.kh + krow);
      kph[1] = *reinterpret_cast<const u32x4v *>(a.kh + krow + 8);
      kph[2] = *reinterpret_cast<const u32x4v *>(a.kl + krow);
      kph[3] = *reinterpret_cast<const u32x4v *>(a.kl + krow + 8);
      ksr = a.ks[(t0 + (sp < nt ? sp : nt - 1)) * a.n_kv + g];
      const size_t vt = ((t0 / kMqTile) * a.n_kv + g) * (2 * kHd * kMqTile);
      const u32x4v *vsrc = reinterpret_cast<const u32x4v *>(a.vh + vt);
#pragma unroll
      for (int r = 0; r < 4; ++r) vpq[r] = vsrc[tid + kMqThreads * r];
      vsr = a.vsh[(t0 / kMqTile) * a.n_kv + g];
      return;
    }
    if constexpr (PL) {
      const size_t prow = (t0 + (sp < nt ? sp : nt - 1)) * a.n_kv + g;
      const uint8_t *src = static_cast<const uint8_t *>(a.kc) + prow * kPlen + 2 * PB * kpart;
#pragma unroll
      for (int h = 0; h < kKWords; ++h)
        kw[h] = kKDw ? reinterpret_cast<const uint32_t *>(src)[h]
                     : static_cast<uint32_t>(reinterpret_cast<const uint16_t *>(src)[h]);
      knr = a.kn[prow];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int pj = 4 * vpg + jj;
        const size_t vpos = t0 + (pj < nt ? pj : nt - 1);
        if constexpr (VQ) {
          const size_t vrow = vpos * a.n_kv + g;
          const uint32_t *vsrc = reinterpret_cast<const uint32_t *>(static_cast<const uint8_t *>(a.vc) + vrow * kPlen);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int bit = (vd + 64 * i) * PB;
            vlo[jj][i] = vsrc[bit >> 5];
            if constexpr (kVTwo) vhi[jj][i] = (bit & 31) + PB > 32 ? vsrc[(bit >> 5) + 1] : 0u;
          }
          vnr[jj] = a.vn[vrow];
        } else {
          const size_t e = vpos * a.kv_stride + head_off + vd;
#pragma unroll
          for (int i = 0; i < 4; ++i) vr[jj][i] = vcp[e + 64 * i];
        }
      }
      return;
    }
    if constexpr (F16) {
      const uint16_t *kcp = static_cast<const uint16_t *>(a.kc);
      kr[0] = *reinterpret_cast<const uint4 *>(kcp + krow);
      kr[1] = *reinterpret_cast<const uint4 *>(kcp + krow + 8);
    } else {
      const float *kcp = static_cast<const float *>(a.kc);
#pragma unroll
      for (int k = 0; k < 4; ++k) kr[k] = *reinterpret_cast<const f32x4 *>(kcp + krow + 4 * k);
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int pj = 4 * vpg + jj;
      const size_t e = (t0 + (pj < nt ? pj : nt - 1)) * a.kv_stride + head_off + vd;
#pragma unroll
      for (int i = 0; i < 4; ++i) vr[jj][i] = vcp[e + 64 * i];
    }
  };
  fetch(beg);
  for (size_t t0 = beg; t0 < end; t0 += kMqTile) {
    const int nt = static_cast<int>(end - t0 < kMqTile ? end - t0 : kMqTile);
    const int vc0 = vcol(4 * vpg);  // the 4 columns of this lane's positions
    if constexpr (PRE) {
      u32x4v *kd = reinterpret_cast<u32x4v *>(sKh + sp * kKStride + 16 * kpart);
      kd[0] = kph[0];
      kd[1] = kph[1];
      u32x4v *kld = reinterpret_cast<u32x4v *>(sKl + sp * kKStride + 16 * kpart);
      kld[0] = kph[2];
      kld[1] = kph[3];
      if (kpart == 0) sKs[sp] = ksr;
      // piece u of an array: dim u / 4, columns 8 (u % 4) .. +7
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int u = (tid + kMqThreads * r) & (4 * kHd - 1);
        _Float16 *dst = (r < 2 ? sVh : sVl) + (u >> 2) * kVStride + 8 * (u & 3);
        *reinterpret_cast<u32x4v *>(dst) = vpq[r];
      }
      cur_vst = vsr;  // the prefetch below overwrites vsr
      __syncthreads();
    } else if constexpr (F16) {
      const uint4 k0 = kr[0], k1 = kr[1];
      uint4 *kd = reinterpret_cast<uint4 *>(sKh + sp * kKStride + 16 * kpart);
      kd[0] = k0;
      kd[1] = k1;
      if (kpart == 0) sKs[sp] = 1.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        half4v col;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) col[jj] = __builtin_bit_cast(_Float16, vr[jj][i]);
        *reinterpret_cast<half4v *>(sVh + (vd + 64 * i) * kVStride + vc0) = col;
      }
      __syncthreads();
    } else {
      if constexpr (PL) {
        // centroids of the staged indices (K: 16 of row sp; V: 4 dims of 4
        // positions, times the V rows' norms)
        constexpr uint32_t kMask = (1u << PB) - 1u;
        unsigned __int128 win = 0;
#pragma unroll
        for (int h = 0; h < kKWords; ++h) win |= static_cast<unsigned __int128>(kw[h]) << ((kKDw ? 32 : 16) * h);
#pragma unroll
        for (int k = 0; k < 4; ++k)
          kr[k] = f32x4{sC[static_cast<uint32_t>(win >> ((4 * k) * PB)) & kMask],
                        sC[static_cast<uint32_t>(win >> ((4 * k + 1) * PB)) & kMask],
                        sC[static_cast<uint32_t>(win >> ((4 * k + 2) * PB)) & kMask],
                        sC[static_cast<uint32_t>(win >> ((4 * k + 3) * PB)) & kMask]};
        if constexpr (VQ) {
#pragma unroll
          for (int jj = 0; jj < 4; ++jj)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              uint64_t b = vlo[jj][i];
              if constexpr (kVTwo) b |= static_cast<uint64_t>(vhi[jj][i]) << 32;
              vr[jj][i] = sC[(b >> (((vd + 64 * i) * PB) & 31)) & kMask] * vnr[jj];
            }
        }
      }
      float km = 0.0f, vm = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        km = fmaxf(km, fmaxf(fmaxf(fabsf(kr[k].x), fabsf(kr[k].y)), fmaxf(fabsf(kr[k].z), fabsf(kr[k].w))));
        vm = fmaxf(vm, fmaxf(fmaxf(fabsf(vr[k][0]), fabsf(vr[k][1])), fmaxf(fabsf(vr[k][2]), fabsf(vr[k][3]))));
      }
      km = lane_group_reduce<16>(km, FMaxOp{});
      vm = lane_group_reduce<64>(vm, FMaxOp{});
      if (l == 0) atomicMax(&sVmax[parity], __float_as_uint(vm));
      const int kb = split_shift(km);
      const float kf = ldexpf(1.0f, kb);
      _Float16 *khp = sKh + sp * kKStride + 16 * kpart;
      _Float16 *klp = sKl + sp * kKStride + 16 * kpart;
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        half8 hv, lv;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const f32x4 x = kr[2 * k2 + k];
          _Float16 h, lo;
          split_hl(x.x * kf, h, lo); hv[4 * k + 0] = h; lv[4 * k + 0] = lo;
          split_hl(x.y * kf, h, lo); hv[4 * k + 1] = h; lv[4 * k + 1] = lo;
          split_hl(x.z * kf, h, lo); hv[4 * k + 2] = h; lv[4 * k + 2] = lo;
          split_hl(x.w * kf, h, lo); hv[4 * k + 3] = h; lv[4 * k + 3] = lo;
        }
        *reinterpret_cast<half8 *>(khp + 8 * k2) = hv;
        *reinterpret_cast<half8 *>(klp + 8 * k2) = lv;
      }
      if (kpart == 0) sKs[sp] = PL ? ldexpf(knr, -kb) : ldexpf(1.0f, -kb);
      __syncthreads();  // sVmax[parity] complete
      const int vst = v_shift(__uint_as_float(sVmax[parity]));
      const int vs = vst > vs_cur ? vst : vs_cur;
      const float vf = ldexpf(1.0f, -vs);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        half4v ch, cl;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          _Float16 h, lo;
          split_hl(vr[jj][i] * vf, h, lo);
          ch[jj] = h;
          cl[jj] = lo;
        }
        *reinterpret_cast<half4v *>(sVh + (vd + 64 * i) * kVStride + vc0) = ch;
        *reinterpret_cast<half4v *>(sVl + (vd + 64 * i) * kVStride + vc0) = cl;
      }
      __syncthreads();
    }
    if (t0 + kMqTile < end) fetch(t0 + kMqTile);  // the next tile, in flight during this one
    int vs = vs_cur;
    float pfac = 1.0f;  // PRE: the tile's V is in units of 2^vst, the block's of 2^vs
    if constexpr (PRE) {
      vs = cur_vst > vs_cur ? cur_vst : vs_cur;
      pfac = pow2f(cur_vst - vs);
    } else if constexpr (!F16) {
      const int vst = v_shift(__uint_as_float(sVmax[parity]));
      vs = vst > vs_cur ? vst : vs_cur;
      // the other slot was last read before the previous tile's final
      // barrier and is next written after this tile's
      if (tid == 0) sVmax[parity ^ 1] = 0u;
      parity ^= 1;
    } else {
      vs = 0;
    }

    // S^T = K' Q'^T: lane holds row r16, positions 16 ct + 4 grp + i
    f32x4 st[2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      const _Float16 *kh = sKh + (16 * ct + r16) * kKStride + 8 * grp;
      const _Float16 *kl = sKl + (F16 ? 0 : (16 * ct + r16) * kKStride + 8 * grp);
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const half8 ka = *reinterpret_cast<const half8 *>(kh + 32 * s);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[s], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            ka, *reinterpret_cast<const half8 *>(qlrow + 32 * s), acc, 0, 0, 0);
        if constexpr (!F16) {
          const half8 kb = *reinterpret_cast<const half8 *>(kl + 32 * s);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb, qh[s], acc, 0, 0, 0);
        }
      }
      st[ct] = acc;
    }
    // scores, masked: causal limit of the row, the tile's valid positions
    float sc[8];
    float tmax = -INFINITY;
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int pj = 16 * ct + 4 * grp + i;
        const bool vis = pj < nt && t0 + pj < limit;
        const float x = st[ct][i] * sKs[pj] * qunscale;
        sc[4 * ct + i] = vis ? x : -INFINITY;
        tmax = fmaxf(tmax, sc[4 * ct + i]);
      }
    tmax = rows4_max(tmax);
    const float m_new = fmaxf(run_m, tmax);
    const bool none = m_new == -INFINITY;
    const float corr = exp_hw(none ? 0.0f : run_m - m_new);
    float psum = 0.0f;
    half8 ph, pl;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float p = exp_hw(none ? -INFINITY : sc[k] - m_new);
      psum += p;
      _Float16 h, lo;
      split_hl(p * (PRE ? 16384.0f * pfac : 16384.0f), h, lo);
      ph[k] = h;
      pl[k] = lo;
    }
    run_l = run_l * corr + rows4_sum(psum);
    run_m = m_new;
    // accumulators: softmax correction and the change of unit (never up)
    const float ocorr = F16 ? corr : corr * pow2f(vs_cur - vs);
    vs_cur = vs;
    // O^T += V'^T P*^T: A = V^T rows 16 dt + r16, columns 8 grp .. +7
    // (the rescale is skipped when no row of the wave needs it: the running
    // maxima and the unit settle after the first tiles)
    if (__builtin_amdgcn_ballot_w64(ocorr != 1.0f) != 0) {
#pragma unroll
      for (int dt = 0; dt < 16; ++dt) o[dt] = o[dt] * ocorr;
    }
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) {
      const half8 va = *reinterpret_cast<const half8 *>(sVh + (16 * dt + r16) * kVStride + 8 * grp);
      f32x4 acc = o[dt];
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, ph, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl, acc, 0, 0, 0);
      if constexpr (!F16) {
        const half8 vb = *reinterpret_cast<const half8 *>(sVl + (16 * dt + r16) * kVStride + 8 * grp);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(vb, ph, acc, 0, 0, 0);
      }
      o[dt] = acc;
    }
    __syncthreads();  // the staged tile is consumed
  }
  if (valid) {
    const float u = F16 ? 1.0f / 16384.0f : pow2f(vs_cur - 14);
    if (a.out != nullptr) {
      // the merge of one chunk: weight e^0 = 1, so (acc * 1) / (l * 1)
      // (the merge's 0 + acc turns an exact -0 into +0; nothing else differs)
      f32x4 *dst = reinterpret_cast<f32x4 *>(a.out + (static_cast<size_t>(qi) * a.n_head + head) * kHd);
#pragma unroll
      for (int dt = 0; dt < 16; ++dt) dst[4 * dt + grp] = (o[dt] * u) / run_l;
    } else {
      if (grp == 0) {
        a.pm[part] = run_m;
        a.pl[part] = run_l;
      }
      f32x4 *acc = reinterpret_cast<f32x4 *>(a.pacc + part * kHd);
#pragma unroll
      for (int dt = 0; dt < 16; ++dt) acc[4 * dt + grp] = o[dt] * u;
    }
  }
}

template <bool F16>
__global__ __launch_bounds__(kMqThreads) void attn_mq_kernel(MqArgs a) {
  mq_body<F16, 0, false>(a, nullptr, nullptr, nullptr);
}

// The f32 path over a pre-split cache (see attn_kv_split_kernel).
__global__ __launch_bounds__(kMqThreads) void attn_mq_pre_kernel(MqArgs a) {
  mq_body<false, 0, false, true>(a, nullptr, nullptr, nullptr);
}

// Splits the f32 cache once for a multi-query call whose blocks would each
// split the same K / V tiles again: block (tile, g) takes positions 32 tile
// .. 32 tile + 31 of kv head g.  Each K row is scaled so its largest |k| lies
// in [2^13, 2^14) (factor 2^-b kept per position) and each 32-position V
// tile by its own shift vst (its largest |v| into [2^13, 2^14)); both are
// split into f16 hi = f16(x') and lo = f16(x' - hi), stored in the caches'
// layout (V per tile in the order the block stages it: [dim][32 halves at
// columns vcol(p)], hi rows then lo rows).  These are the scales and splits
// the f32 staging of mq_body forms
// per tile (the block then multiplies P by 2^(vst - vs) for its running V
// unit vs instead of rescaling V).
__global__ __launch_bounds__(256) void attn_kv_split_kernel(const float *kc, const float *vc,
                                                            size_t n_pos, size_t kv_stride, int n_kv,
                                                            uint16_t *kh, uint16_t *kl, float *ks,
                                                            uint16_t *vt, int *vsh) {
  __shared__ float sm[4];
  const int tile = static_cast<int>(blockIdx.x) / n_kv, g = static_cast<int>(blockIdx.x) % n_kv;
  const size_t p0 = static_cast<size_t>(tile) * kMqTile, head_off = static_cast<size_t>(g) * kHd;
  const int tid = threadIdx.x, sp = tid >> 4, kpart = tid & 15;
#pragma unroll
  for (int pass = 0; pass < kMqTile / 16; ++pass) {
    const size_t p = p0 + 16 * pass + sp;
    const bool ok = p < n_pos;
    const size_t off = p * kv_stride + head_off + 16 * kpart;
    f32x4 x[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      x[k] = ok ? *reinterpret_cast<const f32x4 *>(kc + off + 4 * k) : f32x4{0.f, 0.f, 0.f, 0.f};
    float km = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      km = fmaxf(km, fmaxf(fmaxf(fabsf(x[k].x), fabsf(x[k].y)), fmaxf(fabsf(x[k].z), fabsf(x[k].w))));
    km = lane_group_reduce<16>(km, FMaxOp{});
    const int kb = split_shift(km);
    const float kf = ldexpf(1.0f, kb);
    if (ok) {
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        half8 hv, lv;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const f32x4 y = x[2 * k2 + k];
          _Float16 h, lo;
          split_hl(y.x * kf, h, lo); hv[4 * k + 0] = h; lv[4 * k + 0] = lo;
          split_hl(y.y * kf, h, lo); hv[4 * k + 1] = h; lv[4 * k + 1] = lo;
          split_hl(y.z * kf, h, lo); hv[4 * k + 2] = h; lv[4 * k + 2] = lo;
          split_hl(y.w * kf, h, lo); hv[4 * k + 3] = h; lv[4 * k + 3] = lo;
        }
        *reinterpret_cast<half8 *>(kh + off + 8 * k2) = hv;
        *reinterpret_cast<half8 *>(kl + off + 8 * k2) = lv;
      }
      if (kpart == 0) ks[p * n_kv + g] = ldexpf(1.0f, -kb);
    }
  }
  // V: dim tid of the tile's positions (past the cache's end, copies of
  // its last row: finite values the kernel masks)
  float v[kMqTile];
  float vm = 0.0f;
#pragma unroll
  for (int i = 0; i < kMqTile; ++i) {
    const size_t p = p0 + i < n_pos ? p0 + i : n_pos - 1;
    v[i] = vc[p * kv_stride + head_off + tid];
    vm = fmaxf(vm, fabsf(v[i]));
  }
  vm = wave_max(vm);
  if ((tid & 63) == 0) sm[tid >> 6] = vm;
  __syncthreads();
  vm = fmaxf(fmaxf(sm[0], sm[1]), fmaxf(sm[2], sm[3]));
  const int vst = v_shift(vm);
  if (tid == 0) vsh[tile * n_kv + g] = vst;
  const float vf = ldexpf(1.0f, -vst);
  // the row of dim tid in the staged order (position p at column vcol(p)),
  // hi then lo, 64 contiguous bytes each
  half8 hrow[4], lrow[4];
#pragma unroll
  for (int i = 0; i < kMqTile; ++i) {
    _Float16 h, lo;
    split_hl(v[i] * vf, h, lo);
    const int col = vcol(i);
    hrow[col >> 3][col & 7] = h;
    lrow[col >> 3][col & 7] = lo;
  }
  half8 *dh = reinterpret_cast<half8 *>(vt + ((static_cast<size_t>(tile) * n_kv + g) * 2 * kHd + tid) * kMqTile);
  half8 *dl = reinterpret_cast<half8 *>(vt + ((static_cast<size_t>(tile) * n_kv + g) * 2 * kHd + kHd + tid) * kMqTile);
#pragma unroll
  for (int c4 = 0; c4 < 4; ++c4) {
    dh[c4] = hrow[c4];
    dl[c4] = lrow[c4];
  }
}

template <int PB, bool VQ>
__global__ __launch_bounds__(kMqThreads) void attn_mq_planar_kernel(MqArgs a, PlanarTables tb) {
  mq_body<false, PB, VQ>(a, tb.cent, tb.gc, tb.gs);
}

// Decode over an f16 cache on the matrix cores.  Block (chunk, kv head,
// query) of 4 waves; each wave streams its own 16-position steps (positions
// p0 .. p0 + 15, p0 = chunk start + 16 w + 64 k) with its own online softmax
// and no block barrier.  S^T = K Q^T on v_mfma_f32_16x16x32_f16: the A
// operand is the K rows themselves (lane l: position p0 + l % 16, 8
// consecutive f16 dims, one 16-byte load -- no conversion, no staging), B
// the kv head's REP q rows (zero rows up to 16) split into f16 hi + lo after
// scaling by 2^a (the multi-query kernel's split).  The lane that ends with
// a row's scores of four positions holds exactly that row's P fragment of
// O^T += V^T P^T on v_mfma_f32_16x16x16_f16 (P times 2^14, split hi + lo);
// V^T comes from the wave's 16 V rows staged in its own LDS slice (16-byte
// stores, rows padded by 32 bytes so the four lane groups read distinct
// banks).  The four waves merge once per chunk, as in the VALU kernel.
template <int REP>
__global__ __launch_bounds__(kBlock) void attn_decode_f16_mfma_kernel(DecodeArgs a) {
  static_assert(REP <= 16, "q rows of one MFMA tile");
  constexpr int kVStr = kHd + 16;  // halves per staged V row
  __shared__ __attribute__((aligned(16))) _Float16 s_v[4][16 * kVStr];
  __shared__ float s_wm[4][REP], s_wl[4][REP], s_ww[4][REP];
  // the waves' accumulators for the merge reuse the V slices
  static_assert(sizeof(float) * 4 * REP * kHd <= sizeof(_Float16) * 4 * 16 * kVStr, "merge area");
  auto s_o = reinterpret_cast<float (*)[REP][kHd]>(&s_v[0][0]);
  __shared__ __attribute__((aligned(16))) _Float16 s_qh[16 * kKStride];  // q hi and lo fragments
  __shared__ __attribute__((aligned(16))) _Float16 s_ql[16 * kKStride];  // (every wave's)
  const uint16_t *kc = static_cast<const uint16_t *>(a.kc);
  const uint16_t *vc = static_cast<const uint16_t *>(a.vc);
  const int c = blockIdx.x, g = blockIdx.y, i = blockIdx.z;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, r16 = l & 15, grp = l >> 4;
  const size_t n_pos = a.pos0 + i + 1;
  const size_t beg = static_cast<size_t>(c) * a.chunk;
  const size_t end = beg + a.chunk < n_pos ? beg + a.chunk : n_pos;
  const size_t part0 = (static_cast<size_t>(i) * a.n_head + static_cast<size_t>(g) * REP) *
                       a.n_chunks + c;
  if (beg >= end) {  // this query has no positions in the chunk
    if (tid < REP) {
      a.pm[part0 + static_cast<size_t>(tid) * a.n_chunks] = -INFINITY;
      a.pl[part0 + static_cast<size_t>(tid) * a.n_chunks] = 0.0f;
    }
    for (int o = tid; o < REP * kHd; o += kBlock)
      a.pacc[(part0 + static_cast<size_t>(o / kHd) * a.n_chunks) * kHd + o % kHd] = 0.0f;
    return;
  }
  const size_t head_off = static_cast<size_t>(g) * kHd;
  // q fragments: row r16 (< REP), dims 32 s + 8 grp .. +7, scaled and
  // split, into LDS (every wave needs the same; wave 0 writes them)
  _Float16 *qhrow = s_qh + r16 * kKStride + 8 * grp;
  _Float16 *qlrow = s_ql + r16 * kKStride + 8 * grp;
  int qa = 0;
  {
    const bool rv = r16 < REP;
    const f32x4 *qr = reinterpret_cast<const f32x4 *>(
        a.q + (static_cast<size_t>(i) * a.n_head + g * REP + (rv ? r16 : 0)) * kHd + 8 * grp);
    f32x4 v[16];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      v[2 * s] = rv ? qr[8 * s] : f32x4{0.f, 0.f, 0.f, 0.f};
      v[2 * s + 1] = rv ? qr[8 * s + 1] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; ++k)
      m = fmaxf(m, fmaxf(fmaxf(fabsf(v[k].x), fabsf(v[k].y)), fmaxf(fabsf(v[k].z), fabsf(v[k].w))));
    qa = split_shift(rows4_max(m));
    const float f = ldexpf(1.0f, qa);
#pragma unroll
    for (int s = 0; s < 8; ++s)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const f32x4 x = v[2 * s + h];
        _Float16 hi, lo;
        half4v hi4, lo4;
        split_hl(x.x * f, hi, lo); hi4[0] = hi; lo4[0] = lo;
        split_hl(x.y * f, hi, lo); hi4[1] = hi; lo4[1] = lo;
        split_hl(x.z * f, hi, lo); hi4[2] = hi; lo4[2] = lo;
        split_hl(x.w * f, hi, lo); hi4[3] = hi; lo4[3] = lo;
        if (w == 0) {
          *reinterpret_cast<half4v *>(qhrow + 32 * s + 4 * h) = hi4;
          *reinterpret_cast<half4v *>(qlrow + 32 * s + 4 * h) = lo4;
        }
      }
  }
  __syncthreads();  // s_qh, s_ql
  const float qunscale = ldexpf(a.scale, -qa);  // scores: S' * 2^-a * (1/sqrtf(hd))
  f32x4 o[16];
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float run_m = -INFINITY, run_l = 0.0f;  // row r16's (the same in the four groups)
  _Float16 *sv = s_v[w];
  u32x4v kf[8];  // ext vectors: a HIP vector-struct array here is kept in scratch
  auto load_k = [&](size_t p0) {
    const size_t pos = p0 + r16 < end ? p0 + r16 : end - 1;
    const uint16_t *src = kc + pos * a.kv_stride + head_off + 8 * grp;
#pragma unroll
    for (int s = 0; s < 8; ++s) kf[s] = *reinterpret_cast<const u32x4v *>(src + 32 * s);
  };
  // the 16 V rows: 16-byte unit e = 64 k + l of the wave's 512 is unit
  // e % 32 of row e / 32
  u32x4v vr[8];
  auto load_v = [&](size_t p0) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int e = 64 * k + l, pj = e >> 5, u = e & 31;
      const size_t pos = p0 + pj < end ? p0 + pj : end - 1;
      vr[k] = *reinterpret_cast<const u32x4v *>(vc + pos * a.kv_stride + head_off + 8 * u);
    }
  };
  size_t p0 = beg + 16 * w;
  if (p0 < end) {
    load_k(p0);
    load_v(p0);
  }
  for (; p0 < end; p0 += 64) {
    f32x4 st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const half8 ka = __builtin_bit_cast(half8, kf[s]);
      st = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          ka, *reinterpret_cast<const half8 *>(qhrow + 32 * s), st, 0, 0, 0);
      st = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          ka, *reinterpret_cast<const half8 *>(qlrow + 32 * s), st, 0, 0, 0);
    }
    if (p0 + 64 < end) load_k(p0 + 64);  // the next step's K rows, in flight during this one
    // row r16's scores of positions p0 + 4 grp + j
    float sc[4];
    float tmax = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sc[j] = p0 + 4 * grp + j < end ? st[j] * qunscale : -INFINITY;
      tmax = fmaxf(tmax, sc[j]);
    }
    const float m_new = fmaxf(run_m, rows4_max(tmax));
    const bool none = m_new == -INFINITY;
    const float corr = none ? 1.0f : expf(run_m - m_new);
    float ps = 0.0f;
    half4v ph, pl;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float p = none ? 0.0f : expf(sc[j] - m_new);
      ps += p;
      _Float16 hi, lo;
      split_hl(p * 16384.0f, hi, lo);
      ph[j] = hi;
      pl[j] = lo;
    }
    run_l = run_l * corr + rows4_sum(ps);
    run_m = m_new;
    if (__builtin_amdgcn_ballot_w64(corr != 1.0f) != 0) {
#pragma unroll
      for (int dt = 0; dt < 16; ++dt) o[dt] = o[dt] * corr;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int e = 64 * k + l, pj = e >> 5, u = e & 31;
      *reinterpret_cast<u32x4v *>(sv + pj * kVStr + 8 * u) = vr[k];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (p0 + 64 < end) load_v(p0 + 64);  // the next step's V rows, in flight during P.V and its scores
    // O^T += V^T P^T: A = V^T rows 16 dt + r16, positions 4 grp .. +3
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) {
      half4v va;
#pragma unroll
      for (int j = 0; j < 4; ++j) va[j] = sv[(4 * grp + j) * kVStr + 16 * dt + r16];
      f32x4 acc = o[dt];
      acc = __builtin_amdgcn_mfma_f32_16x16x16f16(va, ph, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pl, acc, 0, 0, 0);
      o[dt] = acc;
    }
    // the staged rows are consumed before the next step writes them
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // merge the four waves: weights e^(m_w - M) per head
  __syncthreads();  // every wave is done with its V slice
  if (r16 < REP) {
#pragma unroll
    for (int dt = 0; dt < 16; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j) s_o[w][r16][16 * dt + 4 * grp + j] = o[dt][j] * (1.0f / 16384.0f);
    if (grp == 0) {
      s_wm[w][r16] = run_m;
      s_wl[w][r16] = run_l;
    }
  }
  __syncthreads();
  if (tid < REP) {
    const int r = tid;
    const float big = fmaxf(fmaxf(s_wm[0][r], s_wm[1][r]), fmaxf(s_wm[2][r], s_wm[3][r]));
    float lsum = 0.0f;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      const float wt = s_wm[ww][r] == -INFINITY ? 0.0f : expf(s_wm[ww][r] - big);
      s_ww[ww][r] = wt;
      lsum += s_wl[ww][r] * wt;
    }
    a.pm[part0 + static_cast<size_t>(r) * a.n_chunks] = big;
    a.pl[part0 + static_cast<size_t>(r) * a.n_chunks] = lsum;
  }
  __syncthreads();
  for (int x = tid; x < REP * kHd; x += kBlock) {
    const int r = x / kHd, dd = x % kHd;
    const float sum = (s_o[0][r][dd] * s_ww[0][r] + s_o[1][r][dd] * s_ww[1][r]) +
                      (s_o[2][r][dd] * s_ww[2][r] + s_o[3][r][dd] * s_ww[3][r]);
    a.pacc[(part0 + static_cast<size_t>(r) * a.n_chunks) * kHd + dd] = sum;
  }
}

// Chunk merge of the multi-query path (few chunks, many rows): one block of
// four waves per (query, head) row, wave w owning dims 64 w .. 64 w + 63 (one
// per lane).  Every wave weighs the chunks itself -- e^(m_c - M) from the
// chunks' (max, sum) pairs, one chunk per lane, a loop beyond 64 -- then adds
// the chunks' accumulators, all of a lane's loads in flight together, and
// divides by the weighted sum.  Chunks with no visible position (max -inf)
// are left out.
// ROT: the inverse Givens rotation of the merged row, as in combine1_body.
template <bool ROT>
__device__ __forceinline__ void merge_rows_body(const float *pm, const float *pl, const float *pacc,
                                                int n_chunks, float *out, const float *gc,
                                                const float *gs) {
  __shared__ float s_w[4][64];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const size_t row = blockIdx.x;
  const float *m = pm + row * n_chunks;
  const float *l = pl + row * n_chunks;
  const float *acc = pacc + row * n_chunks * static_cast<size_t>(kHd) + 64 * w + lane;
  float big = -INFINITY;
  for (int c = lane; c < n_chunks; c += 64) big = fmaxf(big, m[c]);
  big = wave_max(big);
  float den = 0.0f, num = 0.0f;
  for (int c0 = 0; c0 < n_chunks; c0 += 64) {
    const int c = c0 + lane;
    const float mc = c < n_chunks ? m[c] : -INFINITY;
    const float lc = c < n_chunks ? l[c] : 0.0f;
    const float wc = mc != -INFINITY ? expf(mc - big) : 0.0f;
    den += lc * wc;
    s_w[w][lane] = wc;  // read back by this wave only
    __builtin_amdgcn_wave_barrier();
    const int cn = n_chunks - c0 < 64 ? n_chunks - c0 : 64;
#pragma unroll 16
    for (int k = 0; k < cn; ++k) {
      const float a = acc[static_cast<size_t>(c0 + k) * kHd];
      const float wk = s_w[w][k];
      num += wk != 0.0f ? a * wk : 0.0f;
    }
    __builtin_amdgcn_wave_barrier();  // weights consumed before the next tile's
  }
  den = wave_sum(den);
  const float val = num / den;
  const int d = 64 * w + lane;
  if constexpr (ROT) {
    const float other = __shfl_xor(val, 1, 64);
    const float c = gc[d >> 1], sn = gs[d >> 1];
    out[row * kHd + d] = (d & 1) == 0 ? c * val + sn * other : -sn * other + c * val;
  } else {
    out[row * kHd + d] = val;
  }
}

__global__ __launch_bounds__(256) void attn_merge_rows_kernel(const float *pm, const float *pl,
                                                              const float *pacc, int n_chunks,
                                                              float *out) {
  merge_rows_body<false>(pm, pl, pacc, n_chunks, out, nullptr, nullptr);
}

__global__ __launch_bounds__(256) void attn_merge_rows_rot_kernel(const float *pm, const float *pl,
                                                                  const float *pacc, int n_chunks,
                                                                  float *out, PlanarTables tb) {
  merge_rows_body<true>(pm, pl, pacc, n_chunks, out, tb.gc, tb.gs);
}

// ---- generic path ----------------------------------------------------------

struct GenericArgs {
  const float *q;
  const void *kc, *vc;
  float *probs;  // [n_q][n_head][n_max]
  float *out;
  size_t pos0, n_max, kv_stride, hd;
  int n_head, n_rep;
  float scale;
};

// One block per (query, head): scores, max, expf, f64 sum, p = e * inv.
// Each lane only rereads the probs entries it wrote itself.
template <class T>
__global__ __launch_bounds__(kBlock) void attn_probs_kernel(GenericArgs a) {
  __shared__ float s_max[kBlock / 64];
  __shared__ double s_sum[kBlock / 64];
  const T *kc = static_cast<const T *>(a.kc);
  const int h = blockIdx.x, i = blockIdx.y;
  const int tid = threadIdx.x;
  const size_t n_pos = a.pos0 + i + 1;
  const float *qh = a.q + (static_cast<size_t>(i) * a.n_head + h) * a.hd;
  const size_t kv_off = static_cast<size_t>(h / a.n_rep) * a.hd;
  float *pr = a.probs + (static_cast<size_t>(i) * a.n_head + h) * a.n_max;
  float mx = -INFINITY;
  for (size_t j = tid; j < n_pos; j += kBlock) {
    float sum = 0.0f;
    const size_t row = j * a.kv_stride + kv_off;
    for (size_t d = 0; d < a.hd; ++d) sum += qh[d] * Kv<T>::at(kc, row + d);  // :181-183
    const float s = sum * a.scale;
    pr[j] = s;
    mx = fmaxf(mx, s);
  }
  mx = wave_max(mx);
  if (tid % 64 == 0) s_max[tid / 64] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(s_max[0], s_max[1]), fmaxf(s_max[2], s_max[3]));
  double part = 0.0;
  for (size_t j = tid; j < n_pos; j += kBlock) {
    const float e = expf(pr[j] - mx);
    pr[j] = e;
    part += static_cast<double>(e);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off, 64);
  if (tid % 64 == 0) s_sum[tid / 64] = part;
  __syncthreads();
  const double total = (s_sum[0] + s_sum[1]) + (s_sum[2] + s_sum[3]);
  const float inv = 1.0f / static_cast<float>(total);
  for (size_t j = tid; j < n_pos; j += kBlock) pr[j] *= inv;
}

// out[d] = sum_j p_j v_j[d] in position order, skipping p_j == 0.
template <class T>
__global__ __launch_bounds__(kBlock) void attn_pv_kernel(GenericArgs a) {
  const T *vc = static_cast<const T *>(a.vc);
  const int h = blockIdx.x, i = blockIdx.y;
  const size_t d = static_cast<size_t>(blockIdx.z) * kBlock + threadIdx.x;
  if (d >= a.hd) return;
  const size_t n_pos = a.pos0 + i + 1;
  const size_t kv_off = static_cast<size_t>(h / a.n_rep) * a.hd;
  const float *pr = a.probs + (static_cast<size_t>(i) * a.n_head + h) * a.n_max;
  float o = 0.0f;
  for (size_t j = 0; j < n_pos; ++j) {
    const float p = pr[j];
    if (p == 0.0f) continue;
    o += p * Kv<T>::at(vc, j * a.kv_stride + kv_off + d);
  }
  a.out[(static_cast<size_t>(i) * a.n_head + h) * a.hd + d] = o;
}

template <int REP, class T>
int launch_decode(const DecodeArgs &a, int n_kv, int n_q, hipStream_t st) {
  if constexpr (std::is_same<T, uint16_t>::value) {  // f16: the matrix-core form
    BH_LAUNCH((attn_decode_f16_mfma_kernel<REP>), dim3(a.n_chunks, n_kv, n_q), kBlock, 0, st, a);
    return ok();
  }
  if (a.tile == 32)
    BH_LAUNCH((attn_decode_kernel<REP, T, 32>), dim3(a.n_chunks, n_kv, n_q), kBlock, 0, st, a);
  else
    BH_LAUNCH((attn_decode_kernel<REP, T, 64>), dim3(a.n_chunks, n_kv, n_q), kBlock, 0, st, a);
  return ok();
}

// Resident blocks of the multi-query kernel on this device (per cache type).
size_t mq_capacity(bool f16) {
  static std::mutex mu;
  static size_t cap[64][2] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  size_t &c = cap[dev][f16 ? 1 : 0];
  if (c == 0) {
    int per_cu = 0, cus = 0;
    const hipError_t e1 =
        f16 ? hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, attn_mq_kernel<true>, kMqThreads, 0)
            : hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, attn_mq_kernel<false>, kMqThreads, 0);
    if (e1 != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        per_cu <= 0 || cus <= 0)
      return 256;
    c = static_cast<size_t>(per_cu) * static_cast<size_t>(cus);
  }
  return c;
}

template <class T>
int decode_dispatch(int rep, const DecodeArgs &a, int n_kv, int n_q, hipStream_t st) {
  switch (rep) {
    case 1: return launch_decode<1, T>(a, n_kv, n_q, st);
    case 2: return launch_decode<2, T>(a, n_kv, n_q, st);
    case 3: return launch_decode<3, T>(a, n_kv, n_q, st);
    case 4: return launch_decode<4, T>(a, n_kv, n_q, st);
    case 6: return launch_decode<6, T>(a, n_kv, n_q, st);
    case 8: return launch_decode<8, T>(a, n_kv, n_q, st);
    default: return fail(BH_ERR_ARG, "attention: no decode kernel for this grouping");
  }
}

template <bool VQ>
int launch_mq_planar(int bits, const MqArgs &m, dim3 grid, const PlanarTables &tb, hipStream_t st) {
  switch (bits) {
    case 1: BH_LAUNCH((attn_mq_planar_kernel<1, VQ>), grid, kMqThreads, 0, st, m, tb); break;
    case 2: BH_LAUNCH((attn_mq_planar_kernel<2, VQ>), grid, kMqThreads, 0, st, m, tb); break;
    case 3: BH_LAUNCH((attn_mq_planar_kernel<3, VQ>), grid, kMqThreads, 0, st, m, tb); break;
    case 4: BH_LAUNCH((attn_mq_planar_kernel<4, VQ>), grid, kMqThreads, 0, st, m, tb); break;
    case 5: BH_LAUNCH((attn_mq_planar_kernel<5, VQ>), grid, kMqThreads, 0, st, m, tb); break;
    case 6: BH_LAUNCH((attn_mq_planar_kernel<6, VQ>), grid, kMqThreads, 0, st, m, tb); break;
    case 7: BH_LAUNCH((attn_mq_planar_kernel<7, VQ>), grid, kMqThreads, 0, st, m, tb); break;
    default: BH_LAUNCH((attn_mq_planar_kernel<8, VQ>), grid, kMqThreads, 0, st, m, tb); break;
  }
  return ok();
}

bool decode_rep(size_t rep) {
  return rep == 1 || rep == 2 || rep == 3 || rep == 4 || rep == 6 || rep == 8;
}

}  // namespace
}  // namespace bh

using namespace bh;

extern "C" int bh_kv_store(const float *k, const float *v, size_t n_tok, size_t n_kv_elems,
                           void *k_cache, void *v_cache, size_t pos0, int kv_dtype,
                           bh_stream stream) {
  if (kv_dtype != BH_KV_F32 && kv_dtype != BH_KV_F16)
    return fail(BH_ERR_ARG, "kv_store: kv_dtype must be BH_KV_F32 or BH_KV_F16");
  const size_t n = n_tok * n_kv_elems;
  if (n == 0) return ok();
  if (n_kv_elems != 0 && n / n_kv_elems != n_tok) return fail(BH_ERR_SHAPE, "kv_store: size overflow");
  if (!k || !v || !k_cache || !v_cache) return fail(BH_ERR_ARG, "kv_store: null pointer");
  const size_t esz = kv_dtype == BH_KV_F16 ? 2 : 4;
  char *kc = static_cast<char *>(k_cache) + pos0 * n_kv_elems * esz;
  char *vc = static_cast<char *>(v_cache) + pos0 * n_kv_elems * esz;
  const size_t blocks = (n + kBlock - 1) / kBlock;
  if (blocks > 0x7fffffffu) return fail(BH_ERR_SHAPE, "kv_store: too many elements");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (kv_dtype == BH_KV_F16)
    BH_LAUNCH(kv_store_kernel<uint16_t>, static_cast<unsigned>(blocks), kBlock, 0, st, k, v, n,
              reinterpret_cast<uint16_t *>(kc), reinterpret_cast<uint16_t *>(vc));
  else
    BH_LAUNCH(kv_store_kernel<float>, static_cast<unsigned>(blocks), kBlock, 0, st, k, v, n,
              reinterpret_cast<float *>(kc), reinterpret_cast<float *>(vc));
  return ok();
}

extern "C" int bh_attention(const float *q, size_t n_q, size_t pos0, const void *k_cache,
                            const void *v_cache, int kv_dtype, size_t n_head, size_t n_kv,
                            size_t hd, float *out, bh_stream stream) {
  if (kv_dtype != BH_KV_F32 && kv_dtype != BH_KV_F16)
    return fail(BH_ERR_ARG, "attention: kv_dtype must be BH_KV_F32 or BH_KV_F16");
  if (n_kv == 0 || hd == 0 || n_head == 0 || n_head % n_kv != 0)
    return fail(BH_ERR_SHAPE, "attention: n_head " + std::to_string(n_head) +
                                  " must be a positive multiple of n_kv " + std::to_string(n_kv) +
                                  " and hd positive");
  if (n_q == 0) return ok();
  if (!q || !k_cache || !v_cache || !out) return fail(BH_ERR_ARG, "attention: null pointer");
  const size_t n_max = pos0 + n_q;
  if (n_head > 65535 || n_q > 65535 || n_kv > 65535 || n_max > (size_t{1} << 40) ||
      hd > (size_t{1} << 20))
    return fail(BH_ERR_SHAPE, "attention: sizes out of range");
  const size_t rep = n_head / n_kv;
  const float scale = 1.0f / sqrtf(static_cast<float>(hd));  // src/forward.rs:282
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool f16 = kv_dtype == BH_KV_F16;
  const size_t kv_stride = n_kv * hd;
  const size_t esz = f16 ? 2 : 4;

  const bool fast = hd == static_cast<size_t>(kHd) && decode_rep(rep) && aligned16(q) &&
                    (reinterpret_cast<uintptr_t>(k_cache) % (4 * esz)) == 0 &&
                    (reinterpret_cast<uintptr_t>(v_cache) % (4 * esz)) == 0;
  if (fast && n_q * rep >= static_cast<size_t>(kMqMinRows)) {
    // many queries: matrix-core path, about two blocks per CU over (chunk,
    // row tile, kv head); chunks of whole tiles
    const size_t R = n_q * rep;
    const size_t tiles_r = (R + kMqRows - 1) / kMqRows;
    if (tiles_r > 65535 || n_kv > 65535) return fail(BH_ERR_SHAPE, "attention: too many queries");
    // chunks per (row tile, kv head): the most that keep every block resident
    // in one round (a second partial round would double the time)
    const size_t cap = mq_capacity(f16);
    const size_t want = cap / (tiles_r * n_kv) > 0 ? cap / (tiles_r * n_kv) : 1;
    const size_t ptiles = (n_max + kMqTile - 1) / kMqTile;
    const size_t per = (ptiles + want - 1) / want;
    const size_t chunk = per * kMqTile;
    const size_t n_chunks = (n_max + chunk - 1) / chunk;
    if (n_chunks > 65535) return fail(BH_ERR_SHAPE, "attention: too many positions");
    size_t rows = 0, sbytes = 0;
    if (!mul_size(n_q, n_head, n_chunks, &rows) || !mul_size(rows, kHd + 2, 4, &sbytes))
      return fail(BH_ERR_SHAPE, "attention: scratch size overflows");
    float *scratch = static_cast<float *>(device_scratch(sbytes, kScratchAttention, st));
    if (scratch == nullptr) return BH_ERR_HIP;
    MqArgs m{q, k_cache, v_cache, scratch, scratch + rows, scratch + 2 * rows, pos0, kv_stride,
             chunk, static_cast<int>(n_head), static_cast<int>(n_q), static_cast<int>(rep),
             static_cast<int>(n_chunks), static_cast<int>(n_kv), scale, nullptr, nullptr,
             n_chunks == 1 ? out : nullptr};
    // 1-D grid of (chunk, kv head, row tile) in XCD-aware order (the kernel
    // decodes it)
    const size_t nb = n_chunks * n_kv * tiles_r;
    if (nb > 0x7fffffffu) return fail(BH_ERR_SHAPE, "attention: too many blocks");
    const dim3 grid(static_cast<unsigned>(nb));
    // an f32 cache read by many row tiles per kv head (a prefill) is split
    // into f16 hi / lo once instead of in every block
    const bool pre = !f16 && tiles_r >= kMqPreTiles;
    if (pre) {
      const size_t n_tiles = (n_max + kMqTile - 1) / kMqTile;
      const size_t halves = n_max * kv_stride;  // per array
      const size_t kh_b = (halves * 2 + 255) / 256 * 256;
      const size_t ks_b = (n_max * n_kv * 4 + 255) / 256 * 256;
      const size_t vt_b = n_tiles * n_kv * 2 * kHd * kMqTile * 2;  // whole tiles (rows past the end padded)
      const size_t total = 2 * kh_b + vt_b + ks_b + n_tiles * n_kv * 4;
      uint8_t *base = static_cast<uint8_t *>(device_scratch(total, kScratchKvSplit, st));
      if (base == nullptr) return BH_ERR_HIP;
      uint16_t *kh = reinterpret_cast<uint16_t *>(base);
      uint16_t *kl = reinterpret_cast<uint16_t *>(base + kh_b);
      uint16_t *vt = reinterpret_cast<uint16_t *>(base + 2 * kh_b);
      float *ks = reinterpret_cast<float *>(base + 2 * kh_b + vt_b);
      int *vsh = reinterpret_cast<int *>(base + 2 * kh_b + vt_b + ks_b);
      BH_LAUNCH(attn_kv_split_kernel, static_cast<unsigned>(n_tiles * n_kv), 256, 0, st,
                static_cast<const float *>(k_cache), static_cast<const float *>(v_cache), n_max,
                kv_stride, static_cast<int>(n_kv), kh, kl, ks, vt, vsh);
      m.kh = kh;
      m.kl = kl;
      m.vh = vt;
      m.ks = ks;
      m.vsh = vsh;
      BH_LAUNCH(attn_mq_pre_kernel, grid, kMqThreads, 0, st, m);
    } else if (f16)
      BH_LAUNCH(attn_mq_kernel<true>, grid, kMqThreads, 0, st, m);
    else
      BH_LAUNCH(attn_mq_kernel<false>, grid, kMqThreads, 0, st, m);
    if (n_chunks > 1)
      BH_LAUNCH(attn_merge_rows_kernel, static_cast<unsigned>(n_q * n_head), 256, 0, st, m.pm, m.pl,
                m.pacc, static_cast<int>(n_chunks), out);
    return ok();
  }
  if (fast) {
    // chunks of whole tiles: about 512 blocks over (chunk, kv head) for one
    // query, 2048 over (chunk, kv head, query) for several.  Measured at ctx
    // 32768, one query (f32 / f16 cache): 2048 blocks 70 / 41 us, 1024 66 /
    // 39, 512 58 / 40, 256 68 / 57 -- longer chunks amortize the block's q
    // stage and partial writes and shrink the combine; 64 queries at ctx
    // 4096: 2048 blocks 176 us, 1024 197, 4096 180.
    const size_t blocks = n_q == 1 ? 512 : 2048;
    // one query: 32-position tiles for the f32 cache (ctx 32768: 53.7 us
    // against 57.7 with 64; fewer registers), and for the f16 cache over a
    // context too short for 512 blocks of 64-position tiles (at ctx 32768
    // f16 the 64-position tiles are faster: 40.2 us against 46.7)
    const bool short_ctx = (n_max + kTile - 1) / kTile * n_kv < blocks;
    const int tile = n_q == 1 && (!f16 || short_ctx) ? 32 : kTile;
    const size_t tiles = (n_max + tile - 1) / tile;
    const size_t want = (blocks + n_kv * n_q - 1) / (n_kv * n_q);
    const size_t per = (tiles + want - 1) / want;
    const size_t chunk = per * tile;
    const size_t n_chunks = (n_max + chunk - 1) / chunk;
    if (n_chunks > 65535) return fail(BH_ERR_SHAPE, "attention: too many positions");
    const size_t rows = n_q * n_head * n_chunks;
    size_t sbytes;
    if (!mul_size(rows, kHd + 2, 4, &sbytes))
      return fail(BH_ERR_SHAPE, "attention: scratch size overflows");
    float *scratch = static_cast<float *>(device_scratch(sbytes, kScratchAttention, st));
    if (scratch == nullptr) return BH_ERR_HIP;
    DecodeArgs a{q,
                 k_cache,
                 v_cache,
                 scratch,
                 scratch + rows,
                 scratch + 2 * rows,
                 pos0,
                 kv_stride,
                 chunk,
                 static_cast<int>(n_head),
                 static_cast<int>(n_chunks),
                 scale,
                 tile};
    const int e = f16 ? decode_dispatch<uint16_t>(static_cast<int>(rep), a, static_cast<int>(n_kv),
                                                  static_cast<int>(n_q), st)
                      : decode_dispatch<float>(static_cast<int>(rep), a, static_cast<int>(n_kv),
                                               static_cast<int>(n_q), st);
    if (e) return e;
    const dim3 cgrid(static_cast<unsigned>(n_head), static_cast<unsigned>(n_q), kHd / kCombDims);
    if (n_chunks <= 32)
      BH_LAUNCH((attn_combine1_kernel<4, 8>), cgrid, 256, 0, st, a.pm, a.pl, a.pacc,
                static_cast<int>(n_chunks), out);
    else if (n_chunks <= 128)
      BH_LAUNCH((attn_combine1_kernel<16, 8>), cgrid, 1024, 0, st, a.pm, a.pl, a.pacc,
                static_cast<int>(n_chunks), out);
    else
      BH_LAUNCH(attn_combine_kernel<16>, cgrid, 1024, 0, st, a.pm, a.pl, a.pacc,
                static_cast<int>(n_chunks), kHd, out);
    return ok();
  }
  size_t pbytes;
  if (!mul_size(n_q, n_head, n_max, &pbytes) || !mul_size(pbytes, 4, &pbytes))
    return fail(BH_ERR_SHAPE, "attention: probability scratch size overflows");
  float *probs = static_cast<float *>(device_scratch(pbytes, kScratchAttention, st));
  if (probs == nullptr) return BH_ERR_HIP;
  GenericArgs a{q, k_cache, v_cache, probs, out, pos0, n_max, kv_stride, hd,
                static_cast<int>(n_head), static_cast<int>(rep), scale};
  const dim3 grid(static_cast<unsigned>(n_head), static_cast<unsigned>(n_q));
  const dim3 grid_pv(static_cast<unsigned>(n_head), static_cast<unsigned>(n_q),
                     static_cast<unsigned>((hd + kBlock - 1) / kBlock));
  if (f16) {
    BH_LAUNCH(attn_probs_kernel<uint16_t>, grid, kBlock, 0, st, a);
    BH_LAUNCH(attn_pv_kernel<uint16_t>, grid_pv, kBlock, 0, st, a);
  } else {
    BH_LAUNCH(attn_probs_kernel<float>, grid, kBlock, 0, st, a);
    BH_LAUNCH(attn_pv_kernel<float>, grid_pv, kBlock, 0, st, a);
  }
  return ok();
}

extern "C" int bh_attention_planar(const float *q, size_t n_q, size_t pos0, const uint8_t *kq,
                                   const float *kn, const uint8_t *vq, const float *vn,
                                   const float *v_f32, unsigned bits, size_t n_head, size_t n_kv,
                                   size_t hd, float *out, bh_stream stream) {
  if (bits < 1 || bits > 8) return fail(BH_ERR_ARG, "attention_planar: bits must be 1..8");
  if (n_kv == 0 || n_head == 0 || n_head % n_kv != 0)
    return fail(BH_ERR_SHAPE, "attention_planar: n_head " + std::to_string(n_head) +
                                  " must be a positive multiple of n_kv " + std::to_string(n_kv));
  if (hd != static_cast<size_t>(kPlanarHd))
    return fail(BH_ERR_SHAPE, "attention_planar: head_dim must be 256 (got " + std::to_string(hd) + ")");
  if ((vq == nullptr) != (vn == nullptr))
    return fail(BH_ERR_ARG, "attention_planar: vq and vn go together (quantized V) or are both null");
  const size_t rep = n_head / n_kv;
  if (!decode_rep(rep)) return fail(BH_ERR_ARG, "attention_planar: no kernel for this grouping");
  if (n_q == 0) return ok();
  if (!q || !kq || !kn || !out || (vq == nullptr && v_f32 == nullptr))
    return fail(BH_ERR_ARG, "attention_planar: null pointer");
  if (!aligned16(q) || (reinterpret_cast<uintptr_t>(kq) & 3u) != 0 ||
      (vq != nullptr && (reinterpret_cast<uintptr_t>(vq) & 3u) != 0) ||
      (vq == nullptr && !aligned16(v_f32)))
    return fail(BH_ERR_ARG, "attention_planar: q and v_f32 16-byte, kq and vq 4-byte aligned");
  const size_t n_max = pos0 + n_q;
  if (n_head > 65535 || n_q > 65535 || n_kv > 65535 || n_max > (size_t{1} << 40))
    return fail(BH_ERR_SHAPE, "attention_planar: sizes out of range");
  PlanarTables tb;
  if (!planar_tables(hd, bits, &tb)) return fail(BH_ERR_ARG, "attention_planar: no tables");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const float scale = 1.0f / sqrtf(static_cast<float>(hd));  // src/forward.rs:282
  if (n_q * rep >= static_cast<size_t>(kMqMinRows)) {
    // many queries: the matrix-core path with planar staging, chunked as
    // bh_attention's
    const size_t R = n_q * rep;
    const size_t tiles_r = (R + kMqRows - 1) / kMqRows;
    if (tiles_r > 65535) return fail(BH_ERR_SHAPE, "attention_planar: too many queries");
    const size_t cap = mq_capacity(false);
    const size_t want = cap / (tiles_r * n_kv) > 0 ? cap / (tiles_r * n_kv) : 1;
    const size_t ptiles = (n_max + kMqTile - 1) / kMqTile;
    const size_t per = (ptiles + want - 1) / want;
    const size_t chunk = per * kMqTile;
    const size_t n_chunks = (n_max + chunk - 1) / chunk;
    if (n_chunks > 65535) return fail(BH_ERR_SHAPE, "attention_planar: too many positions");
    size_t rows = 0, sbytes = 0;
    if (!mul_size(n_q, n_head, n_chunks, &rows) || !mul_size(rows, kHd + 2, 4, &sbytes))
      return fail(BH_ERR_SHAPE, "attention_planar: scratch size overflows");
    float *scratch = static_cast<float *>(device_scratch(sbytes, kScratchAttention, st));
    if (scratch == nullptr) return BH_ERR_HIP;
    MqArgs m{q, kq, vq != nullptr ? static_cast<const void *>(vq) : static_cast<const void *>(v_f32),
             scratch, scratch + rows, scratch + 2 * rows, pos0, n_kv * kHd, chunk,
             static_cast<int>(n_head), static_cast<int>(n_q), static_cast<int>(rep),
             static_cast<int>(n_chunks), static_cast<int>(n_kv), scale, kn, vn, nullptr};
    const size_t nb = n_chunks * n_kv * tiles_r;
    if (nb > 0x7fffffffu) return fail(BH_ERR_SHAPE, "attention_planar: too many blocks");
    const int e = vq != nullptr ? launch_mq_planar<true>(static_cast<int>(bits), m, dim3(static_cast<unsigned>(nb)), tb, st)
                                : launch_mq_planar<false>(static_cast<int>(bits), m, dim3(static_cast<unsigned>(nb)), tb, st);
    if (e) return e;
    if (vq != nullptr)
      BH_LAUNCH(attn_merge_rows_rot_kernel, static_cast<unsigned>(n_q * n_head), 256, 0, st, m.pm, m.pl,
                m.pacc, static_cast<int>(n_chunks), out, tb);
    else
      BH_LAUNCH(attn_merge_rows_kernel, static_cast<unsigned>(n_q * n_head), 256, 0, st, m.pm, m.pl,
                m.pacc, static_cast<int>(n_chunks), out);
    return ok();
  }
  // chunks of whole tiles: about 512 blocks for one query, 2048 for several,
  // and at most 128 chunks (the one-round-trip merge)
  const size_t blocks = n_q == 1 ? 512 : 2048;
  const size_t tiles = (n_max + kPlTile - 1) / kPlTile;
  size_t want = (blocks + n_kv * n_q - 1) / (n_kv * n_q);
  want = want < 128 ? want : 128;
  const size_t per = (tiles + want - 1) / want;
  const size_t chunk = per * kPlTile;
  const size_t n_chunks = (n_max + chunk - 1) / chunk;
  size_t rows = 0, sbytes = 0;
  if (!mul_size(n_q, n_head, n_chunks, &rows) || !mul_size(rows, kHd + 2, 4, &sbytes))
    return fail(BH_ERR_SHAPE, "attention_planar: scratch size overflows");
  float *scratch = static_cast<float *>(device_scratch(sbytes, kScratchAttention, st));
  if (scratch == nullptr) return BH_ERR_HIP;
  PlanarArgs a{q,       kq,   kn,    vq, vn, v_f32, scratch, scratch + rows, scratch + 2 * rows,
               pos0,    chunk, static_cast<int>(n_head), static_cast<int>(n_chunks),
               static_cast<int>(n_kv), static_cast<int>(bits), scale};
  const dim3 grid(static_cast<unsigned>(n_chunks), static_cast<unsigned>(n_kv), static_cast<unsigned>(n_q));
  int e = BH_OK;
  switch (rep) {
    case 1: e = launch_planar<1>(a, grid, tb, st); break;
    case 2: e = launch_planar<2>(a, grid, tb, st); break;
    case 3: e = launch_planar<3>(a, grid, tb, st); break;
    case 4: e = launch_planar<4>(a, grid, tb, st); break;
    case 6: e = launch_planar<6>(a, grid, tb, st); break;
    default: e = launch_planar<8>(a, grid, tb, st); break;
  }
  if (e) return e;
  const dim3 cgrid(static_cast<unsigned>(n_head), static_cast<unsigned>(n_q), kHd / kCombDims);
  const int nc = static_cast<int>(n_chunks);
  if (vq != nullptr) {
    if (n_chunks <= 32)
      BH_LAUNCH((attn_combine1_rot_kernel<4, 8>), cgrid, 256, 0, st, a.pm, a.pl, a.pacc, nc, out, tb);
    else
      BH_LAUNCH((attn_combine1_rot_kernel<16, 8>), cgrid, 1024, 0, st, a.pm, a.pl, a.pacc, nc, out, tb);
  } else {
    if (n_chunks <= 32)
      BH_LAUNCH((attn_combine1_kernel<4, 8>), cgrid, 256, 0, st, a.pm, a.pl, a.pacc, nc, out);
    else
      BH_LAUNCH((attn_combine1_kernel<16, 8>), cgrid, 1024, 0, st, a.pm, a.pl, a.pacc, nc, out);
  }
  return ok();
}
