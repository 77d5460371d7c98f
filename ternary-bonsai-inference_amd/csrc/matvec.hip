// PQ2_0 matrix-vector and N-column matrix products on the gfx950 matrix cores.
//
// Reference: kernels::pq2_matvec_range (src/kernels.rs:283-333) and
// kernels::pq2_matmul_n (src/kernels.rs:340-423): Y[t][r] = sum_j X[t][j] *
// W[base_row + r][j], where row r of W is ceil(ne0/128) 34-byte blocks (f16
// scale + 32 bytes of 2-bit codes, weight = (code - 1) * scale).  The scalar
// reference row dot (src/kernels.rs:633-653) sums each 128-block in f32 and
// adds scale * block_sum to the row total; its AVX2 path reorders the same
// sums (~1e-6 relative).  This file computes the same per-block structure
// with MFMA tiles, in a different summation order (max relative difference
// well below 1e-5 of the output's largest magnitude).
//
// Mapping onto v_mfma_f32_16x16x32_f16 (D = A * B + C, 16x16 output tile;
// lane l holds A[l % 16][8 (l / 16) .. +7], B[8 (l / 16) .. +7][l % 16],
// D[4 (l / 16) .. +3][l % 16]):
//   M (A rows)    = tokens, 16 per tile (padded with zero tokens);
//   N (B columns) = weight rows, 16 per tile;
//   K             = columns of one 128-weight block, 4 MFMA steps of 32.
// B fragments hold the codes themselves (0..3, exact in f16): a 2-bit code
// in the low bits of a nibble reads as the FP4 (e2m1) value code / 2, so
// with the codes spread one per nibble one packed FP4 -> f16 conversion
// (scale 2) decodes two weights; sum(x * (code - 1)) is then the MFMA's
// sum(x * code) minus the block's sum(x), precomputed per (token, block).
// The x side needs more than f16's 11 bits for a 1e-5 result, so each
// (token, 128-block) of x is scaled by a power of two (its largest |x| in
// [2^14, 2^15)) and split into hi = f16(x') and lo = f16(x' - hi): hi + lo
// carries 22 significant bits, and two MFMAs (hi, lo) per weight tile
// accumulate it in f32.  Each block's f32 tile sum is then multiplied by the
// block's f32 scale times 2^-e (exact) and added to the row total, as the
// reference adds scale * block_sum.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>

#include "common.hpp"

namespace bh {
namespace {

constexpr int kPq2Blk = 34;
constexpr int kMmThreads = 256;  // 4 waves
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4v __attribute__((ext_vector_type(4)));

// Workgroup barrier for LDS traffic only: waits for this wave's LDS
// operations, not for its global loads, so weight and fragment prefetches
// stay in flight across it (__syncthreads() would also drain them).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Block column (0..127) of element e (0..7) of lane group g's A/B fragment
// in MFMA step i (0..3) of a block.  Lane group g owns code bytes [8g, 8g+8)
// of the block (columns [32g, 32g + 32)); step i uses the dword of code bytes
// 8g + 4 (i >> 1) .. +3, spread one code per nibble (the codes of parity
// i & 1), and element e is code 2 (e & 1) + (i & 1) of byte e >> 1.  The MFMA
// sums its k-slots in any order, so only A and B have to agree.
__host__ __device__ constexpr int mm_column(int i, int g, int e) {
  return 32 * g + 16 * (i >> 1) + 4 * (e >> 1) + 2 * (e & 1) + (i & 1);
}

// ---------------------------------------------------------------------------
// Prepare: the hi/lo f16 A fragments, with a power of two per (token,
// 128-block) chosen so the block's largest |x| lands in [2^14, 2^15): hi
// never overflows f16 and lo keeps 11 more bits.  The power of two comes
// back out in the product kernel's per-block f32 step (exact).
//   afrag: [tile][kstep][piece (hi, lo)][64 lanes] x 16 bytes, written only
//          for real tokens (the lanes of absent tokens feed rows that are
//          never stored);
//   binv:  [tile][block][lane group g] two float4: 2^-e and sum(hi + lo) of
//          tokens 4g .. 4g+3.
// ---------------------------------------------------------------------------
struct PrepArgs {
  const float *x;  // [n_tok][ne0]
  uint4 *afrag;
  float *binv;
  int ne0, n_tok, nblk, n_ksteps;
};

// 16 consecutive lanes per (token, block); lane (i, g) builds the hi/lo
// fragments of MFMA step i, lane group g (8 columns).  The block's largest
// |x| and its sum of hi + lo are reduced across the 16 lanes.
__global__ __launch_bounds__(kMmThreads) void pq2_mm_prep_kernel(PrepArgs a) {
  const int item = blockIdx.x * kMmThreads + threadIdx.x;
  const int mb = item >> 4, sub = item & 15;  // the 16 lanes of a group share mb
  const bool live = mb < a.n_tok * a.nblk;
  const int m = live ? mb / a.nblk : 0, blk = live ? mb - m * a.nblk : 0;
  const int i = sub >> 2, g = sub & 3;
  const float *xr = a.x + static_cast<size_t>(m) * a.ne0 + 128 * blk;
  float f[8];
  float mx = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    f[e] = live ? xr[mm_column(i, g, e)] : 0.0f;
    mx = fmaxf(mx, fabsf(f[e]));  // NaN is ignored
  }
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
  int ex = 0;  // an all-zero or non-finite block keeps 2^0
  if (mx > 0.0f && mx <= 3.4e38f) {
    int k;
    (void)frexpf(mx, &k);  // mx = f * 2^k, f in [0.5, 1): mx * 2^(15-k) in [2^14, 2^15)
    ex = 15 - k;
    ex = ex < -126 ? -126 : (ex > 126 ? 126 : ex);  // 2^e and 2^-e stay normal f32
  }
  const float s = ldexpf(1.0f, ex);
  h8 hi, lo;
  float bsum = 0.0f;  // sum of hi + lo over the block (the "- 1" of the fp4 decode)
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float v = f[e] * s;
    const _Float16 hv = static_cast<_Float16>(v);
    hi[e] = hv;
    // an infinite x keeps lo = 0 (inf - inf would turn the term into NaN)
    lo[e] = __builtin_isinf(static_cast<float>(hv)) ? static_cast<_Float16>(0.0f)
                                                   : static_cast<_Float16>(v - static_cast<float>(hv));
    bsum += static_cast<float>(hi[e]) + static_cast<float>(lo[e]);
  }
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) bsum += __shfl_xor(bsum, off, 64);
  if (!live) return;
  const int tile = m >> 4, ml = m & 15;
  uint4 *dst = a.afrag + (static_cast<size_t>(tile) * a.n_ksteps + 4 * blk + i) * 2 * 64 + 16 * g + ml;
  dst[0] = __builtin_bit_cast(uint4, hi);
  dst[64] = __builtin_bit_cast(uint4, lo);
  if (sub == 0) {
    // block factors: [tile][block][token group][inv, sum] x float4 (token & 3)
    float *bx = a.binv + (((static_cast<size_t>(tile) * a.nblk + blk) * 4 + (ml >> 2)) * 2) * 4 + (ml & 3);
    bx[0] = ldexpf(1.0f, -ex);
    bx[4] = bsum;
  }
}

// ---------------------------------------------------------------------------
// Main product.  Block = 4 waves; a wave owns NT 16-row weight tiles and the
// block's MT token tiles.  Lane l: row n = l & 15 of each weight tile, lane
// group g = l >> 4 (code bytes 8g..8g+7 of every block).
//
// Weights are read two blocks (68 bytes, 17 dwords) at a time: with 4-byte
// aligned rows the pair starts on a dword, its odd block's codes are
// dword-aligned and its even block's are 2 bytes off, so every lane reads
// whole dwords inside the pair (dwordx3 + dwordx2 + the two scale dwords)
// and realigns with a funnel shift -- no read ever leaves the pair.
// ---------------------------------------------------------------------------
struct MmArgs {
  const uint8_t *w;    // first row of the range (payload + base_row * row_bytes)
  const uint4 *afrag;
  const float4 *binv;
  float *y;            // [n_tok][y_stride]
  size_t row_bytes;
  int n_rows, nblk, n_ksteps, n_tok, y_stride;
};

// B fragment of step i from its code dword d as the codes themselves (0..3,
// exact f16): a 2-bit code in the low bits of a nibble reads as the FP4
// (e2m1) value code / 2, so with the codes spread one per nibble a packed
// FP4 -> f16 conversion scaled by 2 yields two codes per instruction.  The
// missing "- 1" of (code - 1) is applied per block as - sum(x).
__device__ __forceinline__ h8 decode_fp4(uint32_t d, int i) {
  const uint32_t t = (i & 1) ? ((d >> 2) & 0x33333333u) : (d & 0x33333333u);
  const h2 p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(t, 2.0f, 0);
  const h2 p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(t, 2.0f, 1);
  const h2 p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(t, 2.0f, 2);
  const h2 p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(t, 2.0f, 3);
  return h8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

struct PairData {
  uint32_t e0, e1, e2;  // pair dwords 2g .. 2g+2 (even block's codes, 2 bytes in)
  uint32_t o0, o1;      // pair dwords 9+2g, 10+2g (odd block's codes)
  uint32_t s0, s8;      // pair dwords 0 and 8 (the two f16 scales)
};

__device__ __forceinline__ PairData load_pair(const uint32_t *rp, int g) {
  PairData d;
  const uint3 e = *reinterpret_cast<const uint3 *>(rp + 2 * g);
  const uint2 o = *reinterpret_cast<const uint2 *>(rp + 9 + 2 * g);
  d.e0 = e.x;
  d.e1 = e.y;
  d.e2 = e.z;
  d.o0 = o.x;
  d.o1 = o.y;
  d.s0 = rp[0];
  d.s8 = rp[8];
  return d;
}

// Codes and scale of one block of a pair, ready for the MFMA steps.
struct BlockCodes {
  uint32_t cd[2];  // code bytes 8g..8g+3, 8g+4..8g+7
  float sc;
};

__device__ __forceinline__ BlockCodes block_codes(const PairData &d, int half) {
  BlockCodes c;
  if (half == 0) {
    c.cd[0] = __builtin_amdgcn_alignbyte(d.e1, d.e0, 2);
    c.cd[1] = __builtin_amdgcn_alignbyte(d.e2, d.e1, 2);
    c.sc = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(d.s0)));
  } else {
    c.cd[0] = d.o0;
    c.cd[1] = d.o1;
    c.sc = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(d.s8 >> 16)));
  }
  return c;
}

template <int MT, int NT, bool ALDS>
__global__ __launch_bounds__(kMmThreads) void pq2_mm_kernel(MmArgs a) {
  // ALDS (one token tile of at most kLdsTok tokens): the x side of the whole
  // product is staged in LDS once, fragments [kstep][piece][token][lane
  // group] followed by the block factors [block][lane group]
  extern __shared__ uint4 a_lds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int row_wave = blockIdx.x * (4 * 16 * NT) + wave * 16 * NT;
  const int tile0 = blockIdx.y * MT;

  const uint32_t *wp[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int row = row_wave + 16 * t + n;
    row = row < a.n_rows ? row : a.n_rows - 1;  // tail rows read a valid row, store nothing
    wp[t] = reinterpret_cast<const uint32_t *>(a.w + static_cast<size_t>(row) * a.row_bytes);
  }
  // Row m of an MFMA result depends on row m of A only, so the lanes of a
  // tile's absent tokens may feed any fragment (their rows are never
  // stored): they read a real token's (ALDS) or unwritten scratch.
  const uint4 *af = a.afrag + static_cast<size_t>(tile0) * a.n_ksteps * 2 * 64 + lane;
  const float4 *binv_g = a.binv + (static_cast<size_t>(tile0) * a.nblk * 4 + g) * 2;
  const uint4 *al = a_lds;
  const float4 *binv_l = nullptr;
  int lds_tok_stride = 0;
  if constexpr (ALDS) {
    const int nt = a.n_tok;  // <= kLdsTok: tile 0 only
    const int total = a.n_ksteps * 2 * nt * 4;
    for (int i = threadIdx.x; i < total; i += kMmThreads) {
      const int gq = i & 3, rest = i >> 2;
      const int m = rest % nt, kp = rest / nt;  // kp = 2 * kstep + piece
      a_lds[i] = a.afrag[static_cast<size_t>(kp) * 64 + 16 * gq + m];
    }
    float4 *bl = reinterpret_cast<float4 *>(a_lds + total);
    for (int i = threadIdx.x; i < a.nblk * 8; i += kMmThreads) bl[i] = a.binv[i];
    al = a_lds + (n < nt ? n : 0) * 4 + g;
    lds_tok_stride = nt * 4;
    binv_l = bl + 2 * g;
  }
  if constexpr (ALDS) __syncthreads();  // x staging visible to every wave

  f4v tot[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < NT; ++t) tot[mt][t] = f4v{0.f, 0.f, 0.f, 0.f};

  auto do_block = [&](const BlockCodes(&bc)[NT], int b) {
    f4v acc[MT][NT], acc_lo[MT][NT];  // hi and lo pieces: two independent MFMA chains
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[mt][t] = acc_lo[mt][t] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ks = 4 * b + i;
      h8 ahi[MT], alo[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if constexpr (ALDS) {
          const uint4 *pl = al + (2 * ks) * lds_tok_stride;
          ahi[mt] = __builtin_bit_cast(h8, pl[0]);
          alo[mt] = __builtin_bit_cast(h8, pl[lds_tok_stride]);
        } else {
          const uint4 *pg = af + (static_cast<size_t>(mt) * a.n_ksteps + ks) * 2 * 64;
          ahi[mt] = __builtin_bit_cast(h8, pg[0]);
          alo[mt] = __builtin_bit_cast(h8, pg[64]);
        }
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint32_t d = bc[t].cd[i >> 1];
        const h8 bf = decode_fp4(d, i);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[mt], bf, acc[mt][t], 0, 0, 0);
          acc_lo[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[mt], bf, acc_lo[mt][t], 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[mt][t][q] = acc[mt][t][q] + acc_lo[mt][t][q];
    // src/kernels.rs:651: acc += scale * block_acc -- block_acc arrives
    // multiplied by the block's 2^e, so the factor is scale * 2^-e (exact)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float4 bi, bs;
      if constexpr (ALDS) {
        bi = binv_l[b * 8];
        bs = binv_l[b * 8 + 1];
      } else {
        bi = binv_g[(static_cast<size_t>(mt) * a.nblk + b) * 8];
        bs = binv_g[(static_cast<size_t>(mt) * a.nblk + b) * 8 + 1];
      }
      const float inv[4] = {bi.x, bi.y, bi.z, bi.w};
      const float xs[4] = {bs.x, bs.y, bs.z, bs.w};
#pragma unroll
      for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float f = bc[t].sc * inv[q];
          const float blk = acc[mt][t][q] - xs[q];
          const float prod = f * blk;
          tot[mt][t][q] = tot[mt][t][q] + prod;
        }
      }
    }
  };

  // weight pairs stream two deep: pair p + 2 is requested while pair p runs
  const int npairs = a.nblk >> 1;
  PairData pa[NT], pb[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    pa[t] = load_pair(wp[t], g);
    if (npairs > 1) pb[t] = load_pair(wp[t] + 17, g);
  }
  auto run_pair = [&](PairData(&buf)[NT], int p) {
    BlockCodes b0[NT], b1[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      b0[t] = block_codes(buf[t], 0);
      b1[t] = block_codes(buf[t], 1);
    }
    if (p + 2 < npairs) {
#pragma unroll
      for (int t = 0; t < NT; ++t) buf[t] = load_pair(wp[t] + 17 * (p + 2), g);
    }
    do_block(b0, 2 * p);
    do_block(b1, 2 * p + 1);
  };
  for (int p = 0; p < npairs; p += 2) {
    run_pair(pa, p);
    if (p + 1 < npairs) run_pair(pb, p + 1);
  }

  // lane holds tokens 4g..4g+3 of each token tile, row n of each weight tile
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int m = 16 * (tile0 + mt) + 4 * g + q;
      if (m >= a.n_tok) continue;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int row = row_wave + 16 * t + n;
        if (row < a.n_rows) a.y[static_cast<size_t>(m) * a.y_stride + row] = tot[mt][t][q];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Staged product (16-byte aligned rows, block count a multiple of 8): each
// wave streams its 16 rows through LDS in chunks of 8 blocks (272 bytes per
// row, 17 dwordx4 loads per row, so consecutive lanes read consecutive 16
// bytes of a row), then every lane reads its fragment codes from LDS.  One
// chunk is in flight in registers while the previous one is consumed; the
// stage is private to the wave (in-order LDS, no block barrier).
// ---------------------------------------------------------------------------
constexpr int kStageBlocks = 8;
constexpr int kStageRowBytes = kPq2Blk * kStageBlocks;          // 272
constexpr int kStageStride = 280;  // LDS bytes per staged row: 8-aligned, spreads the banks
constexpr int kStageF4 = kStageRowBytes / 16;                   // 17
constexpr int kStageLoads = (16 * kStageF4 + 63) / 64;          // 5 per lane
constexpr size_t kStageWaveBytes = 16 * kStageStride;           // 4480

__device__ __forceinline__ uint32_t lds_u32(const uint8_t *p) {
  return *reinterpret_cast<const uint32_t *>(p);
}

// TOKQ: accumulator elements per lane that can hold a real token (the tile
// has at most 4 * TOKQ ... lanes of groups g >= 1 hold tokens >= 4, so with
// n_tok <= TOKQ only elements q < TOKQ of group 0 carry results).
template <bool ALDS, int TOKQ>
__global__ __launch_bounds__(kMmThreads) void pq2_mm_staged_kernel(MmArgs a) {
  extern __shared__ uint4 smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int row_wave = blockIdx.x * 64 + wave * 16;

  // x side: whole product in LDS (ALDS) or fragments from global
  const uint4 *af = a.afrag + lane;
  const uint4 *al = smem;
  const float4 *binv_l = nullptr;
  int lds_tok_stride = 0;
  size_t a_words = 0;  // uint4 slots used by the ALDS area
  if constexpr (ALDS) {
    const int nt = a.n_tok;
    const int total = a.n_ksteps * 2 * nt * 4;
    for (int i = threadIdx.x; i < total; i += kMmThreads) {
      const int gq = i & 3, rest = i >> 2;
      const int m = rest % nt, kp = rest / nt;
      smem[i] = a.afrag[static_cast<size_t>(kp) * 64 + 16 * gq + m];
    }
    float4 *bl = reinterpret_cast<float4 *>(smem + total);
    for (int i = threadIdx.x; i < a.nblk * 8; i += kMmThreads) bl[i] = a.binv[i];
    al = smem + (n < nt ? n : 0) * 4 + g;
    lds_tok_stride = nt * 4;
    binv_l = bl + 2 * g;
    a_words = static_cast<size_t>(total) + static_cast<size_t>(a.nblk) * 8;
  }
  uint8_t *stage = reinterpret_cast<uint8_t *>(smem + a_words) + wave * kStageWaveBytes;

  // this lane's share of a chunk: float4 slot k covers row r_k, piece c_k
  const uint8_t *src[kStageLoads];
  int dst[kStageLoads];
  bool live[kStageLoads];
#pragma unroll
  for (int k = 0; k < kStageLoads; ++k) {
    const int idx = lane + 64 * k;
    live[k] = idx < 16 * kStageF4;
    const int r = live[k] ? idx / kStageF4 : 0, c16 = live[k] ? idx % kStageF4 : 0;
    int row = row_wave + r;
    row = row < a.n_rows ? row : a.n_rows - 1;  // tail rows read a valid row, store nothing
    src[k] = a.w + static_cast<size_t>(row) * a.row_bytes + 16 * c16;
    dst[k] = r * kStageStride + 16 * c16;
  }
  uint4 regs[kStageLoads];
  auto gload = [&](int chunk) {
#pragma unroll
    for (int k = 0; k < kStageLoads; ++k)
      if (live[k]) regs[k] = *reinterpret_cast<const uint4 *>(src[k] + static_cast<size_t>(chunk) * kStageRowBytes);
  };
  auto lstore = [&]() {
#pragma unroll
    for (int k = 0; k < kStageLoads; ++k) {
      if (live[k]) {
        uint2 *d = reinterpret_cast<uint2 *>(stage + dst[k]);  // 8-byte aligned
        d[0] = make_uint2(regs[k].x, regs[k].y);
        d[1] = make_uint2(regs[k].z, regs[k].w);
      }
    }
  };
  f4v tot = f4v{0.f, 0.f, 0.f, 0.f};

  const int n_chunks = a.nblk / kStageBlocks;
  gload(0);
  if constexpr (ALDS) __syncthreads();  // x staging visible to every wave
  lstore();
  if (n_chunks > 1) gload(1);
  for (int c = 0; c < n_chunks; ++c) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint8_t *rowp = stage + n * kStageStride;
    for (int bb = 0; bb < kStageBlocks; ++bb) {
      const int b = c * kStageBlocks + bb;
      const uint8_t *blk = rowp + kPq2Blk * bb;
      BlockCodes bc;
      if ((bb & 1) == 0) {  // block starts on a dword: codes are 2 bytes in
        const uint32_t e0 = lds_u32(blk + 8 * g), e1 = lds_u32(blk + 8 * g + 4),
                       e2 = lds_u32(blk + 8 * g + 8);
        bc.cd[0] = __builtin_amdgcn_alignbyte(e1, e0, 2);
        bc.cd[1] = __builtin_amdgcn_alignbyte(e2, e1, 2);
        bc.sc = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(lds_u32(blk))));
      } else {  // block starts 2 bytes into a dword: codes are dword-aligned
        bc.cd[0] = lds_u32(blk + 2 + 8 * g);
        bc.cd[1] = lds_u32(blk + 6 + 8 * g);
        bc.sc = static_cast<float>(
            __builtin_bit_cast(_Float16, static_cast<uint16_t>(lds_u32(blk - 2) >> 16)));
      }
      f4v acc = f4v{0.f, 0.f, 0.f, 0.f}, acc_lo = acc;  // two independent MFMA chains
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ks = 4 * b + i;
        h8 ahi, alo;
        if constexpr (ALDS) {
          const uint4 *pl = al + (2 * ks) * lds_tok_stride;
          ahi = __builtin_bit_cast(h8, pl[0]);
          alo = __builtin_bit_cast(h8, pl[lds_tok_stride]);
        } else {
          const uint4 *pg = af + static_cast<size_t>(ks) * 2 * 64;
          ahi = __builtin_bit_cast(h8, pg[0]);
          alo = __builtin_bit_cast(h8, pg[64]);
        }
        const uint32_t d = bc.cd[i >> 1];
        const h8 bf = decode_fp4(d, i);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi, bf, acc, 0, 0, 0);
        acc_lo = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo, bf, acc_lo, 0, 0, 0);
      }
#pragma unroll
      for (int q = 0; q < TOKQ; ++q) acc[q] = acc[q] + acc_lo[q];
      float4 bi, bs;
      if constexpr (ALDS) {
        bi = binv_l[b * 8];
        bs = binv_l[b * 8 + 1];
      } else {
        bi = a.binv[(static_cast<size_t>(b) * 4 + g) * 2];
        bs = a.binv[(static_cast<size_t>(b) * 4 + g) * 2 + 1];
      }
      const float inv[4] = {bi.x, bi.y, bi.z, bi.w};
      const float xs[4] = {bs.x, bs.y, bs.z, bs.w};
#pragma unroll
      for (int q = 0; q < TOKQ; ++q) {
        const float f = bc.sc * inv[q];  // src/kernels.rs:651, block scale * 2^-e
        const float blk = acc[q] - xs[q];
        const float prod = f * blk;
        tot[q] = tot[q] + prod;
      }
    }
    if (c + 1 < n_chunks) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      lstore();  // chunk c + 1 replaces chunk c (this wave finished reading it)
      if (c + 2 < n_chunks) gload(c + 2);
    }
  }
#pragma unroll
  for (int q = 0; q < TOKQ; ++q) {
    const int m = 4 * g + q;
    const int row = row_wave + n;
    if (m < a.n_tok && row < a.n_rows) a.y[static_cast<size_t>(m) * a.y_stride + row] = tot[q];
  }
}

// ---------------------------------------------------------------------------
// Integer product for the staged shapes (16-byte aligned rows, block count a
// multiple of 8, at most kI8Tok tokens per token group).
//
// x side: each (token, 128-block) is scaled by the power of two 2^e that
// puts its largest |x| in [2^21, 2^22) and rounded to integers X (22
// significant bits), written as three signed base-256 digits
// X = 65536 d0 + 256 d1 + d2 (|d0| <= 65, |d1|, |d2| <= 128).  The codes
// (0..3) are exact int8, so one v_mfma_i32_16x16x64_i8 step sums
// code * digit exactly in i32; a block is two steps.  The three digits of a
// token are three A rows of the same MFMA (A row m = 4 * token + digit, the
// fourth row of each token unused), so one decode of the codes serves every
// digit and up to 4 tokens, and lane (n, g) ends the block holding token
// g's three digit sums for weight row n.  Then
//     sum_j X_j (code_j - 1) = 65536 S0 + 256 S1 + S2 - sum_j X_j
// exactly (|value| <= 2^30, i32 arithmetic, the wrap of the partial terms
// cancels), converted to f32 once, multiplied by 2^-e (exact) and
// accumulated as the reference adds scale * block_sum (src/kernels.rs:651).
//
// Codes: a dword holds codes c0..c15 (2 bits each, c0 lowest).  Bytes
// (w >> 2k) & 0x03030303 are c_k, c_{4+k}, c_{8+k}, c_{12+k}: fragment dword
// k, byte i carries code 4i + k.  The x digits are laid out in the same
// slot order, so the MFMA pairs x_j with code_j.
// ---------------------------------------------------------------------------
constexpr int kI8Tok = 4;  // tokens per MFMA (A rows 4t .. 4t + 3)
typedef int i4v __attribute__((ext_vector_type(4)));


// The digit fragments of one (token, 128-block): its 8 lanes (sub = 2g + h)
// each build the three 16-byte fragments (digits d0, d1, d2) of step 2 blk + h
// for lane group g, block columns 16 (2g + h) .. +15, from xb = x + t * ne0 +
// 128 * blk; every lane of the 8 gets the block factor (bits of sum X,
// 2^-e; NaN when the block holds a NaN or infinity).  Contains cross-lane
// steps inside each 8-lane group: all lanes of the wave must call it
// (dead items with live = false).
__device__ __forceinline__ void i8_prep_item(const float *xb, int sub, bool live, uint4 frag[3],
                                             float2 &fac) {
  const int g = sub >> 1, h = sub & 1;
  const float4 *xr = reinterpret_cast<const float4 *>(xb + 16 * (2 * g + h));
  float f[16];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 v = live ? xr[q] : make_float4(0.f, 0.f, 0.f, 0.f);
    f[4 * q] = v.x;
    f[4 * q + 1] = v.y;
    f[4 * q + 2] = v.z;
    f[4 * q + 3] = v.w;
  }
  float mx = 0.0f;
  int bad = 0;  // a NaN or infinity in the block
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    const bool fin = __builtin_isfinite(f[c]);
    bad |= !fin;
    f[c] = fin ? f[c] : 0.0f;
    mx = fmaxf(mx, fabsf(f[c]));
  }
#pragma unroll
  for (int off = 4; off > 0; off >>= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    bad |= __shfl_xor(bad, off, 64);
  }
  int ex = 0;
  if (mx > 0.0f) {
    int k;
    (void)frexpf(mx, &k);  // mx = f * 2^k, f in [0.5, 1): mx * 2^(22-k) in [2^21, 2^22)
    ex = 22 - k;
    ex = ex > 126 ? 126 : ex;  // tiny blocks round toward zero; 2^-e stays normal
  }
  const float s = ldexpf(1.0f, ex);
  uint32_t dg[3][4] = {};
  int sx = 0;
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    const int X = static_cast<int>(rintf(f[c] * s));  // |X| <= 2^22
    sx += X;
    const int d2 = ((X + 128) & 0xff) - 128;
    const int x1 = (X - d2) >> 8;
    const int d1 = ((x1 + 128) & 0xff) - 128;
    const int d0 = (x1 - d1) >> 8;
    const int k = c & 3, i = c >> 2;  // dword k, byte i holds column 4i + k
    dg[0][k] |= (static_cast<uint32_t>(d0) & 0xffu) << (8 * i);
    dg[1][k] |= (static_cast<uint32_t>(d1) & 0xffu) << (8 * i);
    dg[2][k] |= (static_cast<uint32_t>(d2) & 0xffu) << (8 * i);
  }
#pragma unroll
  for (int off = 4; off > 0; off >>= 1) sx += __shfl_xor(sx, off, 64);
#pragma unroll
  for (int d = 0; d < 3; ++d) frag[d] = make_uint4(dg[d][0], dg[d][1], dg[d][2], dg[d][3]);
  fac = make_float2(__int_as_float(sx), bad ? __builtin_nanf("") : ldexpf(1.0f, -ex));
}

struct MmI8Args {
  const uint8_t *w;     // first row of the range
  const float *x;       // [n_tok][ne0], n_tok <= kI8Tok
  float *y;             // [n_tok][y_stride]
  size_t row_bytes;
  int n_rows, nblk, n_tok, y_stride;
};

__device__ __forceinline__ i4v decode_i8(uint32_t d) {
  return i4v{static_cast<int>(d & 0x03030303u), static_cast<int>((d >> 2) & 0x03030303u),
             static_cast<int>((d >> 4) & 0x03030303u), static_cast<int>((d >> 6) & 0x03030303u)};
}

// x digits of every (token, block) into LDS, by all `lanes` lanes of the
// workgroup: uint4 (step * 4 + g) * arows + 4 t + digit, block factors at
// bf[blk * kI8Tok + t].  The trip count is the same for every wave (the
// prep has cross-lane steps).
__device__ __forceinline__ void i8_stage_x(const MmI8Args &a, uint4 *smem, float2 *bf, int arows,
                                           int lanes) {
  const int n_items = a.n_tok * a.nblk * 8;
  for (int base = 0; base < n_items; base += lanes) {
    const int item = base + static_cast<int>(threadIdx.x);
    const bool live_item = item < n_items;
    const int tb = item >> 3, sub = item & 7;
    const int t = live_item ? tb / a.nblk : 0, blk = live_item ? tb - t * a.nblk : 0;
    uint4 frag[3];
    float2 fac;
    i8_prep_item(a.x + static_cast<size_t>(t) * (128 * a.nblk) + 128 * blk, sub, live_item, frag,
                 fac);
    if (live_item) {
      const int step = 2 * blk + (sub & 1), gg = sub >> 1;
      uint4 *dst = smem + (step * 4 + gg) * arows + 4 * t;
      dst[0] = frag[0];
      dst[1] = frag[1];
      dst[2] = frag[2];
      if (sub == 0) bf[blk * kI8Tok + t] = fac;
    }
  }
}

// One 8-block chunk of a wave's 16-row tile from its LDS stage into the
// row total `tot` (blocks b0 .. b0 + 7 of the row).
__device__ __forceinline__ float i8_chunk(const uint8_t *stage, const uint4 *al, const float2 *bl,
                                          int arows, int n, int g, int b0, float tot) {
  const uint8_t *rowp = stage + n * kStageStride;
#pragma unroll 2
  for (int bb = 0; bb < kStageBlocks; ++bb) {
    const int b = b0 + bb;
    const uint8_t *blk = rowp + kPq2Blk * bb;
    uint32_t cd0, cd1;
    float sc;
    if ((bb & 1) == 0) {  // block starts on a dword: codes are 2 bytes in
      const uint32_t e0 = lds_u32(blk + 8 * g), e1 = lds_u32(blk + 8 * g + 4),
                     e2 = lds_u32(blk + 8 * g + 8);
      cd0 = __builtin_amdgcn_alignbyte(e1, e0, 2);
      cd1 = __builtin_amdgcn_alignbyte(e2, e1, 2);
      sc = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(lds_u32(blk))));
    } else {  // block starts 2 bytes into a dword: codes are dword-aligned
      cd0 = lds_u32(blk + 2 + 8 * g);
      cd1 = lds_u32(blk + 6 + 8 * g);
      sc = static_cast<float>(
          __builtin_bit_cast(_Float16, static_cast<uint16_t>(lds_u32(blk - 2) >> 16)));
    }
    const i4v a0 = __builtin_bit_cast(i4v, al[(2 * b) * 4 * arows]);
    const i4v a1 = __builtin_bit_cast(i4v, al[(2 * b + 1) * 4 * arows]);
    const float2 f = bl[b * kI8Tok];
    i4v acc = i4v{0, 0, 0, 0};
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, decode_i8(cd0), acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, decode_i8(cd1), acc, 0, 0, 0);
    const uint32_t v = (static_cast<uint32_t>(acc[0]) << 16) + (static_cast<uint32_t>(acc[1]) << 8) +
                       static_cast<uint32_t>(acc[2]) - __float_as_uint(f.x);
    const float blk_sum = static_cast<float>(static_cast<int>(v)) * f.y;  // times 2^-e: exact
    tot = fmaf(blk_sum, sc, tot);  // src/kernels.rs:651: acc += scale * block_acc
  }
  return tot;
}

// ---------------------------------------------------------------------------
// One-token integer product (n_tok == 1): the four lane groups of an MFMA
// work on four different 128-blocks.
//
// A 16x16x64 step sums 16 k-slots from each lane group g.  With one token,
// A row m = 4 j + d carries digit d of block 4 Q + j of quad Q (four blocks)
// in the k-slots of lane group j and zeros in the other groups, so step s
// (0..7) of a quad takes code dword s of block 4 Q + g from lane group g of
// every weight row, and lane (n, g) ends the quad holding the four digit
// sums of its own block.  The per-block combine then runs once per quad on
// all 64 lanes (16 rows x 4 blocks), and only the 16 lanes with m / 4 == g
// read A fragments (the others keep zeros).
//
// x side: each 128-block is scaled by the power of two 2^e that puts its
// largest |x| in [2^21, 2^22) and rounded to integers X (|X| <= 2^22, 22
// significant bits), written as four signed base-64 digits
// X = 64^3 d0 + 64^2 d1 + 64 d2 + d3 (|d0| <= 17, d1..d3 in [-32, 31]).  Codes: byte i of a code dword holds
// codes 4i .. 4i+3 at bits 0-1, 2-3, 4-5, 6-7.  The masks w & 0x03030303
// and w & 0x0C0C0C0C give c and 4c per byte (classes 0 and 1), and the same
// masks of w >> 4 give classes 2 and 3; fragment dword k = class k.  The A
// digit of a class-0 or class-2 slot is 4 d (fits int8), of a class-1 or
// class-3 slot d, so every product is 4 d c and each digit sum D_d is 4
// times sum_j d_j code_j.  H = 64 D0 + D1 and L = 64 D2 + D3 are exact
// multiples of 4, so
//     V = 4096 (H >> 2) + (L >> 2) = sum_j X_j code_j
// (|V| <= 2^22 * 3 * 128 < 2^31), and V - sum_j X_j = sum_j X_j (code_j - 1)
// exactly in i32; converted to f32 once and multiplied by 2^-e (exact), it
// is the block sum the reference adds as scale * block_acc
// (src/kernels.rs:651).
// ---------------------------------------------------------------------------

// The four digit fragments of step s of one 128-block: lane s of an aligned
// group of 8 lanes (one block) converts columns 16 s .. 16 s + 15 of
// xb = x + 128 * blk; every lane of the 8 gets the block factor {bits of
// sum X, 2^-e} (NaN factor when the block holds a NaN or infinity).
// Contains cross-lane steps inside each 8-lane group: all lanes of the wave
// must call it (dead items with live = false).
__device__ __forceinline__ void q1_load_item(const float *xb, int s, bool live, float (&f)[16]) {
  const float4 *xr = reinterpret_cast<const float4 *>(xb + 16 * s);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 v = live ? xr[q] : make_float4(0.f, 0.f, 0.f, 0.f);
    f[4 * q] = v.x;
    f[4 * q + 1] = v.y;
    f[4 * q + 2] = v.z;
    f[4 * q + 3] = v.w;
  }
}
__device__ __forceinline__ void q1_digits(float (&f)[16], uint4 frag[4], float2 &fac) {
  float mx = 0.0f;
  int bad = 0;  // a NaN or infinity in the block
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    const bool fin = __builtin_isfinite(f[c]);
    bad |= !fin;
    f[c] = fin ? f[c] : 0.0f;
    mx = fmaxf(mx, fabsf(f[c]));
  }
  mx = lane_group_reduce<8>(mx, MaxOp());
  bad = lane_group_reduce<8>(bad, SumOp());
  int ex = 0;
  if (mx > 0.0f) {
    int k;
    (void)frexpf(mx, &k);  // mx = f * 2^k, f in [0.5, 1): mx * 2^(22-k) in [2^21, 2^22)
    ex = 22 - k;
    ex = ex > 126 ? 126 : ex;  // tiny blocks round toward zero; 2^-e stays normal
  }
  const float sc = ldexpf(1.0f, ex);
  // X + kBias has the unsigned base-64 digits d + 32 (each in [0, 63]) of
  // the balanced digits d of X; they are packed as bytes first and turned
  // into the int8 A values per dword: 4 d = (4 (d + 32)) ^ 0x80 for classes
  // 0 and 2, and d = (d + 32) ^ 0x20 with bit 5 of the result copied into
  // bits 6 and 7 (the sign of a negative d) for classes 1 and 3
  constexpr uint32_t kBias = 32u * (1u + 64u + 4096u + 262144u);
  uint32_t dg[4][4] = {};
  int sx = 0;
#pragma unroll
  for (int c = 0; c < 16; ++c) {
    const int X = static_cast<int>(rintf(f[c] * sc));  // |X| <= 2^22
    sx += X;
    const uint32_t u = static_cast<uint32_t>(X) + kBias;  // in [0, 2^24)
    const int k = c & 3, i = c >> 2;  // class k, byte i: column 4 i + k of the step
#pragma unroll
    for (int d = 0; d < 4; ++d) dg[d][k] |= __builtin_amdgcn_ubfe(u, 6 * (3 - d), 6) << (8 * i);
  }
#pragma unroll
  for (int d = 0; d < 4; ++d) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if ((k & 1) == 0) {
        dg[d][k] = (dg[d][k] << 2) ^ 0x80808080u;
      } else {
        const uint32_t t = dg[d][k] ^ 0x20202020u, sgn = t & 0x20202020u;
        dg[d][k] = t | (sgn << 1) | (sgn << 2);
      }
    }
  }
  sx = lane_group_reduce<8>(sx, SumOp());
#pragma unroll
  for (int d = 0; d < 4; ++d) frag[d] = make_uint4(dg[d][0], dg[d][1], dg[d][2], dg[d][3]);
  fac = make_float2(__int_as_float(sx), bad ? __builtin_nanf("") : ldexpf(1.0f, -ex));
}

// Digit fragments of x into LDS by all `lanes` lanes of the workgroup:
// uint4 (8 Q + s) * 16 + 4 j + d for block 4 Q + j, step s, digit d; block
// factors at bf[blk].  The trip count is the same for every wave.  `f0`
// holds this lane's x values of the first pass, loaded by q1_load_x0 before
// the weight loads so that waiting for x does not wait for them.
__device__ __forceinline__ void q1_load_x0(const MmI8Args &a, float (&f0)[16]) {
  const int item = static_cast<int>(threadIdx.x);
  const bool live_item = item < a.nblk * 8;
  q1_load_item(a.x + 128 * (live_item ? item >> 3 : 0), item & 7, live_item, f0);
}
__device__ __forceinline__ void q1_stage_x(const MmI8Args &a, uint4 *smem, float2 *bf, int lanes,
                                           float (&f0)[16]) {
  const int n_items = a.nblk * 8;
  for (int base = 0; base < n_items; base += lanes) {
    const int item = base + static_cast<int>(threadIdx.x);
    const bool live_item = item < n_items;
    const int blk = live_item ? item >> 3 : 0, s = item & 7;
    uint4 frag[4];
    float2 fac;
    if (base == 0) {
      q1_digits(f0, frag, fac);
    } else {
      float f[16];
      q1_load_item(a.x + 128 * blk, s, live_item, f);
      q1_digits(f, frag, fac);
    }
    if (live_item) {
      uint4 *dst = smem + (8 * (blk >> 2) + s) * 16 + 4 * (blk & 3);
      dst[0] = frag[0];
      dst[1] = frag[1];
      dst[2] = frag[2];
      dst[3] = frag[3];
      if (s == 0) bf[blk] = fac;
    }
  }
}

__device__ __forceinline__ i4v decode_q1(uint32_t w) {
  const uint32_t t = w >> 4;
  return i4v{static_cast<int>(w & 0x03030303u), static_cast<int>(w & 0x0C0C0C0Cu),
             static_cast<int>(t & 0x03030303u), static_cast<int>(t & 0x0C0C0C0Cu)};
}

// One 8-block chunk (two quads) of a wave's 16-row tile from its LDS stage
// into the lane's running sum (blocks b0 + 4 q + g of row n).  `av` holds the
// A fragments; lanes with act == false never load them and keep zeros.
__device__ __forceinline__ float q1_chunk(const uint8_t *stage, const uint4 *al, const float2 *bf,
                                          bool act, int n, int g, int b0, float tot, i4v (&av)[8]) {
  const uint8_t *rowp = stage + n * kStageStride;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int jl = 4 * q + g;         // this lane group's block within the chunk
    const int o = kPq2Blk * jl + 2;   // its first code byte in the staged row
    const uint32_t *rw = reinterpret_cast<const uint32_t *>(rowp + (o & ~3));
    const uint32_t sh = static_cast<uint32_t>(o & 3);  // 2 for even blocks, 0 for odd
    uint32_t r[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) r[i] = rw[i];  // the ninth is read past odd blocks' codes, unused
    const float sc = static_cast<float>(
        __builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t *>(rowp + kPq2Blk * jl)));
    const int quad = (b0 >> 2) + q;
    if (act) {
#pragma unroll
      for (int s = 0; s < 8; ++s) av[s] = __builtin_bit_cast(i4v, al[(8 * quad + s) * 16]);
    }
    const float2 f = bf[b0 + jl];
    i4v acc = i4v{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const uint32_t w = __builtin_amdgcn_alignbyte(r[s + 1], r[s], sh);
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[s], decode_q1(w), acc, 0, 0, 0);
    }
    const int hi = ((acc[0] << 6) + acc[1]) >> 2, lo = ((acc[2] << 6) + acc[3]) >> 2;
    const int v = (hi << 12) + lo - __float_as_int(f.x);
    const float blk_sum = static_cast<float>(v) * f.y;  // times 2^-e: exact
    tot = fmaf(blk_sum, sc, tot);  // src/kernels.rs:651: acc += scale * block_acc
  }
  return tot;
}

// Sum of the four lane groups' partials (blocks = g mod 4) of a row, the same
// bits on every lane.  All lanes of the wave must be active.
__device__ __forceinline__ float q1_row_total(float tot) {
  float lo, hi;
  lane_swap<16>(tot, lo, hi);
  tot = lo + hi;
  lane_swap<32>(tot, lo, hi);
  return lo + hi;
}

// Workgroup = RT row tiles x KS waves each; wave (rt, ks) streams the chunks
// c = ks, ks + KS, ... of row tile blockIdx.x * RT + rt through its private
// LDS stage, and the KS partial sums of a tile are added in ks order at the
// end.  The fragments of the (single) token group and its block factors are
// copied to LDS once per workgroup, only the A rows of live tokens.
template <int KS, int RT, bool Q1>
__global__ __launch_bounds__(64 * KS * RT) __attribute__((amdgpu_waves_per_eu(4)))
void pq2_i8_kernel(MmI8Args a) {
  constexpr int kWaves = KS * RT;
  extern __shared__ uint4 smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int rt = wave / KS, ks = wave - rt * KS;
  const int row0 = (blockIdx.x * RT + rt) * 16;
  const int nsteps = 2 * a.nblk;

  const int arows = 4 * a.n_tok;  // live A rows (n_tok <= kI8Tok)
  const int total = Q1 ? nsteps * 16 : nsteps * 4 * arows;
  float2 *bf = reinterpret_cast<float2 *>(smem + total);
  const size_t a_words = static_cast<size_t>(total) +
                         (Q1 ? (static_cast<size_t>(a.nblk) + 1) / 2
                             : (static_cast<size_t>(a.nblk) * kI8Tok + 1) / 2);
  // rows of absent tokens and the unused fourth digit row feed D rows that
  // are never read: any in-bounds fragment will do
  const uint4 *al = Q1 ? smem + n : smem + g * arows + (n < arows ? n : (n & 3));
  const float2 *bl = Q1 ? bf : bf + g;
  const bool act = (n >> 2) == g;  // one-token form: lanes that carry A data
  i4v av[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) av[s] = i4v{0, 0, 0, 0};
  uint8_t *stage = reinterpret_cast<uint8_t *>(smem + a_words) + wave * kStageWaveBytes;

  const uint8_t *src[kStageLoads];
  int dst[kStageLoads];
  bool live[kStageLoads];
#pragma unroll
  for (int k = 0; k < kStageLoads; ++k) {
    const int idx = lane + 64 * k;
    live[k] = idx < 16 * kStageF4;
    // lanes past the stage read the last piece again (a load with no branch
    // keeps the compiler's wait counts exact) and store nothing
    const int r = live[k] ? idx / kStageF4 : 15, c16 = live[k] ? idx % kStageF4 : kStageF4 - 1;
    int row = row0 + r;
    row = row < a.n_rows ? row : a.n_rows - 1;  // tail rows read a valid row, store nothing
    src[k] = a.w + static_cast<size_t>(row) * a.row_bytes + 16 * c16;
    dst[k] = r * kStageStride + 16 * c16;
  }
  uint4 regs[kStageLoads];
  auto gload = [&](int chunk) {
#pragma unroll
    for (int k = 0; k < kStageLoads; ++k)
      regs[k] = *reinterpret_cast<const uint4 *>(src[k] + static_cast<size_t>(chunk) * kStageRowBytes);
  };
  auto lstore = [&]() {
#pragma unroll
    for (int k = 0; k < kStageLoads; ++k) {
      if (live[k]) {
        uint2 *d = reinterpret_cast<uint2 *>(stage + dst[k]);  // 8-byte aligned
        d[0] = make_uint2(regs[k].x, regs[k].y);
        d[1] = make_uint2(regs[k].z, regs[k].w);
      }
    }
  };

  float tot = 0.0f;
  const int n_chunks = a.nblk / kStageBlocks;
  int c = ks;
  float xf0[16];
  if constexpr (Q1) q1_load_x0(a, xf0);  // x before the weights: its wait does not cover them
  gload(c < n_chunks ? c : n_chunks - 1);  // in flight while x is staged (waves without a chunk re-read one)
  if constexpr (Q1)
    q1_stage_x(a, smem, bf, 64 * kWaves, xf0);
  else
    i8_stage_x(a, smem, bf, arows, 64 * kWaves);
  __syncthreads();  // x staging visible to every wave
  if (c < n_chunks) {
    lstore();
    if (c + KS < n_chunks) gload(c + KS);
  }
  for (; c < n_chunks; c += KS) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if constexpr (Q1)
      tot = q1_chunk(stage, al, bl, act, n, g, c * kStageBlocks, tot, av);
    else
      tot = i8_chunk(stage, al, bl, arows, n, g, c * kStageBlocks, tot);
    if (c + KS < n_chunks) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      lstore();  // chunk c + KS replaces chunk c (this wave finished reading it)
      if (c + 2 * KS < n_chunks) gload(c + 2 * KS);
    }
  }

  const int row = row0 + n;
  if constexpr (Q1) tot = q1_row_total(tot);
  if constexpr (KS > 1) {
    __syncthreads();  // every wave is done with its stage: reuse the LDS
    float *part = reinterpret_cast<float *>(smem);
    part[wave * 64 + lane] = tot;
    __syncthreads();
    if (ks == 0) {
      float s = part[(rt * KS) * 64 + lane];
#pragma unroll
      for (int k = 1; k < KS; ++k) s += part[(rt * KS + k) * 64 + lane];  // fixed order
      tot = s;
    }
  }
  if (ks == 0 && g < a.n_tok && row < a.n_rows) a.y[static_cast<size_t>(g) * a.y_stride + row] = tot;
}

// Persistent form for matrices with more row tiles than one round of
// workgroups holds (the LM head): G workgroups of RT waves, G sized to one
// round; workgroup w builds the x fragments once, then wave rt walks the row
// tiles (w + i G) RT + rt, i = 0, 1, ..., as one flat stream of (tile, chunk)
// items through its LDS stage -- the next item's loads in flight across tile
// boundaries -- and writes each tile's outputs when its last chunk is done.
// No prepare launch, no scratch, no later rounds of workgroups each repeating
// the x preparation.
template <int RT, bool Q1>
__global__ __launch_bounds__(64 * RT) void pq2_i8_persist_kernel(MmI8Args a) {
  extern __shared__ uint4 smem[];
  const int lane = threadIdx.x & 63, rt = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int nsteps = 2 * a.nblk;
  const int arows = 4 * a.n_tok;
  const int total = Q1 ? nsteps * 16 : nsteps * 4 * arows;
  float2 *bf = reinterpret_cast<float2 *>(smem + total);
  const size_t a_words = static_cast<size_t>(total) +
                         (Q1 ? (static_cast<size_t>(a.nblk) + 1) / 2
                             : (static_cast<size_t>(a.nblk) * kI8Tok + 1) / 2);
  const uint4 *al = Q1 ? smem + n : smem + g * arows + (n < arows ? n : (n & 3));
  const float2 *bl = Q1 ? bf : bf + g;
  const bool act = (n >> 2) == g;  // one-token form: lanes that carry A data
  i4v av[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) av[s] = i4v{0, 0, 0, 0};
  uint8_t *stage = reinterpret_cast<uint8_t *>(smem + a_words) + rt * kStageWaveBytes;

  const int n_chunks = a.nblk / kStageBlocks;
  const int tiles = (a.n_rows + 15) / 16;
  const int groups = (tiles + RT - 1) / RT;
  const int gw = static_cast<int>(blockIdx.x), G = static_cast<int>(gridDim.x);
  const int my_groups = groups > gw ? (groups - gw + G - 1) / G : 0;
  const int n_items = my_groups * n_chunks;
  auto item_tile = [&](int q) { return (gw + (q / n_chunks) * G) * RT + rt; };

  int r_of[kStageLoads], c16_of[kStageLoads], dst[kStageLoads];
  bool live[kStageLoads];
#pragma unroll
  for (int k = 0; k < kStageLoads; ++k) {
    const int idx = lane + 64 * k;
    live[k] = idx < 16 * kStageF4;
    // lanes past the stage read the last piece again (a load with no branch
    // keeps the compiler's wait counts exact) and store nothing
    r_of[k] = live[k] ? idx / kStageF4 : 15;
    c16_of[k] = live[k] ? idx % kStageF4 : kStageF4 - 1;
    dst[k] = r_of[k] * kStageStride + 16 * c16_of[k];
  }
  uint4 regs[kStageLoads];
  auto gload = [&](int q) {
    const int tile = item_tile(q), c = q % n_chunks;
#pragma unroll
    for (int k = 0; k < kStageLoads; ++k) {
      int row = tile * 16 + r_of[k];
      row = row < a.n_rows ? row : a.n_rows - 1;  // tail rows read a valid row, store nothing
      regs[k] = *reinterpret_cast<const uint4 *>(a.w + static_cast<size_t>(row) * a.row_bytes +
                                                 16 * c16_of[k] + static_cast<size_t>(c) * kStageRowBytes);
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int k = 0; k < kStageLoads; ++k) {
      if (live[k]) {
        uint2 *d = reinterpret_cast<uint2 *>(stage + dst[k]);
        d[0] = make_uint2(regs[k].x, regs[k].y);
        d[1] = make_uint2(regs[k].z, regs[k].w);
      }
    }
  };

  float xf0[16];
  if constexpr (Q1) q1_load_x0(a, xf0);  // x before the weights: its wait does not cover them
  gload(0);  // in flight while x is prepared (every workgroup of the grid has a tile group)
  if constexpr (Q1)
    q1_stage_x(a, smem, bf, 64 * RT, xf0);
  else
    i8_stage_x(a, smem, bf, arows, 64 * RT);
  __syncthreads();  // x staging visible to every wave
  if (n_items > 0) {
    lstore();
    if (n_items > 1) gload(1);
  }
  float tot = 0.0f;
  for (int q = 0; q < n_items; ++q) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int c = q % n_chunks;
    if constexpr (Q1)
      tot = q1_chunk(stage, al, bl, act, n, g, c * kStageBlocks, tot, av);
    else
      tot = i8_chunk(stage, al, bl, arows, n, g, c * kStageBlocks, tot);
    if (c == n_chunks - 1) {  // the tile's last chunk: its outputs are final
      const int row = item_tile(q) * 16 + n;
      if constexpr (Q1) tot = q1_row_total(tot);
      if (g < a.n_tok && row < a.n_rows) a.y[static_cast<size_t>(g) * a.y_stride + row] = tot;
      tot = 0.0f;
    }
    if (q + 1 < n_items) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      lstore();  // item q + 1 replaces item q (this wave finished reading it)
      if (q + 2 < n_items) gload(q + 2);
    }
  }
}

// ---------------------------------------------------------------------------
// Integer product for more than kI8Tok tokens (prefill batches).  Tokens go
// in groups of 4 (A rows 4 t + digit of an MFMA, as above).  A prepare launch
// writes every group's digit fragments once, laid out so one block of all
// groups is contiguous: uint4 [block][step in block][group][lane group][16
// rows], block factors float2 [block][group][token slot].  A workgroup is W
// waves (W row tiles of 16) x G token groups: per block, the block's
// fragments of its groups (2 G KB) are copied to a double-buffered LDS
// stage shared by the W waves -- the next block's copy is loaded into
// registers while the current block is multiplied -- and each wave decodes
// its tile's codes once and runs two integer MFMAs per group.  The barrier
// between blocks waits for LDS traffic only, so the weight chunks each wave
// prefetches stay in flight across it.
// ---------------------------------------------------------------------------

struct GemmI8Args {
  const uint8_t *w;     // first row of the range
  const uint4 *afrag;   // [nblk][2][n_groups][4][16]
  const float2 *bfac;   // [nblk][n_groups][4]
  float *y;             // [n_tok][y_stride]
  size_t row_bytes;
  int n_rows, nblk, n_tok, n_groups, y_stride;
};

struct GprepArgs {
  const float *x;  // [n_tok][ne0]
  uint4 *afrag;
  float2 *bfac;
  int ne0, n_tok, nblk, n_groups;
};

__global__ __launch_bounds__(kMmThreads) void pq2_gemm_i8_prep_kernel(GprepArgs a) {
  const int item = blockIdx.x * kMmThreads + threadIdx.x;
  const int tb = item >> 3, sub = item & 7;
  const bool live = tb < a.n_tok * a.nblk;
  const int t = live ? tb / a.nblk : 0, blk = live ? tb - t * a.nblk : 0;
  uint4 frag[3];
  float2 fac;
  i8_prep_item(a.x + static_cast<size_t>(t) * a.ne0 + 128 * blk, sub, live, frag, fac);
  if (!live) return;
  const int grp = t / kI8Tok, tq = t % kI8Tok;
  const int h = sub & 1, g = sub >> 1;
  uint4 *dst = a.afrag + ((static_cast<size_t>(blk) * 2 + h) * a.n_groups + grp) * 64 + g * 16 + 4 * tq;
#pragma unroll
  for (int d = 0; d < 3; ++d) dst[d] = frag[d];
  if (sub == 0) a.bfac[(static_cast<size_t>(blk) * a.n_groups + grp) * kI8Tok + tq] = fac;
}

template <int W, int G>
__global__ __launch_bounds__(64 * W) void pq2_gemm_i8_kernel(GemmI8Args a) {
  extern __shared__ uint4 smem[];
  constexpr int kThreads = 64 * W;
  constexpr int kFrag = 2 * G * 64;  // uint4 per staged block
  constexpr int kFac = G * kI8Tok;   // float2 per staged block
  static_assert(kFrag <= 2 * kThreads && kFac <= kThreads, "at most two uint4 per lane");
  uint4 *sa = smem;                                       // [2][kFrag]
  float2 *sf = reinterpret_cast<float2 *>(smem + 2 * kFrag);  // [2][kFac]
  uint8_t *stage = reinterpret_cast<uint8_t *>(sf + 2 * kFac) + (threadIdx.x >> 6) * kStageWaveBytes;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int row0 = (blockIdx.x * W + wave) * 16;
  const int grp0 = blockIdx.y * G;
  const int ng = a.n_groups - grp0 < G ? a.n_groups - grp0 : G;

  // weight staging per wave, as pq2_i8_kernel (8-block chunks, 17 x 16 B per row)
  const uint8_t *src[kStageLoads];
  int dst[kStageLoads];
  bool live[kStageLoads];
#pragma unroll
  for (int k = 0; k < kStageLoads; ++k) {
    const int idx = lane + 64 * k;
    live[k] = idx < 16 * kStageF4;
    const int r = live[k] ? idx / kStageF4 : 0, c16 = live[k] ? idx % kStageF4 : 0;
    int row = row0 + r;
    row = row < a.n_rows ? row : a.n_rows - 1;  // tail rows read a valid row, store nothing
    src[k] = a.w + static_cast<size_t>(row) * a.row_bytes + 16 * c16;
    dst[k] = r * kStageStride + 16 * c16;
  }
  uint4 regs[kStageLoads];
  auto gload = [&](int chunk) {
#pragma unroll
    for (int k = 0; k < kStageLoads; ++k)
      if (live[k]) regs[k] = *reinterpret_cast<const uint4 *>(src[k] + static_cast<size_t>(chunk) * kStageRowBytes);
  };
  auto lstore = [&]() {
#pragma unroll
    for (int k = 0; k < kStageLoads; ++k) {
      if (live[k]) {
        uint2 *d = reinterpret_cast<uint2 *>(stage + dst[k]);
        d[0] = make_uint2(regs[k].x, regs[k].y);
        d[1] = make_uint2(regs[k].z, regs[k].w);
      }
    }
  };
  // the workgroup's fragments of block b: step h of group gi at [h][gi][64];
  // lane i moves uint4 i and i + kThreads (two named registers: an array
  // here is indexed through a pointer select and lands in scratch memory)
  const size_t fblk = 2 * static_cast<size_t>(a.n_groups) * 64;  // uint4 per block, all groups
  auto fsrc_of = [&](int i, bool &live_i) {
    const int h = i / (G * 64), gi = (i / 64) % G;
    live_i = i < kFrag && gi < ng;
    return a.afrag + (static_cast<size_t>(h) * a.n_groups + grp0 + (live_i ? gi : 0)) * 64 + (i & 63);
  };
  bool fl0, fl1;
  const uint4 *fs0 = fsrc_of(static_cast<int>(threadIdx.x), fl0);
  const uint4 *fs1 = fsrc_of(static_cast<int>(threadIdx.x) + kThreads, fl1);
  uint4 fr0 = make_uint4(0, 0, 0, 0), fr1 = make_uint4(0, 0, 0, 0);
  float2 fc = make_float2(0.f, 0.f);
  const bool fclive = threadIdx.x < kFac && static_cast<int>(threadIdx.x) / kI8Tok < ng;
  // predicated loads and a branch per group keep the register count low
  // (unconditional loads and straight-line groups measured slower: more
  // registers, fewer waves per SIMD)
  auto fload = [&](int b) {
    if (fl0) fr0 = fs0[b * fblk];
    if (fl1) fr1 = fs1[b * fblk];
    if (fclive) fc = a.bfac[(static_cast<size_t>(b) * a.n_groups + grp0) * kI8Tok + threadIdx.x];
  };
  auto fstore = [&](int b) {
    if (threadIdx.x < kFrag) sa[(b & 1) * kFrag + threadIdx.x] = fr0;
    if (threadIdx.x + kThreads < kFrag) sa[(b & 1) * kFrag + kThreads + threadIdx.x] = fr1;
    if (threadIdx.x < kFac) sf[(b & 1) * kFac + threadIdx.x] = fc;
  };

  float tot[G];
#pragma unroll
  for (int gi = 0; gi < G; ++gi) tot[gi] = 0.0f;
  const int n_chunks = a.nblk / kStageBlocks;
  gload(0);
  fload(0);
  fstore(0);
  lstore();
  if (n_chunks > 1) gload(1);
  if (a.nblk > 1) fload(1);
  lds_barrier();  // block 0's fragments and this wave's first chunk staged
  for (int c = 0; c < n_chunks; ++c) {
    const uint8_t *rowp = stage + n * kStageStride;
    for (int bb = 0; bb < kStageBlocks; ++bb) {
      const int b = c * kStageBlocks + bb;
      const uint8_t *blk = rowp + kPq2Blk * bb;
      uint32_t cd0, cd1;
      float sc;
      if ((bb & 1) == 0) {  // block starts on a dword: codes are 2 bytes in
        const uint32_t e0 = lds_u32(blk + 8 * g), e1 = lds_u32(blk + 8 * g + 4),
                       e2 = lds_u32(blk + 8 * g + 8);
        cd0 = __builtin_amdgcn_alignbyte(e1, e0, 2);
        cd1 = __builtin_amdgcn_alignbyte(e2, e1, 2);
        sc = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(lds_u32(blk))));
      } else {  // block starts 2 bytes into a dword: codes are dword-aligned
        cd0 = lds_u32(blk + 2 + 8 * g);
        cd1 = lds_u32(blk + 6 + 8 * g);
        sc = static_cast<float>(
            __builtin_bit_cast(_Float16, static_cast<uint16_t>(lds_u32(blk - 2) >> 16)));
      }
      const i4v b0 = decode_i8(cd0), b1 = decode_i8(cd1);
      const uint4 *fa = sa + (b & 1) * kFrag + g * 16 + n;
      const float2 *ff = sf + (b & 1) * kFac + g;
#pragma unroll
      for (int gi = 0; gi < G; ++gi) {
        if (gi < ng) {
          const i4v a0 = __builtin_bit_cast(i4v, fa[gi * 64]);
          const i4v a1 = __builtin_bit_cast(i4v, fa[(G + gi) * 64]);
          i4v acc = i4v{0, 0, 0, 0};
          acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, acc, 0, 0, 0);
          const float2 f = ff[gi * kI8Tok];
          const uint32_t v = (static_cast<uint32_t>(acc[0]) << 16) +
                             (static_cast<uint32_t>(acc[1]) << 8) + static_cast<uint32_t>(acc[2]) -
                             __float_as_uint(f.x);
          const float blk_sum = static_cast<float>(static_cast<int>(v)) * f.y;  // times 2^-e: exact
          tot[gi] = fmaf(blk_sum, sc, tot[gi]);  // src/kernels.rs:651
        }
      }
      // block b + 1's fragments to the other buffer (its readers passed the
      // last barrier), block b + 2's requested
      if (b + 1 < a.nblk) fstore(b + 1);
      if (b + 2 < a.nblk) fload(b + 2);
      if (bb == kStageBlocks - 1 && c + 1 < n_chunks) {
        lstore();  // chunk c + 1 replaces chunk c (this wave finished reading it)
        if (c + 2 < n_chunks) gload(c + 2);
      }
      lds_barrier();
    }
  }
  const int row = row0 + n;
  if (row < a.n_rows) {
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      const int t = (grp0 + gi) * kI8Tok + g;
      if (gi < ng && t < a.n_tok) a.y[static_cast<size_t>(t) * a.y_stride + row] = tot[gi];
    }
  }
}

// Any ne0 or alignment: the scalar reference loop (src/kernels.rs:633-653),
// one wave per (row, token), lanes over blocks, block sums in order, then a
// fixed-order reduction of the lanes' scale * block_sum terms.
__global__ __launch_bounds__(64) void pq2_mm_generic_kernel(const uint8_t *w, size_t row_bytes,
                                                            int ne0, const float *x, int n_tok,
                                                            float *y, int n_rows) {
  const int row = blockIdx.x;
  const int m = blockIdx.y;
  if (row >= n_rows || m >= n_tok) return;
  const uint8_t *raw = w + static_cast<size_t>(row) * row_bytes;
  const float *xr = x + static_cast<size_t>(m) * ne0;
  const int nblk = (ne0 + 127) / 128;
  float acc = 0.0f;
  for (int b = threadIdx.x; b < nblk; b += 64) {
    const uint8_t *blk = raw + b * kPq2Blk;
    const uint32_t h = static_cast<uint32_t>(blk[0]) | (static_cast<uint32_t>(blk[1]) << 8);
    const float scale = __uint_as_float(half_bits_to_f32_bits(h));
    const int start = b * 128, end = start + 128 < ne0 ? start + 128 : ne0;
    float bacc = 0.0f;
    for (int j = start; j < end; ++j) {
      const uint32_t code = (blk[2 + (j - start) / 4] >> (((j - start) % 4) * 2)) & 3u;
      bacc += xr[j] * static_cast<float>(static_cast<int>(code) - 1);
    }
    acc += scale * bacc;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (threadIdx.x == 0) y[static_cast<size_t>(m) * n_rows + row] = acc;
}

__global__ void fill_zero_kernel(float *y, size_t n) {
  const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) y[i] = 0.0f;
}

constexpr int kLdsTok = 4;                 // token counts staged whole in LDS
constexpr size_t kLdsABytes = 104 * 1024;  // their LDS budget (with 4 wave stages: 121 KB)

template <int MT, int NT, bool ALDS = false>
int launch_mm(const MmArgs &a, int n_tiles, hipStream_t st) {
  const unsigned gx = static_cast<unsigned>((a.n_rows + 64 * NT - 1) / (64 * NT));
  const unsigned gy = static_cast<unsigned>((n_tiles + MT - 1) / MT);
  size_t lds = 0;
  if constexpr (ALDS) {
    lds = static_cast<size_t>(a.n_ksteps) * 2 * a.n_tok * 4 * sizeof(uint4) +
          static_cast<size_t>(a.nblk) * 8 * sizeof(float4);
    if (int e = check_hip(hipFuncSetAttribute(reinterpret_cast<const void *>(pq2_mm_kernel<MT, NT, true>),
                                              hipFuncAttributeMaxDynamicSharedMemorySize,
                                              static_cast<int>(kLdsABytes)),
                          "hipFuncSetAttribute"))
      return e;
  }
  BH_LAUNCH((pq2_mm_kernel<MT, NT, ALDS>), dim3(gx, gy), kMmThreads, lds, st, a);
  return ok();
}

template <bool ALDS, int TOKQ>
int launch_staged(const MmArgs &a, hipStream_t st) {
  const unsigned gx = static_cast<unsigned>((a.n_rows + 63) / 64);
  size_t lds = 4 * kStageWaveBytes;
  if constexpr (ALDS)
    lds += static_cast<size_t>(a.n_ksteps) * 2 * a.n_tok * 4 * sizeof(uint4) +
           static_cast<size_t>(a.nblk) * 8 * sizeof(float4);
  if (int e = check_hip(hipFuncSetAttribute(reinterpret_cast<const void *>(pq2_mm_staged_kernel<ALDS, TOKQ>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize,
                                            static_cast<int>(kLdsABytes + 4 * kStageWaveBytes)),
                        "hipFuncSetAttribute"))
    return e;
  BH_LAUNCH((pq2_mm_staged_kernel<ALDS, TOKQ>), gx, kMmThreads, lds, st, a);
  return ok();
}

template <int KS, int RT = 8 / KS, bool Q1 = false>
int launch_i8(const MmI8Args &a, size_t lds_a, hipStream_t st) {
  const int tiles = (a.n_rows + 15) / 16;
  const unsigned gx = static_cast<unsigned>((tiles + RT - 1) / RT);
  const size_t lds = lds_a + static_cast<size_t>(KS * RT) * kStageWaveBytes;
  if (int e = check_hip(hipFuncSetAttribute(reinterpret_cast<const void *>(pq2_i8_kernel<KS, RT, Q1>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize,
                                            static_cast<int>(lds)),
                        "hipFuncSetAttribute"))
    return e;
  BH_LAUNCH((pq2_i8_kernel<KS, RT, Q1>), gx, 64 * KS * RT, lds, st, a);
  return ok();
}

// The integer product for n_tok <= kI8Tok on staged shapes.  Every
// workgroup turns x into its digit fragments in LDS while its first weight
// chunks load: no prepare launch, no scratch (ffn_up N=1: 20.3 -> 14.9 us
// against a prepare launch).  Up to kI8RoundTiles row tiles the grid is one
// workgroup per tile group, and small matrices split each row tile's chunks
// over KS waves so the grid still holds a few thousand waves; beyond that
// (the LM head) a persistent grid of one round walks the tiles, so the x
// preparation is not repeated by later rounds of workgroups.  Q1 selects the
// one-token layout (four blocks per MFMA, see q1_chunk) for n_tok == 1.
constexpr size_t kI8RoundTiles = 4096;
template <bool Q1>
int pq2_i8(const uint8_t *w, size_t ne0, size_t n_rows, const float *x, size_t n_tok, float *y,
           size_t a_bytes, hipStream_t st) {
  const int nblk = static_cast<int>(ne0 / 128);
  MmI8Args a{w, x, y, bh_pq2_row_bytes(ne0), static_cast<int>(n_rows), nblk,
             static_cast<int>(n_tok), static_cast<int>(n_rows)};
  const size_t lds = a_bytes;
  const size_t tiles = (n_rows + 15) / 16;
  const int n_chunks = nblk / kStageBlocks;
  int ks = 1;
  while (ks < 8 && ks < n_chunks && tiles * ks < 4096) ks *= 2;
  if (tiles <= kI8RoundTiles) {
    // wide x (an 8-wave workgroup's LDS leaves room for one per CU) and few
    // row tiles: two tiles per 16-wave workgroup, 8 waves each, so the grid
    // is one round over the CUs instead of two (ffn_down N=1, 320 row tiles:
    // 13.7 us, against 20.2 with 8 waves and 14.8 with 4 waves per tile)
    if (n_chunks >= 8 && 2 * (a_bytes + 8 * kStageWaveBytes) > 160 * 1024 &&
        tiles <= 2 * device_cu_count() && a_bytes + 16 * kStageWaveBytes <= 160 * 1024)
      return launch_i8<8, 2, Q1>(a, lds, st);
    // the most waves per row tile whose grid still runs in one round: a
    // workgroup is 8 waves (8 / ks row tiles), as many per CU as LDS and the
    // wave limit allow (ffn_up N=1: 4 waves per tile made 544 workgroups for
    // 512 slots, a 32-workgroup second round)
    const size_t wg_lds = a_bytes + 8 * kStageWaveBytes;
    const size_t per_cu = std::min<size_t>(4, (160 * 1024) / wg_lds);
    const size_t slots = per_cu * device_cu_count();
    // (a wave count past the chunk count still pays when it shortens the
    // longest chain: 5 chunks over 8 waves are one round trip, over 4 two)
    for (int k = 8; k >= 1; k >>= 1) {
      const size_t wgs = (tiles + (8 / k) - 1) / (8 / k);
      const bool shorter = k == 1 || (n_chunks + k - 1) / k < (n_chunks + k / 2 - 1) / (k / 2);
      if (shorter && per_cu > 0 && wgs <= slots) {
        ks = k;
        break;
      }
    }
    switch (ks) {
      case 8: return launch_i8<8, 1, Q1>(a, lds, st);
      case 4: return launch_i8<4, 2, Q1>(a, lds, st);
      case 2: return launch_i8<2, 4, Q1>(a, lds, st);
      default: return launch_i8<1, 8, Q1>(a, lds, st);
    }
  }
  // many row tiles: the persistent kernel, one round of 8-wave workgroups
  constexpr int kPRT = 8;
  const size_t plds = a_bytes + kPRT * kStageWaveBytes;
  const size_t per_cu = std::max<size_t>(1, std::min<size_t>(4, (160 * 1024) / plds));
  const size_t groups = (tiles + kPRT - 1) / kPRT;
  const size_t G = std::min(groups, per_cu * device_cu_count());
  if (int e = check_hip(hipFuncSetAttribute(reinterpret_cast<const void *>(pq2_i8_persist_kernel<kPRT, Q1>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize,
                                            static_cast<int>(plds)),
                        "hipFuncSetAttribute"))
    return e;
  BH_LAUNCH((pq2_i8_persist_kernel<kPRT, Q1>), static_cast<unsigned>(G), 64 * kPRT, plds, st, a);
  return ok();
}

template <int W, int G>
int launch_gemm(const GemmI8Args &a, int n_groups, hipStream_t st) {
  const size_t lds = 2 * (2 * G * 64) * sizeof(uint4) + 2 * (G * kI8Tok) * sizeof(float2) +
                     W * kStageWaveBytes;
  if (int e = check_hip(hipFuncSetAttribute(reinterpret_cast<const void *>(pq2_gemm_i8_kernel<W, G>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize,
                                            static_cast<int>(lds)),
                        "hipFuncSetAttribute"))
    return e;
  const unsigned gx = static_cast<unsigned>((a.n_rows + 16 * W - 1) / (16 * W));
  const unsigned gy = static_cast<unsigned>((n_groups + G - 1) / G);
  if (gy > 65535) return fail(BH_ERR_SHAPE, "pq2_matmul_n: too many tokens for one launch");
  BH_LAUNCH((pq2_gemm_i8_kernel<W, G>), dim3(gx, gy), 64 * W, lds, st, a);
  return ok();
}

// Integer product for more than kI8Tok tokens: prepare launch, then one
// product launch over (row-tile groups of 8, token-group sets of 8).
int pq2_gemm_i8(const uint8_t *w, size_t ne0, size_t n_rows, const float *x, size_t n_tok,
                float *y, hipStream_t st) {
  const int nblk = static_cast<int>(ne0 / 128);
  const int n_groups = static_cast<int>((n_tok + kI8Tok - 1) / kI8Tok);
  const size_t frag_bytes = static_cast<size_t>(nblk) * 2 * n_groups * 64 * sizeof(uint4);
  const size_t fac_off = (frag_bytes + 255) / 256 * 256;
  const size_t fac_bytes = static_cast<size_t>(nblk) * n_groups * kI8Tok * sizeof(float2);
  char *scratch = static_cast<char *>(device_scratch(fac_off + fac_bytes, kScratchMatmul, st));
  if (scratch == nullptr) return BH_ERR_HIP;
  GprepArgs pa{x, reinterpret_cast<uint4 *>(scratch), reinterpret_cast<float2 *>(scratch + fac_off),
               static_cast<int>(ne0), static_cast<int>(n_tok), nblk, n_groups};
  const size_t items = n_tok * nblk * 8;
  if (items > static_cast<size_t>(INT32_MAX) - kMmThreads)  // the prepare kernel indexes items in int
    return fail(BH_ERR_SHAPE, "pq2_matmul_n: n_tok * ne0 too large for one call");
  BH_LAUNCH(pq2_gemm_i8_prep_kernel, static_cast<unsigned>((items + kMmThreads - 1) / kMmThreads),
            kMmThreads, 0, st, pa);
  GemmI8Args a{w, pa.afrag, pa.bfac, y, bh_pq2_row_bytes(ne0), static_cast<int>(n_rows), nblk,
               static_cast<int>(n_tok), n_groups, static_cast<int>(n_rows)};
  // 8 row tiles x 4 token groups (16 tokens) per workgroup: of 8x8, 8x4,
  // 8x2, 8x1, 4x4 and 4x2 the fastest for ffn_up N=64 and the LM head N=16
  // (more workgroups per CU outweigh the extra weight passes of smaller sets)
  return launch_gemm<8, 4>(a, n_groups, st);
}

// Y[n_tok][n_rows] = X[n_tok][ne0] * W[rows][ne0]^T on the device.
int pq2_mm(const uint8_t *w, size_t ne0, size_t n_rows, const float *x, size_t n_tok, float *y,
           hipStream_t st) {
  if (n_rows == 0 || n_tok == 0) return ok();
  const size_t row_bytes = bh_pq2_row_bytes(ne0);
  if (n_rows > 0x7fffffffu || n_tok > 0xffffu || ne0 > 0x7fffffffu)
    return fail(BH_ERR_SHAPE, "pq2_matmul_n: shape too large for one launch");
  if (ne0 == 0) {
    const size_t total = n_tok * n_rows;
    BH_LAUNCH(fill_zero_kernel, static_cast<unsigned>((total + 255) / 256), 256, 0, st, y, total);
    return ok();
  }
  // fast path: whole 128-blocks, an even block count (rows and block pairs
  // start on dwords), 16-byte aligned x rows
  const size_t nblk = ne0 / 128;
  const bool fast = ne0 % 128 == 0 && nblk % 2 == 0 && aligned16(x) &&
                    (reinterpret_cast<uintptr_t>(w) & 3u) == 0;
  if (!fast) {
    BH_LAUNCH(pq2_mm_generic_kernel, dim3(static_cast<unsigned>(n_rows), static_cast<unsigned>(n_tok)),
              64, 0, st, w, row_bytes, static_cast<int>(ne0), x, static_cast<int>(n_tok), y,
              static_cast<int>(n_rows));
    return ok();
  }
  const bool stageable = nblk % kStageBlocks == 0 && (reinterpret_cast<uintptr_t>(w) & 15u) == 0 &&
                         bh_pq2_row_bytes(ne0) % 16 == 0;
  if (stageable && n_tok == 1) {
    // LDS: 16 uint4 per MFMA step (two steps per block), a float2 per block
    const size_t a_bytes = 2 * nblk * 16 * sizeof(uint4) + (nblk * sizeof(float2) + 15) / 16 * 16;
    if (a_bytes <= kLdsABytes) return pq2_i8<true>(w, ne0, n_rows, x, n_tok, y, a_bytes, st);
  }
  if (stageable && n_tok <= static_cast<size_t>(kI8Tok)) {
    // LDS: the live A rows of every step, the block factors (float2 per
    // block and token slot), rounded to whole uint4
    const size_t a_bytes = 2 * nblk * 4 * (4 * n_tok) * sizeof(uint4) +
                           (nblk * kI8Tok * sizeof(float2) + 15) / 16 * 16;
    if (a_bytes <= kLdsABytes) return pq2_i8<false>(w, ne0, n_rows, x, n_tok, y, a_bytes, st);
  }
  if (stageable && n_tok > static_cast<size_t>(kI8Tok)) return pq2_gemm_i8(w, ne0, n_rows, x, n_tok, y, st);
  const int n_ksteps = static_cast<int>(ne0 / 32);
  const int n_tiles = static_cast<int>((n_tok + 15) / 16);
  const int mt = n_tiles >= 4 ? 4 : (n_tiles >= 2 ? 2 : 1);
  const int tiles_padded = (n_tiles + mt - 1) / mt * mt;
  // scratch: A fragments, then the per-(token, block) powers of two
  const size_t frag_bytes = static_cast<size_t>(tiles_padded) * n_ksteps * 2 * 64 * sizeof(uint4);
  const size_t binv_off = (frag_bytes + 255) / 256 * 256;
  const size_t binv_bytes = static_cast<size_t>(tiles_padded) * nblk * 8 * sizeof(float4);
  char *scratch = static_cast<char *>(device_scratch(binv_off + binv_bytes, kScratchMatmul, st));
  if (scratch == nullptr) return BH_ERR_HIP;
  PrepArgs pa{x, reinterpret_cast<uint4 *>(scratch), reinterpret_cast<float *>(scratch + binv_off),
              static_cast<int>(ne0), static_cast<int>(n_tok), static_cast<int>(nblk), n_ksteps};
  const size_t items = n_tok * nblk * 16;
  if (items > static_cast<size_t>(INT32_MAX) - kMmThreads)  // the prepare kernel indexes items in int
    return fail(BH_ERR_SHAPE, "pq2_matmul_n: n_tok * ne0 too large for one call");
  BH_LAUNCH(pq2_mm_prep_kernel, static_cast<unsigned>((items + kMmThreads - 1) / kMmThreads),
            kMmThreads, 0, st, pa);

  MmArgs a{w, pa.afrag, reinterpret_cast<const float4 *>(pa.binv), y, row_bytes,
           static_cast<int>(n_rows), static_cast<int>(nblk), n_ksteps, static_cast<int>(n_tok),
           static_cast<int>(n_rows)};
  // a wave takes 4 row tiles when that still leaves >= 2 blocks per CU
  const bool wide = n_rows >= static_cast<size_t>(256) * 2 * 256;
  const bool staged = nblk % kStageBlocks == 0 && (reinterpret_cast<uintptr_t>(w) & 15u) == 0 &&
                      row_bytes % 16 == 0 && n_tiles == 1;
  const bool a_in_lds = n_tok <= kLdsTok && static_cast<size_t>(n_ksteps) * 2 * n_tok * 4 * sizeof(uint4) +
                                                 nblk * 8 * sizeof(float4) <= kLdsABytes;
  if (staged) {
    if (a_in_lds) return n_tok == 1 ? launch_staged<true, 1>(a, st) : launch_staged<true, 4>(a, st);
    return launch_staged<false, 4>(a, st);
  }
  if (a_in_lds)
    return wide ? launch_mm<1, 4, true>(a, n_tiles, st) : launch_mm<1, 1, true>(a, n_tiles, st);
  switch (mt) {
    case 4: return wide ? launch_mm<4, 4>(a, n_tiles, st) : launch_mm<4, 1>(a, n_tiles, st);
    case 2: return wide ? launch_mm<2, 4>(a, n_tiles, st) : launch_mm<2, 1>(a, n_tiles, st);
    default: return wide ? launch_mm<1, 4>(a, n_tiles, st) : launch_mm<1, 1>(a, n_tiles, st);
  }
}

// Byte length of rows [0, base_row + n_rows), or false on overflow.
bool range_bytes(uint64_t base_row, size_t n_rows, size_t row_bytes, size_t *out) {
  const unsigned __int128 end = static_cast<unsigned __int128>(base_row) + n_rows;
  const unsigned __int128 bytes = end * row_bytes;
  if (bytes > static_cast<unsigned __int128>(SIZE_MAX)) return false;
  *out = static_cast<size_t>(bytes);
  return true;
}

}  // namespace
}  // namespace bh

using namespace bh;

extern "C" int bh_pq2_matvec_range(const uint8_t *payload, size_t payload_len, size_t ne0,
                                   uint64_t base_row, size_t n_rows, const float *x, size_t x_len,
                                   float *y, size_t y_len, bh_stream stream) {
  if (x_len != ne0)
    return fail(BH_ERR_SHAPE, "pq2_matvec_range: x length " + std::to_string(x_len) +
                                  " != ne0 " + std::to_string(ne0));
  if (y_len < n_rows) return fail(BH_ERR_SHAPE, "pq2_matvec_range: y too small");
  const size_t row_bytes = bh_pq2_row_bytes(ne0);
  size_t byte_len = 0;
  if (!range_bytes(base_row, n_rows, row_bytes, &byte_len))
    return fail(BH_ERR_SHAPE, "pq2_matvec_range: row range byte length overflows");
  if (byte_len > payload_len)
    return fail(BH_ERR_SHAPE, "pq2_matvec_range: rows " + std::to_string(base_row) + ".." +
                                  std::to_string(base_row + n_rows) + " need " +
                                  std::to_string(byte_len) + " bytes, payload is " +
                                  std::to_string(payload_len));
  if (n_rows == 0) return ok();
  if (payload == nullptr || x == nullptr || y == nullptr)
    return fail(BH_ERR_ARG, "pq2_matvec_range: null pointer");
  return pq2_mm(payload + base_row * row_bytes, ne0, n_rows, x, 1, y,
                static_cast<hipStream_t>(stream));
}

extern "C" int bh_pq2_matmul_n(const uint8_t *payload, size_t payload_len, size_t ne0,
                               uint64_t base_row, size_t n_rows, const float *x, size_t x_len,
                               size_t n_tok, float *y, size_t y_len, bh_stream stream) {
  if (x_len != n_tok * ne0)
    return fail(BH_ERR_SHAPE, "pq2_matmul_n: x length " + std::to_string(x_len) + " != n_tok " +
                                  std::to_string(n_tok) + " * ne0 " + std::to_string(ne0));
  if (y_len < n_tok * n_rows) return fail(BH_ERR_SHAPE, "pq2_matmul_n: y too small");
  const size_t row_bytes = bh_pq2_row_bytes(ne0);
  size_t need = 0;
  if (!range_bytes(base_row, n_rows, row_bytes, &need))
    return fail(BH_ERR_SHAPE, "pq2_matmul_n: overflow");
  if (need > payload_len) return fail(BH_ERR_SHAPE, "pq2_matmul_n: row range exceeds payload");
  if (n_rows == 0 || n_tok == 0) return ok();
  if (payload == nullptr || x == nullptr || y == nullptr)
    return fail(BH_ERR_ARG, "pq2_matmul_n: null pointer");
  return pq2_mm(payload + base_row * row_bytes, ne0, n_rows, x, n_tok, y,
                static_cast<hipStream_t>(stream));
}
