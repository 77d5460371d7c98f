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
// Mapping onto v_mfma_f32_16x16x32_f16 (D = A * B + C, 16x16 output tile):
//   M (A rows)    = tokens, 16 per tile (padded with zero tokens);
//   N (B columns) = weight rows, 16 per tile;
//   K             = columns of one 128-weight block, 4 MFMA steps of 32.
// The 2-bit codes become exact f16 values (code - 1) in {-1, 0, 1, 2}: the
// code lands in the mantissa of 1024.0 (bit pattern 0x6400 | code << p) and
// one packed f16 FMA maps 1024 + code * 2^p to code - 1 exactly.  The x side
// needs more than f16's 11 bits for a 1e-5 result, so every x value is
// scaled by a per-token power of two (largest |x| of the token in
// [2^14, 2^15)) and split into hi = f16(x') and lo = f16(x' - hi): hi + lo
// carries 22 significant bits, and two MFMAs (hi, lo) per weight tile
// accumulate it in f32.  Each block's f32 tile sum is then multiplied by
// the block's f32 scale and added to the row total, as the reference does;
// the power of two is removed at the end (exact).
//
// K order: the MFMA sums its 32 k-slots in any order, so lanes may take
// them in whatever order the codes unpack fastest; the A fragments are
// written in that same order by the prepare kernel (mm_column()).
#include <hip/hip_runtime.h>

#include <string>

#include "common.hpp"

namespace bh {
namespace {

constexpr int kPq2Blk = 34;
constexpr int kMmThreads = 256;  // 4 waves
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4v __attribute__((ext_vector_type(4)));

// Block column (0..127) of element e (= 2j + h) of lane group g's A/B
// fragment in MFMA step i (0..3) of a block.  Lane group g owns code bytes
// [8g, 8g + 8) of the block, i.e. columns [32g, 32g + 32); step i uses the
// dword of code bytes 8g + 4(i >> 1) .. +3; half h of pair j takes code j of
// byte 2h + (i & 1) of that dword.
__host__ __device__ constexpr int mm_column(int i, int g, int j, int h) {
  return 32 * g + 16 * (i >> 1) + 4 * (2 * h + (i & 1)) + j;
}

// ---------------------------------------------------------------------------
// Prepare: per-token power-of-two scale and the hi/lo f16 A fragments.
// afrag layout: [tile][kstep][piece (hi, lo)][64 lanes] x 16 bytes.
// ---------------------------------------------------------------------------
struct PrepArgs {
  const float *x;     // [n_tok][ne0]
  uint4 *afrag;
  float *tok_scale;   // [n_tok]: 2^e of each token
  float *tok_inv;     // [n_tok]: 2^-e
  int ne0, n_tok, n_ksteps, n_tiles;
};

// One block per token: the power of two that puts the token's largest |x|
// in [2^14, 2^15), so hi never overflows f16 and lo keeps 11 more bits.
__global__ __launch_bounds__(kMmThreads) void pq2_mm_scale_kernel(PrepArgs a) {
  __shared__ float part[kMmThreads / 64];
  const int m = blockIdx.x;
  const float *xr = a.x + static_cast<size_t>(m) * a.ne0;
  float mx = 0.0f;
  for (int j = threadIdx.x; j < a.ne0; j += kMmThreads) mx = fmaxf(mx, fabsf(xr[j]));  // NaN ignored
  mx = group_reduce<kMmThreads>(mx, MaxOp{}, part);
  if (threadIdx.x == 0) {
    int e = 0;
    if (mx > 0.0f && mx <= 3.4e38f) {
      int k;
      (void)frexpf(mx, &k);  // mx = f * 2^k, f in [0.5, 1): mx * 2^(15-k) in [2^14, 2^15)
      e = 15 - k;
      e = e < -126 ? -126 : (e > 126 ? 126 : e);  // 2^e and 2^-e stay normal f32
    }
    a.tok_scale[m] = ldexpf(1.0f, e);
    a.tok_inv[m] = ldexpf(1.0f, -e);
  }
}

__global__ __launch_bounds__(kMmThreads) void pq2_mm_prep_kernel(PrepArgs a) {
  const int tile = blockIdx.x;
  const int n_items = a.n_ksteps * 64;
  for (int item = blockIdx.y * kMmThreads + threadIdx.x; item < n_items;
       item += gridDim.y * kMmThreads) {
    const int ks = item >> 6, l = item & 63;
    const int ml = l & 15, g = l >> 4, i = ks & 3, blk = ks >> 2;
    const int m = 16 * tile + ml;
    h8 hi, lo;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      hi[e] = static_cast<_Float16>(0.0f);
      lo[e] = static_cast<_Float16>(0.0f);
    }
    if (m < a.n_tok) {
      const float s = a.tok_scale[m];
      const float *xr = a.x + static_cast<size_t>(m) * a.ne0 + 128 * blk;
      const float4 p0 = *reinterpret_cast<const float4 *>(xr + mm_column(i, g, 0, 0));
      const float4 p1 = *reinterpret_cast<const float4 *>(xr + mm_column(i, g, 0, 1));
      const float v[8] = {p0.x * s, p1.x * s, p0.y * s, p1.y * s,
                          p0.z * s, p1.z * s, p0.w * s, p1.w * s};  // element 2j + h
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const _Float16 h = static_cast<_Float16>(v[e]);
        hi[e] = h;
        // an infinite x keeps lo = 0 (inf - inf would turn the term into NaN)
        lo[e] = __builtin_isinf(static_cast<float>(h))
                    ? static_cast<_Float16>(0.0f)
                    : static_cast<_Float16>(v[e] - static_cast<float>(h));
      }
    }
    uint4 *dst = a.afrag + (static_cast<size_t>(tile) * a.n_ksteps + ks) * 2 * 64 + l;
    dst[0] = __builtin_bit_cast(uint4, hi);
    dst[64] = __builtin_bit_cast(uint4, lo);
  }
}

// ---------------------------------------------------------------------------
// Main product.  Block = 4 waves; a wave owns NT 16-row weight tiles and the
// block's MT token tiles.  Lane l: row n = l & 15 of each weight tile, lane
// group g = l >> 4 (code bytes 8g..8g+7 of every block).
// ---------------------------------------------------------------------------
struct MmArgs {
  const uint8_t *w;      // first row of the range (payload + base_row * row_bytes)
  const uint4 *afrag;
  const float *tok_inv;
  float *y;              // [n_tok][y_stride]
  size_t row_bytes;
  int n_rows, nblk, n_ksteps, n_tok, y_stride;
};

// f16 pairs (code_lo - 1, code_hi - 1) of the codes at bits (2j, 2j + 16)
// of t, for j = 0..3, as the 8 halves of a B fragment.
__device__ __forceinline__ h8 decode_codes(uint32_t t) {
  h8 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t mask = (3u << (2 * j)) | (3u << (2 * j + 16));
    const uint32_t bits = (t & mask) | 0x64006400u;  // 1024 + code * 2^(2j), exact
    const h2 v = __builtin_bit_cast(h2, bits);
    const _Float16 k = static_cast<_Float16>(1.0f / static_cast<float>(1 << (2 * j)));
    const _Float16 c = static_cast<_Float16>(-(1024.0f / static_cast<float>(1 << (2 * j)) + 1.0f));
    const h2 kk = {k, k}, cc = {c, c};
    const h2 w = __builtin_elementwise_fma(v, kk, cc);  // exact: a small integer
    r[2 * j] = w[0];
    r[2 * j + 1] = w[1];
  }
  return r;
}

template <int MT, int NT>
__global__ __launch_bounds__(kMmThreads) void pq2_mm_kernel(MmArgs a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int row_wave = blockIdx.x * (4 * 16 * NT) + wave * 16 * NT;
  const int tile0 = blockIdx.y * MT;

  const uint16_t *wp[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int row = row_wave + 16 * t + n;
    row = row < a.n_rows ? row : a.n_rows - 1;  // tail rows read a valid row, store nothing
    wp[t] = reinterpret_cast<const uint16_t *>(a.w + static_cast<size_t>(row) * a.row_bytes);
  }
  // halfword index of block b's scale is 17b; its code bytes 8g..8g+7 are
  // halfwords 17b + 1 + 4g .. +3 (every block and row starts on an even byte)
  uint32_t nxt_c[NT][4], nxt_s[NT];
  auto load_block = [&](int b) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const uint16_t *p = wp[t] + 17 * b;
      nxt_s[t] = p[0];
#pragma unroll
      for (int q = 0; q < 4; ++q) nxt_c[t][q] = p[1 + 4 * g + q];
    }
  };

  f4v tot[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < NT; ++t) tot[mt][t] = f4v{0.f, 0.f, 0.f, 0.f};

  const uint4 *af = a.afrag + static_cast<size_t>(tile0) * a.n_ksteps * 2 * 64 + lane;
  load_block(0);
  for (int b = 0; b < a.nblk; ++b) {
    uint32_t cd[NT][2], sc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      cd[t][0] = nxt_c[t][0] | (nxt_c[t][1] << 16);  // code bytes 8g .. 8g+3
      cd[t][1] = nxt_c[t][2] | (nxt_c[t][3] << 16);  // code bytes 8g+4 .. 8g+7
      sc[t] = nxt_s[t];
    }
    if (b + 1 < a.nblk) load_block(b + 1);

    f4v acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[mt][t] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ks = 4 * b + i;
      h8 ahi[MT], alo[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const uint4 *p = af + (static_cast<size_t>(mt) * a.n_ksteps + ks) * 2 * 64;
        ahi[mt] = __builtin_bit_cast(h8, p[0]);
        alo[mt] = __builtin_bit_cast(h8, p[64]);
      }
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const uint32_t d = cd[t][i >> 1];
        const h8 bf = decode_codes((i & 1) ? (d >> 8) : d);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[mt], bf, acc[mt][t], 0, 0, 0);
          acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[mt], bf, acc[mt][t], 0, 0, 0);
        }
      }
    }
    // src/kernels.rs:651: acc += scale * block_acc (f32 product, then sum)
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const float s = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(sc[t])));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        f4v p;
#pragma unroll
        for (int q = 0; q < 4; ++q) p[q] = s * acc[mt][t][q];
#pragma unroll
        for (int q = 0; q < 4; ++q) tot[mt][t][q] = tot[mt][t][q] + p[q];
      }
    }
  }
  // lane holds tokens 4g..4g+3 of each token tile, row n of each weight tile
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int m = 16 * (tile0 + mt) + 4 * g + q;
      if (m >= a.n_tok) continue;
      const float inv = a.tok_inv[m];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int row = row_wave + 16 * t + n;
        if (row < a.n_rows) a.y[static_cast<size_t>(m) * a.y_stride + row] = tot[mt][t][q] * inv;
      }
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

template <int MT, int NT>
int launch_mm(const MmArgs &a, int n_tiles, hipStream_t st) {
  const unsigned gx = static_cast<unsigned>((a.n_rows + 64 * NT - 1) / (64 * NT));
  const unsigned gy = static_cast<unsigned>((n_tiles + MT - 1) / MT);
  BH_LAUNCH((pq2_mm_kernel<MT, NT>), dim3(gx, gy), kMmThreads, 0, st, a);
  return ok();
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
  const bool fast = ne0 % 128 == 0 && aligned16(x) && (reinterpret_cast<uintptr_t>(w) & 1u) == 0;
  if (!fast) {
    BH_LAUNCH(pq2_mm_generic_kernel, dim3(static_cast<unsigned>(n_rows), static_cast<unsigned>(n_tok)),
              64, 0, st, w, row_bytes, static_cast<int>(ne0), x, static_cast<int>(n_tok), y,
              static_cast<int>(n_rows));
    return ok();
  }
  const int n_ksteps = static_cast<int>(ne0 / 32);
  const int n_tiles = static_cast<int>((n_tok + 15) / 16);
  const int mt = n_tiles >= 4 ? 4 : (n_tiles >= 2 ? 2 : 1);
  const int tiles_padded = (n_tiles + mt - 1) / mt * mt;
  // scratch: A fragments, then the per-token 2^e and 2^-e
  const size_t frag_bytes = static_cast<size_t>(tiles_padded) * n_ksteps * 2 * 64 * sizeof(uint4);
  const size_t sc_off = (frag_bytes + 255) / 256 * 256;
  char *scratch =
      static_cast<char *>(device_scratch(sc_off + 2 * n_tok * sizeof(float), kScratchMatmul));
  if (scratch == nullptr) return BH_ERR_HIP;
  PrepArgs pa{x, reinterpret_cast<uint4 *>(scratch), reinterpret_cast<float *>(scratch + sc_off),
              reinterpret_cast<float *>(scratch + sc_off) + n_tok, static_cast<int>(ne0),
              static_cast<int>(n_tok), n_ksteps, tiles_padded};
  BH_LAUNCH(pq2_mm_scale_kernel, static_cast<unsigned>(n_tok), kMmThreads, 0, st, pa);
  const unsigned splits = static_cast<unsigned>((n_ksteps * 64 + kMmThreads * 4 - 1) / (kMmThreads * 4));
  BH_LAUNCH(pq2_mm_prep_kernel, dim3(static_cast<unsigned>(tiles_padded), splits), kMmThreads, 0, st, pa);

  MmArgs a{w, pa.afrag, pa.tok_inv, y, row_bytes, static_cast<int>(n_rows),
           static_cast<int>(ne0 / 128), n_ksteps, static_cast<int>(n_tok),
           static_cast<int>(n_rows)};
  // a wave takes 4 row tiles when that still leaves >= 2 blocks per CU
  const bool wide = n_rows >= static_cast<size_t>(256) * 2 * 256;
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
