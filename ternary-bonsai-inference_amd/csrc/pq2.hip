// PQ2_0 embedding gather-dequant for gfx950, alone and fused with RMSNorm.
//
//   bh_pq2_embed_gather      batched Weights::row_f32 on token_embd.weight
//                            (src/weights.rs:333-349, src/prefill.rs:143-154)
//                            = kernels::decode_pq2_0_row per id (src/kernels.rs:214-229)
//   bh_pq2_embed_gather_rms  + the first rms_norm (src/forward.rs:691, 701-702)
//
// PQ2_0 layout (src/kernels.rs:204-229): a row of ne0 weights is ceil(ne0/128)
// blocks of 34 bytes: a little-endian f16 scale, then 32 bytes holding 128
// 2-bit codes, LSB first (weight j of the block: byte j/4, bits 2*(j%4)).
// Weight = (code - 1) * scale.
//
// Design.  One block of 256 lanes per output row.  The packed row (1360 B for
// ne0 = 5120) is first staged into LDS with 16-byte loads by the first
// row_bytes/16 lanes -- one HBM transaction stream per row, independent of
// the odd 34-byte block stride.  Each lane then produces float4 outputs: a
// float4 of weights 4q..4q+3 of block b is exactly byte q of that block's
// codes, so one LDS byte plus the block's scale give one 16-byte coalesced
// store.  The output (20 KB per row) dominates the traffic; the packed read
// is 1/15 of it.  With the fused norm, the sum of squares is accumulated
// while the embedding row is stored, reduced across the block, and the norm
// row is decoded again from LDS (no second HBM read).
//
// Bit-exactness: the f16 scale is widened with integer arithmetic (exact for
// all patterns, see half_bits_to_f32_bits) and the weight is one multiply of
// an exact small integer by it, so the product is exactly the CPU's.
#include <hip/hip_runtime.h>

#include <string>

#include "common.hpp"

namespace bh {
namespace {

constexpr int kBlock = 256;
constexpr int kPq2Block = 34;

// Decodes float4 number f (weights 4f..4f+3 of the row) from the staged row.
__device__ __forceinline__ float4 decode4(const uint8_t *rowb, int f) {
  const int b = f >> 5;  // 32 float4 per 128-weight block
  const int q = f & 31;
  const uint8_t *blk = rowb + b * kPq2Block;
  const uint32_t h = static_cast<uint32_t>(blk[0]) | (static_cast<uint32_t>(blk[1]) << 8);
  const float scale = __uint_as_float(half_bits_to_f32_bits(h));
  const bool finite = (h & 0x7c00u) != 0x7c00u;
  const uint32_t c = blk[2 + q];
  return make_float4(pq2_weight(c & 3u, scale, finite), pq2_weight((c >> 2) & 3u, scale, finite),
                     pq2_weight((c >> 4) & 3u, scale, finite),
                     pq2_weight((c >> 6) & 3u, scale, finite));
}

// Fast path: row_bytes % 16 == 0, ne0 % 4 == 0, 16-byte aligned pointers.
template <bool NORM>
__global__ __launch_bounds__(kBlock) void pq2_gather_kernel(
    const uint8_t *__restrict__ table, int row_bytes, int ne0, uint32_t n_rows,
    const uint32_t *__restrict__ ids, float *__restrict__ out, const float *__restrict__ w,
    float eps, float *__restrict__ out_norm, uint32_t *bad_id) {
  extern __shared__ uint4 stage[];
  __shared__ float lds[kBlock / 64];
  const size_t t = blockIdx.x;
  const uint32_t id = ids[t];
  const int n4 = ne0 >> 2;
  float4 *o4 = reinterpret_cast<float4 *>(out) + t * n4;
  if (id >= n_rows) {  // block-uniform: no barrier is skipped by only some lanes
    if (bad_id != nullptr && threadIdx.x == 0) *bad_id = id;
    for (int f = threadIdx.x; f < n4; f += kBlock) o4[f] = make_float4(0, 0, 0, 0);
    if constexpr (NORM) {
      float4 *n4p = reinterpret_cast<float4 *>(out_norm) + t * n4;
      for (int f = threadIdx.x; f < n4; f += kBlock) n4p[f] = make_float4(0, 0, 0, 0);
    }
    return;
  }
  const uint4 *src = reinterpret_cast<const uint4 *>(table + static_cast<size_t>(id) * row_bytes);
  for (int i = threadIdx.x; i < (row_bytes >> 4); i += kBlock) stage[i] = src[i];
  __syncthreads();
  const uint8_t *rowb = reinterpret_cast<const uint8_t *>(stage);

  float ss = 0.0f;
  for (int f = threadIdx.x; f < n4; f += kBlock) {
    const float4 v = decode4(rowb, f);
    o4[f] = v;
    if constexpr (NORM) {
      ss += v.x * v.x;
      ss += v.y * v.y;
      ss += v.z * v.z;
      ss += v.w * v.w;
    }
  }
  if constexpr (NORM) {
    ss = group_reduce<kBlock>(ss, SumOp{}, lds);
    const float scale = 1.0f / sqrtf(ss / static_cast<float>(ne0) + eps);
    const float4 *w4 = reinterpret_cast<const float4 *>(w);
    float4 *n4p = reinterpret_cast<float4 *>(out_norm) + t * n4;
    for (int f = threadIdx.x; f < n4; f += kBlock) {
      const float4 v = decode4(rowb, f);
      const float4 wv = w4[f];
      n4p[f] = make_float4((v.x * scale) * wv.x, (v.y * scale) * wv.y, (v.z * scale) * wv.z,
                           (v.w * scale) * wv.w);
    }
  }
}

// Any ne0 / alignment: byte reads straight from the table.
template <bool NORM>
__global__ __launch_bounds__(kBlock) void pq2_gather_loop_kernel(
    const uint8_t *__restrict__ table, size_t row_bytes, int ne0, uint32_t n_rows,
    const uint32_t *__restrict__ ids, float *__restrict__ out, const float *__restrict__ w,
    float eps, float *__restrict__ out_norm, uint32_t *bad_id) {
  __shared__ float lds[kBlock / 64];
  const size_t t = blockIdx.x;
  const uint32_t id = ids[t];
  float *orow = out + t * ne0;
  if (id >= n_rows) {
    if (bad_id != nullptr && threadIdx.x == 0) *bad_id = id;
    for (int j = threadIdx.x; j < ne0; j += kBlock) {
      orow[j] = 0.0f;
      if constexpr (NORM) out_norm[t * ne0 + j] = 0.0f;
    }
    return;
  }
  const uint8_t *rowb = table + static_cast<size_t>(id) * row_bytes;
  auto weight = [&](int j) {
    const uint8_t *blk = rowb + (j >> 7) * kPq2Block;
    const uint32_t h = static_cast<uint32_t>(blk[0]) | (static_cast<uint32_t>(blk[1]) << 8);
    const int jj = j & 127;
    const uint32_t code = (static_cast<uint32_t>(blk[2 + (jj >> 2)]) >> ((jj & 3) * 2)) & 3u;
    return pq2_weight(code, __uint_as_float(half_bits_to_f32_bits(h)), (h & 0x7c00u) != 0x7c00u);
  };
  float ss = 0.0f;
  for (int j = threadIdx.x; j < ne0; j += kBlock) {
    const float v = weight(j);
    orow[j] = v;
    ss += v * v;
  }
  if constexpr (NORM) {
    ss = group_reduce<kBlock>(ss, SumOp{}, lds);
    const float scale = 1.0f / sqrtf(ss / static_cast<float>(ne0) + eps);
    for (int j = threadIdx.x; j < ne0; j += kBlock)
      out_norm[t * ne0 + j] = (weight(j) * scale) * w[j];
  }
}

int gather_impl(const uint8_t *table, size_t ne0, size_t n_rows, const uint32_t *ids,
                size_t n_ids, const float *w, float eps, float *out, float *out_norm,
                uint32_t *bad_id, hipStream_t st, bool norm) {
  if (n_ids == 0 || ne0 == 0) return ok();
  if (ne0 > 0x7fffffffu || n_ids > 0x7fffffffu)
    return fail(BH_ERR_SHAPE, "pq2 gather: ne0 or n_ids exceeds 2^31-1");
  if (n_rows > 0xffffffffu) return fail(BH_ERR_SHAPE, "pq2 gather: n_rows exceeds 2^32-1");
  const size_t row_bytes = bh_pq2_row_bytes(ne0);
  const unsigned grid = static_cast<unsigned>(n_ids);
  const uint32_t nr = static_cast<uint32_t>(n_rows);
  const bool fast = (row_bytes % 16 == 0) && (ne0 % 4 == 0) && row_bytes <= 65536 &&
                    aligned16(table) && aligned16(out) &&
                    (!norm || (aligned16(out_norm) && aligned16(w)));
  if (fast) {
    if (norm) {
      BH_LAUNCH((pq2_gather_kernel<true>), grid, kBlock, row_bytes, st, table,
                static_cast<int>(row_bytes), static_cast<int>(ne0), nr, ids, out, w, eps,
                out_norm, bad_id);
    } else {
      BH_LAUNCH((pq2_gather_kernel<false>), grid, kBlock, row_bytes, st, table,
                static_cast<int>(row_bytes), static_cast<int>(ne0), nr, ids, out, w, eps,
                out_norm, bad_id);
    }
  } else {
    if (norm) {
      BH_LAUNCH((pq2_gather_loop_kernel<true>), grid, kBlock, 0, st, table, row_bytes,
                static_cast<int>(ne0), nr, ids, out, w, eps, out_norm, bad_id);
    } else {
      BH_LAUNCH((pq2_gather_loop_kernel<false>), grid, kBlock, 0, st, table, row_bytes,
                static_cast<int>(ne0), nr, ids, out, w, eps, out_norm, bad_id);
    }
  }
  return ok();
}

}  // namespace
}  // namespace bh

using namespace bh;

extern "C" int bh_pq2_embed_gather(const uint8_t *table, size_t ne0, size_t n_rows,
                                   const uint32_t *ids, size_t n_ids, float *out,
                                   uint32_t *bad_id, bh_stream stream) {
  if (n_ids && ne0 && (!table || !ids || !out))
    return fail(BH_ERR_ARG, "pq2_embed_gather: null pointer");
  return gather_impl(table, ne0, n_rows, ids, n_ids, nullptr, 0.0f, out, nullptr, bad_id,
                     as_stream(stream), false);
}

extern "C" int bh_pq2_embed_gather_rms(const uint8_t *table, size_t ne0, size_t n_rows,
                                       const uint32_t *ids, size_t n_ids, const float *w,
                                       size_t w_len, float eps, float *out_embed,
                                       float *out_norm, uint32_t *bad_id, bh_stream stream) {
  if (w_len != ne0)
    return fail(BH_ERR_SHAPE, "pq2_embed_gather_rms: weight len " + std::to_string(w_len) +
                                  " != ne0 " + std::to_string(ne0));
  if (n_ids && ne0 && (!table || !ids || !out_embed || !out_norm || !w))
    return fail(BH_ERR_ARG, "pq2_embed_gather_rms: null pointer");
  return gather_impl(table, ne0, n_rows, ids, n_ids, w, eps, out_embed, out_norm, bad_id,
                     as_stream(stream), true);
}
