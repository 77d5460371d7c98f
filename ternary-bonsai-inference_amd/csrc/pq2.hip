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
// is 1/15 of it.
//
// Fused RMSNorm, bit-exact.  The reference sums the 5120 squares of a row
// one after another in f32 (src/kernels.rs:65-68); on quantised embedding
// rows that sequence drifts ~1e-5 from any tree-ordered sum, so the fused
// kernel reproduces the sequence itself.  A block owns kSeqRows rows: its
// rows are staged in LDS, "producer" waves decode them chunk by chunk (128
// columns), store the embedding rows and write the f32 squares to an LDS
// ring laid out column-major, while one "chain" wave adds them in column
// order, one row per lane -- the same additions in the same order as the
// CPU, so the norm output is bit-identical too.  The chain (5120 dependent
// adds, ~10 us) runs under the embedding stores; the norm rows are then
// decoded a second time from LDS and stored.
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

// Plain gather, fast path: row_bytes % 16 == 0, ne0 % 4 == 0, 16-byte
// aligned pointers.  One block per output row.
__global__ __launch_bounds__(kBlock) void pq2_gather_kernel(
    const uint8_t *__restrict__ table, int row_bytes, int ne0, uint32_t n_rows,
    const uint32_t *__restrict__ ids, float *__restrict__ out, uint32_t *bad_id) {
  extern __shared__ uint4 stage[];
  const size_t t = blockIdx.x;
  const uint32_t id = ids[t];
  const int n4 = ne0 >> 2;
  float4 *o4 = reinterpret_cast<float4 *>(out) + t * n4;
  if (id >= n_rows) {  // block-uniform: no barrier is skipped by only some lanes
    if (bad_id != nullptr && threadIdx.x == 0) *bad_id = id;
    for (int f = threadIdx.x; f < n4; f += kBlock) o4[f] = make_float4(0, 0, 0, 0);
    return;
  }
  const uint4 *src = reinterpret_cast<const uint4 *>(table + static_cast<size_t>(id) * row_bytes);
  for (int i = threadIdx.x; i < (row_bytes >> 4); i += kBlock) stage[i] = src[i];
  __syncthreads();
  const uint8_t *rowb = reinterpret_cast<const uint8_t *>(stage);
  for (int f = threadIdx.x; f < n4; f += kBlock) o4[f] = decode4(rowb, f);
}

// Fused gather + RMSNorm with the reference's sequential f32 sum of squares
// (see the file comment).  Requires the fast-path layout.
constexpr int kSeqRows = 16;                 // rows per block = chain lanes
constexpr int kSeqThreads = 256;             // wave 0: chain, waves 1..3: producers
constexpr int kChunkQ = 32;                  // float4 columns per chunk (128 weights)
constexpr int kRingStride = kSeqRows + 1;    // float4 slots per column (padded)

__global__ __launch_bounds__(kSeqThreads) void pq2_gather_rms_seq_kernel(
    const uint8_t *__restrict__ table, int row_bytes, int ne0, uint32_t n_rows,
    const uint32_t *__restrict__ ids, int n_ids, float *__restrict__ out,
    const float *__restrict__ w, float eps, float *__restrict__ out_norm, uint32_t *bad_id) {
  extern __shared__ uint4 smem[];
  const int rb16 = row_bytes >> 4;
  uint4 *stage = smem;                                                       // [kSeqRows][rb16]
  float4 *ring = reinterpret_cast<float4 *>(smem + kSeqRows * rb16);         // [2][kChunkQ][kRingStride]
  __shared__ float row_scale[kSeqRows];
  __shared__ int row_ok[kSeqRows];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const size_t row0 = static_cast<size_t>(blockIdx.x) * kSeqRows;
  const int nr = (n_ids - static_cast<int>(row0)) < kSeqRows ? n_ids - static_cast<int>(row0)
                                                             : kSeqRows;
  const int n4 = ne0 >> 2;

  if (tid < kSeqRows) {
    int ok = 0;
    if (tid < nr) {
      const uint32_t id = ids[row0 + tid];
      ok = id < n_rows;
      if (!ok && bad_id != nullptr) *bad_id = id;
    }
    row_ok[tid] = ok;
  }
  // stage the packed rows (16-byte loads; rows with a bad id are not read)
  for (int i = tid; i < nr * rb16; i += kSeqThreads) {
    const int r = i / rb16;
    const int k = i - r * rb16;
    const uint32_t id = ids[row0 + r];
    if (id < n_rows)
      stage[i] = reinterpret_cast<const uint4 *>(table + static_cast<size_t>(id) * row_bytes)[k];
  }
  __syncthreads();

  const int n_chunks = (n4 + kChunkQ - 1) / kChunkQ;
  float ss = 0.0f;  // chain lane `lane` accumulates row `lane`
  for (int c = 0; c <= n_chunks; ++c) {
    if (wave != 0) {
      if (c < n_chunks) {
        float4 *dst = ring + (c & 1) * (kChunkQ * kRingStride);
        for (int i = tid - 64; i < kSeqRows * kChunkQ; i += kSeqThreads - 64) {
          const int r = i / kChunkQ;
          const int q = i - r * kChunkQ;
          const int f = c * kChunkQ + q;
          float4 t = make_float4(0.f, 0.f, 0.f, 0.f);  // adding +0 leaves a sum unchanged
          if (r < nr && f < n4) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (row_ok[r]) {
              v = decode4(reinterpret_cast<const uint8_t *>(stage + r * rb16), f);
              t = make_float4(v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w);
            }
            reinterpret_cast<float4 *>(out)[(row0 + r) * n4 + f] = v;
          }
          dst[q * kRingStride + r] = t;
        }
      }
    } else if (c > 0 && lane < kSeqRows) {
      const float4 *src = ring + ((c - 1) & 1) * (kChunkQ * kRingStride);
#pragma unroll 8
      for (int q = 0; q < kChunkQ; ++q) {
        const float4 t = src[q * kRingStride + lane];
        ss += t.x;
        ss += t.y;
        ss += t.z;
        ss += t.w;
      }
    }
    __syncthreads();
  }
  if (wave == 0 && lane < kSeqRows) {
    // src/kernels.rs:69-70: mean = ss / n; scale = 1 / sqrt(mean + eps)
    row_scale[lane] = 1.0f / sqrtf(ss / static_cast<float>(ne0) + eps);
  }
  __syncthreads();
  // norm rows: column-outer so each lane loads its weight float4 once, then
  // writes that column of every row (stores stay coalesced along each row)
  const float4 *w4 = reinterpret_cast<const float4 *>(w);
  for (int f = tid; f < n4; f += kSeqThreads) {
    const float4 wv = w4[f];
#pragma unroll 4
    for (int r = 0; r < nr; ++r) {
      float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
      if (row_ok[r]) {
        const float4 v = decode4(reinterpret_cast<const uint8_t *>(stage + r * rb16), f);
        const float scale = row_scale[r];
        o = make_float4((v.x * scale) * wv.x, (v.y * scale) * wv.y, (v.z * scale) * wv.z,
                        (v.w * scale) * wv.w);
      }
      reinterpret_cast<float4 *>(out_norm)[(row0 + r) * n4 + f] = o;
    }
  }
}

size_t seq_smem_bytes(size_t row_bytes) {
  return kSeqRows * row_bytes + 2 * kChunkQ * kRingStride * sizeof(float4);
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
  for (int j = threadIdx.x; j < ne0; j += kBlock) orow[j] = weight(j);
  if constexpr (NORM) {
    // the reference's sequential f32 sum (src/kernels.rs:65-68), one lane;
    // this path only serves layouts the staged kernels cannot take
    __syncthreads();
    if (threadIdx.x == 0) {
      float ss = 0.0f;
      for (int j = 0; j < ne0; ++j) ss += orow[j] * orow[j];
      lds[0] = 1.0f / sqrtf(ss / static_cast<float>(ne0) + eps);
    }
    __syncthreads();
    const float scale = lds[0];
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
  if (fast && norm && seq_smem_bytes(row_bytes) <= 65536) {
    const unsigned sgrid = static_cast<unsigned>((n_ids + kSeqRows - 1) / kSeqRows);
    BH_LAUNCH(pq2_gather_rms_seq_kernel, sgrid, kSeqThreads, seq_smem_bytes(row_bytes), st,
              table, static_cast<int>(row_bytes), static_cast<int>(ne0), nr, ids,
              static_cast<int>(n_ids), out, w, eps, out_norm, bad_id);
  } else if (fast && !norm) {
    BH_LAUNCH(pq2_gather_kernel, grid, kBlock, row_bytes, st, table, static_cast<int>(row_bytes),
              static_cast<int>(ne0), nr, ids, out, bad_id);
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
