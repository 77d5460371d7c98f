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
// Design.  One float4 of output per lane over the flat [n_ids][ne0/4]
// range: the lane reads its 128-block's f16 scale (an aligned halfword:
// blocks start on even bytes) and one code byte -- exactly the 4 weights of
// its float4 -- and stores 16 bytes.  The output (20 KB per row) dominates the
// traffic; the packed read (1360 B per row, cache-resident across the 320
// lanes that share it) is 1/15 of it.
//
// Fused RMSNorm, bit-exact.  The reference sums the 5120 squares of a row
// one after another in f32 (src/kernels.rs:65-68); on quantised embedding
// rows that sequence drifts ~1e-5 from any tree-ordered sum, so the fused
// kernel reproduces the sequence itself.  A block owns kFusedRows rows: its
// rows are staged in LDS, "producer" waves decode them chunk by chunk (256
// or 512 columns), store the embedding rows and write the f32 squares to an LDS
// ring laid out column-major, while one "chain" wave adds them in column
// order, one row per lane -- the same additions in the same order as the
// CPU, so the norm output is bit-identical too.  The chain (5120 dependent
// adds, ~21 us) runs under the embedding stores; the norm rows are then
// decoded a second time from LDS and stored.  Batches of at least 16 rows per
// CU take two launches instead, with flat writers: the row scales come from
// runs of identical squares evaluated in closed form (seqsum.hpp), computed
// by the first blocks of the launch that writes the embedding rows, and a
// second launch writes the norm rows.
//
// Bit-exactness: the f16 scale is widened with integer arithmetic (exact for
// all patterns, see half_bits_to_f32_bits) and the weight is one multiply of
// an exact small integer by it, so the product is exactly the CPU's.
#include <hip/hip_runtime.h>

#include <string>

#include "common.hpp"
#include "seqsum.hpp"

namespace bh {
namespace {

constexpr int kBlock = 256;
constexpr int kPq2Block = 34;
constexpr size_t kMaxSeqSmem = 128 * 1024;  // LDS cap of a fused block (gfx950: 160 KB per CU)


// ---------------------------------------------------------------------------
// Fused gather + RMSNorm with the reference's sequential f32 sum of squares:
// one launch, one block of kFusedThreads lanes per kFusedRows output rows.
// ---------------------------------------------------------------------------
// Block shapes: kFusedRows rows per block (= chain lanes), kFusedThreads
// lanes (wave 0 the chain, the others producers) and kChunkQ float4 columns
// per chunk of the ring (one barrier per chunk).

// LDS of a block of `rows` rows: staged packed rows, the f32 scale of every
// (row, 128-block) and the two-chunk ring of squared weights.
size_t fused_smem_bytes(size_t row_bytes, int rows, int chunk_q) {
  const size_t n_scales = (rows * (row_bytes / kPq2Block) + 3) & ~static_cast<size_t>(3);
  return rows * row_bytes + n_scales * sizeof(float) + 2 * chunk_q * (rows + 1) * sizeof(float4);
}

struct GatherArgs {
  const uint8_t *table;
  const uint32_t *ids;
  float *out;       // embedding rows
  float *out_norm;  // norm rows
  const float *w;
  uint32_t *bad_id;
  int row_bytes, ne0, n_ids;
  uint32_t n_rows;
  float eps;
};

// Phase 1 (column chunks of 4 kChunkQ weights, ring of squares):
//   producer waves decode chunk c of all the block's rows, store those
//   embedding float4 and write their f32 squares to the ring, column-major;
//   the chain wave (lane = row) adds chunk c-1 in column order -- the same
//   additions in the same order as src/kernels.rs:65-68, so the row scale
//   is bit-identical to the CPU's.  The chain is latency-bound (~10 cycles
//   per dependent add, ~21 us for 5120 weights) and runs under the stores.
// Phase 2: all waves decode the rows again from LDS and store the norm rows
//   (v * scale) * w (src/kernels.rs:71-73), flat over the block's rows.
template <int kFusedRows, int kFusedThreads, int kChunkQ>
__global__ __launch_bounds__(kFusedThreads) void pq2_gather_rms_kernel(GatherArgs a) {
  constexpr int kRingStride = kFusedRows + 1;  // float4 slots per column (padded)
  extern __shared__ uint4 smem[];
  __shared__ int row_ok[kFusedRows];
  __shared__ float row_scale[kFusedRows];
  const int rb16 = a.row_bytes >> 4;
  const int nblk = a.row_bytes / kPq2Block;
  uint4 *stage = smem;                                                  // [rows][rb16]
  float *scales = reinterpret_cast<float *>(smem + kFusedRows * rb16);  // [rows][nblk]
  float4 *ring = reinterpret_cast<float4 *>(scales + ((kFusedRows * nblk + 3) & ~3));
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const size_t row0 = static_cast<size_t>(blockIdx.x) * kFusedRows;
  const int nr = (a.n_ids - static_cast<int>(row0)) < kFusedRows ? a.n_ids - static_cast<int>(row0)
                                                                 : kFusedRows;
  const int n4 = a.ne0 >> 2;

  if (tid < kFusedRows) {
    int okr = 0;
    if (tid < nr) {
      const uint32_t id = a.ids[row0 + tid];
      okr = id < a.n_rows;
      if (!okr && a.bad_id != nullptr) *a.bad_id = id;
    }
    row_ok[tid] = okr;
  }
  for (int i = tid; i < nr * rb16; i += kFusedThreads) {
    const int r = i / rb16;
    const uint32_t id = a.ids[row0 + r];
    if (id < a.n_rows)
      stage[i] = reinterpret_cast<const uint4 *>(a.table + static_cast<size_t>(id) * a.row_bytes)[i - r * rb16];
  }
  __syncthreads();
  // f32 scale of every staged 128-block (the f16 bits kept in the scale slot
  // would be needed only for non-finite scales, which are re-read from the row)
  for (int i = tid; i < nr * nblk; i += kFusedThreads) {
    const int r = i / nblk;
    const uint8_t *bp = reinterpret_cast<const uint8_t *>(stage + r * rb16) + (i - r * nblk) * kPq2Block;
    const uint32_t h = static_cast<uint32_t>(bp[0]) | (static_cast<uint32_t>(bp[1]) << 8);
    scales[i] = __uint_as_float(half_bits_to_f32_bits(h));
  }
  __syncthreads();

  const int n_chunks = (n4 + kChunkQ - 1) / kChunkQ;
  float ss = 0.0f;  // chain lane `lane` accumulates row `lane`
  for (int c = 0; c <= n_chunks; ++c) {
    if (wave != 0) {
      if (c < n_chunks) {
        float4 *dst = ring + (c & 1) * (kChunkQ * kRingStride);
        for (int i = tid - 64; i < kFusedRows * kChunkQ; i += kFusedThreads - 64) {
          const int r = i / kChunkQ;  // lanes walk a row's kChunkQ columns: long store runs
          const int q = i - r * kChunkQ;
          const int f = c * kChunkQ + q;
          float4 t = make_float4(0.f, 0.f, 0.f, 0.f);  // adding +0 leaves a sum unchanged
          if (r < nr && f < n4) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (row_ok[r]) {
              const uint8_t *rowb = reinterpret_cast<const uint8_t *>(stage + r * rb16);
              const int b = f >> 5;
              const uint32_t h = static_cast<uint32_t>(rowb[b * kPq2Block]) |
                                 (static_cast<uint32_t>(rowb[b * kPq2Block + 1]) << 8);
              const uint32_t code = rowb[b * kPq2Block + 2 + (f & 31)];
              const float sc = scales[r * nblk + b];
              const bool finite = (h & 0x7c00u) != 0x7c00u;
              v = make_float4(pq2_weight(code & 3u, sc, finite), pq2_weight((code >> 2) & 3u, sc, finite),
                              pq2_weight((code >> 4) & 3u, sc, finite), pq2_weight((code >> 6) & 3u, sc, finite));
              t = make_float4(v.x * v.x, v.y * v.y, v.z * v.z, v.w * v.w);
            }
            store_stream(reinterpret_cast<float4 *>(a.out) + (row0 + r) * n4 + f, v);
          }
          dst[q * kRingStride + r] = t;
        }
      }
    } else if (c > 0 && lane < kFusedRows) {
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
  if (wave == 0 && lane < kFusedRows) {
    // src/kernels.rs:69-70: mean = ss / n; scale = 1 / sqrt(mean + eps)
    row_scale[lane] = 1.0f / sqrtf(ss / static_cast<float>(a.ne0) + a.eps);
  }
  __syncthreads();

  const float4 *w4 = reinterpret_cast<const float4 *>(a.w);
  float4 *on = reinterpret_cast<float4 *>(a.out_norm) + row0 * n4;
  const int total = nr * n4;
  for (int i = tid; i < total; i += kFusedThreads) {
    const int r = i / n4;
    const int f = i - r * n4;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    if (row_ok[r]) {
      const uint8_t *rowb = reinterpret_cast<const uint8_t *>(stage + r * rb16);
      const int b = f >> 5;
      const uint32_t h = static_cast<uint32_t>(rowb[b * kPq2Block]) |
                         (static_cast<uint32_t>(rowb[b * kPq2Block + 1]) << 8);
      const uint32_t code = rowb[b * kPq2Block + 2 + (f & 31)];
      const float sc = scales[r * nblk + b];
      const bool finite = (h & 0x7c00u) != 0x7c00u;
      const float4 v = make_float4(pq2_weight(code & 3u, sc, finite), pq2_weight((code >> 2) & 3u, sc, finite),
                                   pq2_weight((code >> 4) & 3u, sc, finite), pq2_weight((code >> 6) & 3u, sc, finite));
      const float4 wv = w4[f];
      const float rs = row_scale[r];
      o = make_float4((v.x * rs) * wv.x, (v.y * rs) * wv.y, (v.z * rs) * wv.z, (v.w * rs) * wv.w);
    }
    store_stream(on + i, o);
  }
}

// Decodes float4 f of the packed row at `rowb` straight from global memory
// (the scale halfword and one code byte; the row is 16-byte aligned and a
// block starts on an even byte, so the halfword load is aligned).
__device__ __forceinline__ float4 decode4_global(const uint8_t *rowb, int f) {
  const uint8_t *blk = rowb + (f >> 5) * kPq2Block;
  const uint32_t h = *reinterpret_cast<const uint16_t *>(blk);
  const uint32_t c = blk[2 + (f & 31)];
  const float scale = __uint_as_float(half_bits_to_f32_bits(h));
  const bool finite = (h & 0x7c00u) != 0x7c00u;
  return make_float4(pq2_weight(c & 3u, scale, finite), pq2_weight((c >> 2) & 3u, scale, finite),
                     pq2_weight((c >> 4) & 3u, scale, finite),
                     pq2_weight((c >> 6) & 3u, scale, finite));
}

// ---------------------------------------------------------------------------
// Gather + RMSNorm in two launches with flat writers.
// ---------------------------------------------------------------------------
// Launch 1 (pq2_scale_embed_kernel): its first blocks compute every row's
// 1 / sqrt(ss / n + eps)
// with ss the reference's sequential f32 sum of squares, bit for bit, without
// decoding the row: on a block of ternary codes (0, 1, 2) every square is d*d
// or +0, and +0 leaves the sum unchanged, so the block adds d*d as many times
// as it has codes other than 1 -- a run that repeat_add_f32 evaluates in
// closed form.  A block holding code 3 (square 4*d*d) or a non-finite scale
// is added weight by weight instead.  One lane walks one row, so the walk is
// a chain of ~55 dependent steps (one per block plus one per binade the sum
// crosses, ~20 us); the launch's other blocks write the embedding rows from a
// flat grid meanwhile.  Launch 2 (pq2_norm_write_kernel) writes the norm rows
// from a flat grid.  Both writers keep the streaming-store shape: no block
// stores a region longer than 4 KB.
constexpr int kScaleRows = 16;  // rows per scale block: one per lane of its walk

// Logical block of physical block p when a grid of 8 * per blocks is
// numbered XCD-contiguously: the hardware hands block p to XCD p % 8, and
// that XCD takes logical blocks [(p % 8) * per, (p % 8 + 1) * per) in order.
// (Only the speed depends on that dispatch order, never the results.)
__device__ __forceinline__ unsigned xcd_block(unsigned p, unsigned per) {
  return (p & 7u) * per + (p >> 3);
}

// Sum-of-squares summary of one 128-weight block of a staged row: the run
// value d*d (f32 bits) and the run length, or the fallback flag.
struct BlockRun {
  uint32_t xbits;
  uint32_t n;  // bit 31: add this block weight by weight
};

// Scale block `sblk` of launch 1: rows sblk*kScaleRows .. (+kScaleRows).
__device__ __forceinline__ void row_scale_block(const GatherArgs &a, float *row_scale,
                                                unsigned sblk, BlockRun *runs) {
  const int nblk = a.row_bytes / kPq2Block;
  const int tid = threadIdx.x;
  const size_t row0 = static_cast<size_t>(sblk) * kScaleRows;
  const int nr = (a.n_ids - static_cast<int>(row0)) < kScaleRows ? a.n_ids - static_cast<int>(row0)
                                                                 : kScaleRows;
  // one lane per (row, block), straight from the table: count the codes
  // other than 1 among the block's valid weights, flag code 3 and
  // non-finite scales.  The block's 34 bytes start on an even byte: eight
  // aligned words and one halfword cover them without reading past it.
  // A lane takes up to kScalePairs pairs per round and issues all their
  // loads (ids, then table words) before it uses any: under the writers'
  // HBM traffic a load round trip is long, and the walk waits for this.
  constexpr int kScalePairs = 4;
  const int total = nr * nblk;
  for (int base = 0; base < total; base += 256 * kScalePairs) {
    uint32_t idp[kScalePairs];
#pragma unroll
    for (int p = 0; p < kScalePairs; ++p) {
      const int i = base + p * 256 + tid;
      idp[p] = i < total ? a.ids[row0 + i / nblk] : a.n_rows;
    }
    uint32_t dw[kScalePairs][8];
    uint32_t h16[kScalePairs];
#pragma unroll
    for (int p = 0; p < kScalePairs; ++p) {
      const int i = base + p * 256 + tid;
      const int b = i - (i / nblk) * nblk;
      const bool even = (b & 1) == 0;  // block start 4-aligned (rows are 16-aligned)
      h16[p] = 0u;
#pragma unroll
      for (int k = 0; k < 8; ++k) dw[p][k] = 0u;
      if (idp[p] < a.n_rows) {
        const uint8_t *blk = a.table + static_cast<size_t>(idp[p]) * a.row_bytes + b * kPq2Block;
        const uint32_t *w32 = reinterpret_cast<const uint32_t *>(blk + (even ? 0 : 2));
        h16[p] = *reinterpret_cast<const uint16_t *>(blk + (even ? 32 : 0));
#pragma unroll
        for (int k = 0; k < 8; ++k) dw[p][k] = w32[k];
      }
    }
#pragma unroll
    for (int p = 0; p < kScalePairs; ++p) {
      const int i = base + p * 256 + tid;
      if (idp[p] >= a.n_rows) continue;  // past the pairs, or a bad id (no scale)
      const int b = i - (i / nblk) * nblk;
      const bool even = (b & 1) == 0;
      const uint32_t h = even ? (dw[p][0] & 0xffffu) : h16[p];
      const int valid = (a.ne0 - b * 128) < 128 ? a.ne0 - b * 128 : 128;
      uint32_t ones = 0, threes = 0;
#pragma unroll
      for (int k = 0; k < 8; ++k) {  // 16 codes per 32-bit word
        const uint32_t w =
            even ? ((dw[p][k] >> 16) | ((k < 7 ? dw[p][k < 7 ? k + 1 : 0] : h16[p]) << 16)) : dw[p][k];
        const int lo = valid - 16 * k;
        const uint32_t mask = lo >= 16 ? 0x55555555u : (lo <= 0 ? 0u : 0x55555555u & ((1u << (2 * lo)) - 1u));
        const uint32_t t = w ^ 0x55555555u;  // code 1 -> 00
        ones += __popc(~(t | (t >> 1)) & mask);
        threes |= w & (w >> 1) & mask;
      }
      const bool finite = (h & 0x7c00u) != 0x7c00u;
      const float d = __uint_as_float(half_bits_to_f32_bits(h));
      BlockRun br;
      br.xbits = __float_as_uint(d * d);
      br.n = static_cast<uint32_t>(valid) - ones;
      if (threes != 0u || !finite) br.n |= 0x80000000u;
      runs[i] = br;
    }
  }
  __syncthreads();
  if (tid >= nr) return;
  const uint32_t id = a.ids[row0 + tid];
  if (id >= a.n_rows) return;
  // the walk is the launch's latency-critical path: its wave goes first
  // when it shares a SIMD with the writer waves
  __builtin_amdgcn_s_setprio(3);
  const BlockRun *rr = runs + tid * nblk;
  // Each lane walks its own row's blocks; one repeat_add_step_f32 per loop
  // trip, and a lane whose block is done moves to its next one in the same
  // trip, so the wave's trips are the most any of its rows needs rather
  // than the sum of per-block maxima.
  float ss = 0.0f;
  int b = 0;
  BlockRun cur = rr[0];
  BlockRun next = rr[nblk > 1 ? 1 : 0];  // an index select: both from LDS
  while (b < nblk) {
    uint32_t left = cur.n;
    if (left & 0x80000000u) {
      // weight by weight, as src/kernels.rs:65-68 (code 3 or a non-finite scale)
      const uint8_t *blk = a.table + static_cast<size_t>(id) * a.row_bytes + b * kPq2Block;
      const uint32_t h = *reinterpret_cast<const uint16_t *>(blk);
      const float sc = __uint_as_float(half_bits_to_f32_bits(h));
      const bool finite = (h & 0x7c00u) != 0x7c00u;
      const int valid = (a.ne0 - b * 128) < 128 ? a.ne0 - b * 128 : 128;
      for (int j = 0; j < valid; ++j) {
        const uint32_t code = (static_cast<uint32_t>(blk[2 + (j >> 2)]) >> ((j & 3) * 2)) & 3u;
        const float v = pq2_weight(code, sc, finite);
        ss += v * v;  // no contraction: built with -ffp-contract=off
      }
      left = 0u;
    } else if (left != 0u && cur.xbits != 0u) {
      left = repeat_add_step_f32(ss, __uint_as_float(cur.xbits), left);
    } else {
      left = 0u;  // d = 0 or only code 1: the squares are all +0
    }
    cur.n = left;
    if (left == 0u) {
      ++b;
      cur = next;
      if (b + 1 < nblk) next = rr[b + 1];
    }
  }
  // src/kernels.rs:69-70: mean = ss / n; scale = 1 / sqrt(mean + eps)
  row_scale[row0 + tid] = 1.0f / sqrtf(ss / static_cast<float>(a.ne0) + a.eps);
}

// Launch 1: blocks [0, n_scale) compute the row scales (dispatched first, so
// their walks run under the stores), the rest write the embedding rows, one
// float4 per lane over the flat [n_ids][ne0/4] range.
__global__ __launch_bounds__(256) void pq2_scale_embed_kernel(GatherArgs a, float *row_scale,
                                                              unsigned n_scale, unsigned s_per,
                                                              unsigned e_per) {
  extern __shared__ BlockRun runs[];  // [kScaleRows][nblk]
  if (blockIdx.x < n_scale) {
    // scale blocks in the same XCD-contiguous order as the writers, so a
    // row's summary pass runs on the XCD that writes it
    const unsigned sblk = xcd_block(blockIdx.x, s_per);
    if (sblk * kScaleRows < static_cast<unsigned>(a.n_ids)) row_scale_block(a, row_scale, sblk, runs);
    return;
  }
  // one float4 per lane; the writer blocks are numbered XCD-contiguously:
  // the blocks one XCD runs (every 8th) write one contiguous range of rows,
  // so each gathered row is fetched into one XCD's L2 (and its address
  // translations warmed there) instead of the five XCDs its 5 blocks would
  // otherwise spread over
  const uint32_t n4 = static_cast<uint32_t>(a.ne0) >> 2;
  const uint32_t idx = xcd_block(blockIdx.x - n_scale, e_per) * 256u + threadIdx.x;
  if (idx >= static_cast<uint32_t>(a.n_ids) * n4) return;
  const uint32_t t = idx / n4;
  const uint32_t f = idx - t * n4;
  const uint32_t id = a.ids[t];
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (id < a.n_rows) {
    v = decode4_global(a.table + static_cast<size_t>(id) * a.row_bytes, f);
  } else if (f == 0 && a.bad_id != nullptr) {
    *a.bad_id = id;
  }
  store_stream(reinterpret_cast<float4 *>(a.out) + idx, v);
}

size_t scale_smem_bytes(size_t row_bytes) {
  return kScaleRows * (row_bytes / kPq2Block) * sizeof(BlockRun);
}

// Plain gather: one float4 of output per lane over the flat [n_ids][ne0/4]
// range (fits 32 bits: checked by the host).
__global__ __launch_bounds__(256) void pq2_rows_write_kernel(GatherArgs a, unsigned per) {
  const uint32_t n4 = static_cast<uint32_t>(a.ne0) >> 2;
  // XCD-contiguous block order: a row's blocks share one XCD's L2
  const uint32_t idx = xcd_block(blockIdx.x, per) * 256u + threadIdx.x;
  if (idx >= static_cast<uint32_t>(a.n_ids) * n4) return;
  const uint32_t t = idx / n4;
  const uint32_t f = idx - t * n4;
  const uint32_t id = a.ids[t];
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
  if (id < a.n_rows) {
    o = decode4_global(a.table + static_cast<size_t>(id) * a.row_bytes, f);
  } else if (f == 0 && a.bad_id != nullptr) {
    *a.bad_id = id;
  }
  store_stream(reinterpret_cast<float4 *>(a.out) + idx, o);
}

// Launch 2: the norm rows (v * scale) * w (src/kernels.rs:71-73), one float4
// per lane over the flat [n_ids][ne0/4] range, with the row scales of
// launch 1 (bad ids: zeros, as the embedding rows).
__global__ __launch_bounds__(256) void pq2_norm_write_kernel(GatherArgs a, const float *row_scale,
                                                             unsigned per) {
  const uint32_t n4 = static_cast<uint32_t>(a.ne0) >> 2;
  const uint32_t idx = xcd_block(blockIdx.x, per) * 256u + threadIdx.x;  // as launch 1
  if (idx >= static_cast<uint32_t>(a.n_ids) * n4) return;
  const uint32_t t = idx / n4;
  const uint32_t f = idx - t * n4;
  const uint32_t id = a.ids[t];
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
  if (id < a.n_rows) {
    const float rs = row_scale[t];
    const float4 wv = reinterpret_cast<const float4 *>(a.w)[f];
    const float4 v = decode4_global(a.table + static_cast<size_t>(id) * a.row_bytes, f);
    o = make_float4((v.x * rs) * wv.x, (v.y * rs) * wv.y, (v.z * rs) * wv.z, (v.w * rs) * wv.w);
  }
  store_stream(reinterpret_cast<float4 *>(a.out_norm) + idx, o);
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
  // writers: one float4 per lane (16-byte stores, halfword table loads); the
  // fused kernel stages rows with 16-byte loads
  const bool rows_ok = (ne0 % 4 == 0) && n_ids * (ne0 / 4) < 0xfffff000u && aligned16(table) &&
                       aligned16(out) && (!norm || (aligned16(out_norm) && aligned16(w)));
  const unsigned wgrid = static_cast<unsigned>((n_ids * (ne0 / 4) + 255) / 256);
  GatherArgs ga{};
  ga.table = table;
  ga.ids = ids;
  ga.out = out;
  ga.out_norm = out_norm;
  ga.w = w;
  ga.bad_id = bad_id;
  ga.row_bytes = static_cast<int>(row_bytes);
  ga.ne0 = static_cast<int>(ne0);
  ga.n_ids = static_cast<int>(n_ids);
  ga.n_rows = nr;
  ga.eps = eps;
  if (rows_ok && !norm) {
    const unsigned per = (wgrid + 7) / 8;
    BH_LAUNCH(pq2_rows_write_kernel, 8 * per, 256, 0, st, ga, per);
    return ok();
  }
  const size_t cus = device_cu_count();
  if (rows_ok && norm && row_bytes % 16 == 0 && n_ids >= 16 * cus &&
      scale_smem_bytes(row_bytes) <= kMaxSeqSmem) {
    // Long batches: row scales + embedding rows, then the norm rows (two
    // flat writers).  The scale walk (~20 us of dependent steps) hides under
    // the embedding stores only when there are enough of them: measured at
    // T=8192 55.5-64 us against 69-72 for the one-launch kernel below, at
    // T=2048 32.0 against 30.0 (so shorter batches stay on that kernel).
    float *scales = static_cast<float *>(device_scratch(n_ids * sizeof(float), kScratchGather, st));
    if (scales == nullptr) return BH_ERR_HIP;
    const size_t smem = scale_smem_bytes(row_bytes);
    if (int e = check_hip(hipFuncSetAttribute(reinterpret_cast<const void *>(pq2_scale_embed_kernel),
                                              hipFuncAttributeMaxDynamicSharedMemorySize,
                                              static_cast<int>(smem)),
                          "hipFuncSetAttribute"))
      return e;
    const unsigned scale_blocks = static_cast<unsigned>((n_ids + kScaleRows - 1) / kScaleRows);
    const unsigned s_per = (scale_blocks + 7) / 8;
    const unsigned e_per = (wgrid + 7) / 8;
    BH_LAUNCH(pq2_scale_embed_kernel, 8 * s_per + 8 * e_per, 256, smem, st, ga, scales, 8 * s_per,
              s_per, e_per);
    BH_LAUNCH(pq2_norm_write_kernel, 8 * e_per, 256, 0, st, ga, scales, e_per);
    return ok();
  }
  if (rows_ok && norm && row_bytes % 16 == 0 && fused_smem_bytes(row_bytes, 16, 128) <= kMaxSeqSmem) {
    // 16 rows per block while that still gives every CU a block; fewer rows
    // per block (more blocks) for short batches: the chain's latency is the
    // same for any number of rows, the rest of a block's work is not.
    // Measured (us, T=2048 / 8192, chunks of 32 float4): 16 rows x 1024
    // lanes 39.0 / 70.3, 8 x 1024 34.6 / 81, 8 x 512 37.0 / 70.7, 4 x 512
    // 35.1 / 85, 4 x 256 38.6 / 69.  Longer chunks (fewer barriers on the
    // chain's path): 8 rows, chunks of 64 / 128 float4 33.3 / 32.7 at
    // T=2048; 16 rows, 64: 70.2 at T=8192 (128: 80.5).
    const int rows = n_ids >= 16 * cus ? 16 : (n_ids >= 8 * cus ? 8 : 4);
    auto launch = [&](auto kern, int r, int threads, int chunk_q) -> int {
      const size_t smem = fused_smem_bytes(row_bytes, r, chunk_q);
      if (int e = check_hip(hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                                static_cast<int>(smem)),
                            "hipFuncSetAttribute"))
        return e;
      const unsigned fgrid = static_cast<unsigned>((n_ids + r - 1) / r);
      BH_LAUNCH(kern, fgrid, threads, smem, st, ga);
      return ok();
    };
    if (rows == 16) return launch(pq2_gather_rms_kernel<16, 1024, 64>, 16, 1024, 64);
    if (rows == 8) return launch(pq2_gather_rms_kernel<8, 1024, 128>, 8, 1024, 128);
    return launch(pq2_gather_rms_kernel<4, 512, 128>, 4, 512, 128);
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
