// Gated delta-net recurrence over a batch of tokens.
//
// Reference: gdn_step, src/gdn.rs:17-77 (one token): for every v-head h
// (q/k head h % h_k) with state M = state[h] (s x s, row j contiguous):
//   M *= expf(gate[h]);
//   delta[j] = (v[j] - dot(M[j], k)) * beta[h];
//   M[j] += k * delta[j];
//   attn[j] = dot(M[j], q) * (1 / sqrtf(s)).
// Each row M[j] only ever meets its own delta[j] and the head's vectors, so
// the h_v * s rows are independent recurrences of s floats.  The fast path
// (s = 128) gives a row to 16 lanes, 8 floats each, held in registers for
// the whole token batch: per token the lanes take both row dots from the
// state before the token (a depth-3 tree in the lane, then a DPP tree over
// the 16 lanes; see token_step for the algebra), update the row and store
// one output; batches go two tokens per update (the step loop of
// gdn_step128_kernel); the state is read and written once per call.
// A block's 16 rows share one head, so a block stages the token inputs (q
// and k of the head, v of its rows, gate, beta) 32 tokens at a time in LDS.
// The reference sums the 128 products of a dot in index order; the tree
// order and the regrouping differ by rounding only (outputs and state within
// 1e-5 of the reference's scale).
// Batches of kChunkMin tokens or more take the recurrence's closed form per
// 64-token chunk on f32 matrix cores instead (gdn_chunk_prep_kernel, then
// gdn_chunk_walk_kernel; the algebra is written out above them).
#include <hip/hip_runtime.h>

#include <string>

#include "common.hpp"

namespace bh {
namespace {

constexpr int kBlock = 256;
constexpr int kLanesPerRow = 16;
constexpr int kRowsPerBlock = kBlock / kLanesPerRow;  // 16, never straddling a head
constexpr int kFast = 128;                            // s of the fast path
constexpr int kPerLane = kFast / kLanesPerRow;        // 8 state floats per lane

struct GdnStepArgs {
  const float *q, *k, *v, *gate, *beta;
  float *state, *attn;
  size_t n_tok;
  int h_k, h_v, s;
  float scale;
  int xcd_map;  // 1: place the blocks of one q/k head on one XCD (see row_tile)
};

// The row tile (of `bph` per v-head) a block works on.  Workgroups go to the
// chip's 8 XCDs round robin (block b to XCD b % 8), and every block of the
// v-heads that share a q/k head reads that head's q and k rows; with
// xcd_map the blocks are renumbered so all of them land on one XCD and its
// L2 serves the re-reads (otherwise each XCD would fetch them from HBM):
// XCD x takes the q/k heads x, x + 8, ..., each with its rep * bph blocks.
// Used when h_k % 8 == 0 and h_v % h_k == 0 (the model's 16 / 48 heads);
// it changes which block does what, never the results.
__device__ __forceinline__ int row_tile(const GdnStepArgs &a, int bph) {
  const int p = static_cast<int>(blockIdx.x);
  if (!a.xcd_map) return p;
  const int g = (a.h_v / a.h_k) * bph;  // blocks per q/k head
  const int x = p % 8, sl = p / 8;
  const int kh = (sl / g) * 8 + x;
  const int local = sl % g;
  const int h = kh + (local / bph) * a.h_k;
  return h * bph + local % bph;
}

// Sum over the 16 lanes of a row group (lanes 16r .. 16r+15), every lane
// receiving the same total: DPP swaps within quads (xor 1, xor 2), then
// row_half_mirror (quad pairs) and row_mirror (half rows).  fp addition is
// commutative, so both partners of each swap hold the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float row16_sum(float x) {
  x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp<0x141>(x);  // row_half_mirror
  x += dpp<0x140>(x);  // row_mirror
  return x;
}

// In-lane part of a dot over the lane's 8 elements: two fused multiply-add
// chains (the library builds with contraction off) and their sum.
__device__ __forceinline__ float part8(const float (&m)[kPerLane], const float4 a, const float4 b) {
  const float s0 = fmaf(m[3], a.w, fmaf(m[2], a.z, fmaf(m[1], a.y, m[0] * a.x)));
  const float s1 = fmaf(m[7], b.w, fmaf(m[6], b.z, fmaf(m[5], b.y, m[4] * b.x)));
  return s0 + s1;
}

// One token on the lane's 8 state floats; returns the row's attn value
// (valid in every lane of the group).  With d_k = M.k and d_q = M.q on the
// state before the token, the reference's sequence (decay, delta from the
// decayed row, outer update, readout from the updated row) is
//   delta = (v - eg d_k) beta,  M' = eg M + k delta,
//   M'.q  = eg d_q + delta (k.q),
// so both row dots come from the old state at once and k.q does not depend
// on the state (rounding differs from the reference's order only).
__device__ __forceinline__ float token_step(float (&m)[kPerLane], const float4 k0, const float4 k1,
                                            const float4 q0, const float4 q1, float v, float g,
                                            float beta, float scale) {
  const float eg = expf(g);
  const float kq = row16_sum(part8({k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w}, q0, q1));
  const float dk = row16_sum(part8(m, k0, k1));
  const float dq = row16_sum(part8(m, q0, q1));
  const float delta = fmaf(-eg, dk, v) * beta;
  m[0] = fmaf(k0.x, delta, eg * m[0]); m[1] = fmaf(k0.y, delta, eg * m[1]);
  m[2] = fmaf(k0.z, delta, eg * m[2]); m[3] = fmaf(k0.w, delta, eg * m[3]);
  m[4] = fmaf(k1.x, delta, eg * m[4]); m[5] = fmaf(k1.y, delta, eg * m[5]);
  m[6] = fmaf(k1.z, delta, eg * m[6]); m[7] = fmaf(k1.w, delta, eg * m[7]);
  return fmaf(eg, dq, delta * kq) * scale;
}

__device__ __forceinline__ void load_state(const float *mp, float (&m)[kPerLane]) {
  const float4 x = reinterpret_cast<const float4 *>(mp)[0];
  const float4 y = reinterpret_cast<const float4 *>(mp)[1];
  m[0] = x.x; m[1] = x.y; m[2] = x.z; m[3] = x.w;
  m[4] = y.x; m[5] = y.y; m[6] = y.z; m[7] = y.w;
}

__device__ __forceinline__ void store_state(float *mp, const float (&m)[kPerLane]) {
  float4 *d = reinterpret_cast<float4 *>(mp);
  d[0] = make_float4(m[0], m[1], m[2], m[3]);
  d[1] = make_float4(m[4], m[5], m[6], m[7]);
}

// Few tokens (decode): each lane loads its token inputs straight from
// global memory, the next token's while the current one computes.
__global__ __launch_bounds__(kBlock) void gdn_step128_direct_kernel(GdnStepArgs a) {
  const int row = row_tile(a, kFast / kRowsPerBlock) * kRowsPerBlock +
                  threadIdx.x / kLanesPerRow;  // h * 128 + j
  const int sub = threadIdx.x % kLanesPerRow;
  const int h = row / kFast, j = row % kFast;
  const int kh = h % a.h_k;
  float *mp = a.state + static_cast<size_t>(row) * kFast + kPerLane * sub;
  float m[kPerLane];
  load_state(mp, m);
  float4 k0, k1, q0, q1;
  float v, g, b;
  auto load_tok = [&](size_t t) {
    const float4 *kp = reinterpret_cast<const float4 *>(a.k + (t * a.h_k + kh) * kFast) + 2 * sub;
    const float4 *qp = reinterpret_cast<const float4 *>(a.q + (t * a.h_k + kh) * kFast) + 2 * sub;
    k0 = kp[0]; k1 = kp[1]; q0 = qp[0]; q1 = qp[1];
    v = a.v[(t * a.h_v + h) * kFast + j];
    g = a.gate[t * a.h_v + h];
    b = a.beta[t * a.h_v + h];
  };
  load_tok(0);
  for (size_t t = 0; t < a.n_tok; ++t) {
    const float4 ck0 = k0, ck1 = k1, cq0 = q0, cq1 = q1;
    const float cv = v, cg = g, cb = b;
    if (t + 1 < a.n_tok) load_tok(t + 1);
    const float out = token_step(m, ck0, ck1, cq0, cq1, cv, cg, cb, a.scale);
    if (sub == 0) a.attn[(t * a.h_v + h) * kFast + j] = out;
  }
  store_state(mp, m);
}

// Batches: the token inputs are staged per chunk in LDS (q and k rows of
// the block's k-head, v of its rows, gate and beta of its v-head, plus
// expf(gate) and k.q once per token).  Chunk c + 1 is loaded into
// registers while chunk c runs from LDS, so HBM latency is paid once per
// chunk.  The loads clamp the token index to the batch (a short last chunk
// re-reads its last token; those LDS entries are never used), so they need
// no branches.  A row goes to L lanes of 128 / L floats: L = 16 gives 1536
// waves for the model's 6144 rows (two waves on the busiest SIMDs hide each
// other's latency); L = 8 halves the cross-lane work but leaves one wave
// per SIMD with its dependency chain exposed; L = 32 (3072 waves, a
// permlane swap more per row dot) measured slower at T=256: 82-84 us
// against 73-74.
constexpr int kChunk = 32;
constexpr size_t kDirectMax = 4;  // token counts that skip the LDS staging
constexpr int kStagedLanes = 16;  // measured faster than 8 on MI355X
constexpr int kQkVec = kChunk * 2 * (kFast / 4);  // float4s of q and k per chunk
constexpr int kQkPerThread = kQkVec / kBlock;     // 8
constexpr int kDotLanes = kBlock / kChunk;        // 8 lanes per token for k.q
static_assert(kQkVec % kBlock == 0, "chunk split");
static_assert(kDotLanes == 8, "k.q is an 8-lane DPP tree");

// Sum over the L lanes of a row (lanes L*r .. L*r + L-1), every lane
// receiving the same total.
template <int L>
__device__ __forceinline__ float row_sum(float x) {
  static_assert(L == 8 || L == 16, "row sums over 8 or 16 lanes");
  x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp<0x141>(x);  // row_half_mirror
  if (L == 16) x += dpp<0x140>(x);  // row_mirror
  return x;
}

template <int L>
struct StagedShape {
  static constexpr int kPer = kFast / L;        // state floats per lane
  static constexpr int kVec = kPer / 4;         // float4s per lane
  static constexpr int kRows = kBlock / L;      // rows per block, one head
  static constexpr int kVPerThread = kChunk * kRows / kBlock;
  static_assert((kChunk * kRows) % kBlock == 0 && kFast % kRows == 0, "staged shape");
};

template <int ROWS>
struct ChunkLds {
  float4 qk[kChunk][2][kFast / 4];  // [token][q, k][col4]
  float v[kChunk][ROWS];
  float gb[2][kChunk];  // gate, beta as loaded
  float eg[kChunk];     // expf(gate)
  float kq[kChunk];     // k . q
  float kk[kChunk];     // k_t . k_{t+1} (token pairs)
  float kqn[kChunk];    // k_t . q_{t+1}
};

template <int ROWS, int VPT>
__device__ __forceinline__ void load_chunk(const GdnStepArgs &a, f32x4 (&rqk)[kQkPerThread],
                                           float (&rv)[VPT], float &rgb, size_t t0, int nt, int h,
                                           int kh, int j0) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < kQkPerThread; ++i) {
    const int f = tid + kBlock * i;
    const int tok = min(f / (2 * kFast / 4), nt - 1);
    const int part = (f / (kFast / 4)) & 1, c4 = f % (kFast / 4);
    const float *src = (part ? a.k : a.q) + ((t0 + tok) * a.h_k + kh) * kFast;
    rqk[i] = reinterpret_cast<const f32x4 *>(src)[c4];
  }
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int e = tid + kBlock * i;
    const int tok = min(e / ROWS, nt - 1), rr = e % ROWS;
    rv[i] = a.v[((t0 + tok) * a.h_v + h) * kFast + j0 + rr];
  }
  const int tok = min(tid % kChunk, nt - 1);
  rgb = ((tid / kChunk) & 1 ? a.beta : a.gate)[(t0 + tok) * a.h_v + h];
}

template <int ROWS, int VPT>
__device__ __forceinline__ void store_chunk(ChunkLds<ROWS> &l, const f32x4 (&rqk)[kQkPerThread],
                                            const float (&rv)[VPT], float rgb) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < kQkPerThread; ++i)
    reinterpret_cast<f32x4 *>(&l.qk[0][0][0])[tid + kBlock * i] = rqk[i];
#pragma unroll
  for (int i = 0; i < VPT; ++i) (&l.v[0][0])[tid + kBlock * i] = rv[i];
  if (tid < 2 * kChunk) (&l.gb[0][0])[tid] = rgb;
}

// Per-token constants of a staged chunk: 8 lanes per token sum 16 products
// of k.q each, then an 8-lane DPP tree; lane 0 of the 8 also takes expf.
// For the next token (within the chunk) the same lanes form k_t . k_{t+1}
// and k_t . q_{t+1}, which a pair of tokens needs (see the step loop).
template <int ROWS>
__device__ __forceinline__ void chunk_constants(ChunkLds<ROWS> &l) {
  const int tid = threadIdx.x;
  const int t = tid / kDotLanes, part = tid % kDotLanes;
  const int tn = t + 1 < kChunk ? t + 1 : t;
  const float4 *q = l.qk[t][0] + 4 * part;
  const float4 *k = l.qk[t][1] + 4 * part;
  const float4 *qn = l.qk[tn][0] + 4 * part;
  const float4 *kn = l.qk[tn][1] + 4 * part;
  float s = 0.0f, skk = 0.0f, skq = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 a = q[i], b = k[i], c = kn[i], d = qn[i];
    s += (a.x * b.x + a.y * b.y) + (a.z * b.z + a.w * b.w);
    skk += (b.x * c.x + b.y * c.y) + (b.z * c.z + b.w * c.w);
    skq += (b.x * d.x + b.y * d.y) + (b.z * d.z + b.w * d.w);
  }
  s = row_sum<8>(s);
  skk = row_sum<8>(skk);
  skq = row_sum<8>(skq);
  if (part == 0) {
    l.kq[t] = s;
    l.kk[t] = skk;
    l.kqn[t] = skq;
    l.eg[t] = expf(l.gb[0][t]);
  }
}

// In-lane part of a row dot over the lane's 4 * N floats, as a tree.
template <int N>
__device__ __forceinline__ float part_dot(const float (&m)[4 * N], const f32x4 (&x)[N]) {
  float p[N];
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const f32x4 v = x[i];
    // fused multiply-adds (the library builds with contraction off)
    p[i] = fmaf(m[4 * i + 3], v.w, fmaf(m[4 * i + 2], v.z, fmaf(m[4 * i + 1], v.y, m[4 * i] * v.x)));
  }
#pragma unroll
  for (int w = 1; w < N; w *= 2)
#pragma unroll
    for (int i = 0; i + w < N; i += 2 * w) p[i] += p[i + w];
  return p[0];
}

template <int L>
__global__ __launch_bounds__(kBlock) void gdn_step128_kernel(GdnStepArgs a) {
  using S = StagedShape<L>;
  __shared__ ChunkLds<S::kRows> lds;
  const int row0 = row_tile(a, kFast / S::kRows) * S::kRows;  // h * 128 + j0
  const int rl = threadIdx.x / L;
  const int sub = threadIdx.x % L;
  const int h = row0 / kFast, j0 = row0 % kFast;
  const int kh = h % a.h_k;
  float *mp = a.state + static_cast<size_t>(row0 + rl) * kFast + S::kPer * sub;
  float m[S::kPer];
#pragma unroll
  for (int i = 0; i < S::kVec; ++i) {
    const f32x4 x = reinterpret_cast<const f32x4 *>(mp)[i];
    m[4 * i] = x.x; m[4 * i + 1] = x.y; m[4 * i + 2] = x.z; m[4 * i + 3] = x.w;
  }
  f32x4 rqk[kQkPerThread];
  float rv[S::kVPerThread], rgb;
  const int n_chunks = static_cast<int>((a.n_tok + kChunk - 1) / kChunk);
  const int last_len = static_cast<int>(a.n_tok - static_cast<size_t>(n_chunks - 1) * kChunk);
  load_chunk<S::kRows>(a, rqk, rv, rgb, 0, n_chunks > 1 ? kChunk : last_len, h, kh, j0);
  for (int c = 0; c < n_chunks; ++c) {
    const int nt = c + 1 < n_chunks ? kChunk : last_len;
    __syncthreads();  // the previous chunk's LDS reads are done
    store_chunk(lds, rqk, rv, rgb);
    __syncthreads();
    if (c + 1 < n_chunks)
      load_chunk<S::kRows>(a, rqk, rv, rgb, static_cast<size_t>(c + 1) * kChunk,
                           c + 2 < n_chunks ? kChunk : last_len, h, kh, j0);
    chunk_constants(lds);
    __syncthreads();
    float *attn = a.attn + (static_cast<size_t>(c) * kChunk * a.h_v + h) * kFast + j0 + rl;
    // one token: the algebra of token_step on the lane's floats
    auto step = [&](int t) {
      f32x4 kc[S::kVec], qc[S::kVec];
      const f32x4 *kp = reinterpret_cast<const f32x4 *>(lds.qk[t][1]) + S::kVec * sub;
      const f32x4 *qp = reinterpret_cast<const f32x4 *>(lds.qk[t][0]) + S::kVec * sub;
#pragma unroll
      for (int i = 0; i < S::kVec; ++i) {
        kc[i] = kp[i];
        qc[i] = qp[i];
      }
      const float eg = lds.eg[t], kq = lds.kq[t], beta = lds.gb[1][t], v = lds.v[t][rl];
      const float dk = row_sum<L>(part_dot<S::kVec>(m, kc));
      const float dq = row_sum<L>(part_dot<S::kVec>(m, qc));
      const float delta = fmaf(-eg, dk, v) * beta;
#pragma unroll
      for (int i = 0; i < S::kVec; ++i) {
        m[4 * i] = fmaf(kc[i].x, delta, eg * m[4 * i]);
        m[4 * i + 1] = fmaf(kc[i].y, delta, eg * m[4 * i + 1]);
        m[4 * i + 2] = fmaf(kc[i].z, delta, eg * m[4 * i + 2]);
        m[4 * i + 3] = fmaf(kc[i].w, delta, eg * m[4 * i + 3]);
      }
      const float out = fmaf(eg, dq, delta * kq) * a.scale;
      if (sub == 0) attn[static_cast<size_t>(t) * a.h_v * kFast] = out;
    };
    // two tokens from one state: all four row dots (k and q of both tokens)
    // against the state before the pair, the second token's through
    //   M' . x = eg (M . x) + delta (k . x)   (M' the state after the first)
    // with k . k' and k . q' from the chunk constants, then one update
    //   M'' = (eg eg') M + (eg' delta) k + delta' k'
    // -- the reference's sequence regrouped again (rounding only), half the
    // dependent steps and three operations per state float instead of four
    auto step2 = [&](int t) {
      f32x4 k0[S::kVec], q0[S::kVec], k1[S::kVec], q1[S::kVec];
      const f32x4 *k0p = reinterpret_cast<const f32x4 *>(lds.qk[t][1]) + S::kVec * sub;
      const f32x4 *q0p = reinterpret_cast<const f32x4 *>(lds.qk[t][0]) + S::kVec * sub;
      const f32x4 *k1p = reinterpret_cast<const f32x4 *>(lds.qk[t + 1][1]) + S::kVec * sub;
      const f32x4 *q1p = reinterpret_cast<const f32x4 *>(lds.qk[t + 1][0]) + S::kVec * sub;
#pragma unroll
      for (int i = 0; i < S::kVec; ++i) {
        k0[i] = k0p[i];
        q0[i] = q0p[i];
        k1[i] = k1p[i];
        q1[i] = q1p[i];
      }
      const float eg0 = lds.eg[t], eg1 = lds.eg[t + 1];
      const float b0 = lds.gb[1][t], b1 = lds.gb[1][t + 1];
      const float v0 = lds.v[t][rl], v1 = lds.v[t + 1][rl];
      const float kq0 = lds.kq[t], kq1 = lds.kq[t + 1], kk = lds.kk[t], kqn = lds.kqn[t];
      const float a0 = row_sum<L>(part_dot<S::kVec>(m, k0));
      const float c0 = row_sum<L>(part_dot<S::kVec>(m, q0));
      const float a1 = row_sum<L>(part_dot<S::kVec>(m, k1));
      const float c1 = row_sum<L>(part_dot<S::kVec>(m, q1));
      const float delta0 = fmaf(-eg0, a0, v0) * b0;
      const float out0 = fmaf(eg0, c0, delta0 * kq0) * a.scale;
      const float mk1 = fmaf(eg0, a1, delta0 * kk);   // M' . k'
      const float mq1 = fmaf(eg0, c1, delta0 * kqn);  // M' . q'
      const float delta1 = fmaf(-eg1, mk1, v1) * b1;
      const float out1 = fmaf(eg1, mq1, delta1 * kq1) * a.scale;
      const float e01 = eg0 * eg1, d0 = eg1 * delta0;
#pragma unroll
      for (int i = 0; i < S::kVec; ++i) {
        m[4 * i] = fmaf(k1[i].x, delta1, fmaf(k0[i].x, d0, e01 * m[4 * i]));
        m[4 * i + 1] = fmaf(k1[i].y, delta1, fmaf(k0[i].y, d0, e01 * m[4 * i + 1]));
        m[4 * i + 2] = fmaf(k1[i].z, delta1, fmaf(k0[i].z, d0, e01 * m[4 * i + 2]));
        m[4 * i + 3] = fmaf(k1[i].w, delta1, fmaf(k0[i].w, d0, e01 * m[4 * i + 3]));
      }
      if (sub == 0) {
        attn[static_cast<size_t>(t) * a.h_v * kFast] = out0;
        attn[static_cast<size_t>(t + 1) * a.h_v * kFast] = out1;
      }
    };
    int t = 0;
    for (; t + 1 < nt; t += 2) step2(t);
    if (t < nt) step(t);
  }
#pragma unroll
  for (int i = 0; i < S::kVec; ++i)
    reinterpret_cast<f32x4 *>(mp)[i] = f32x4{m[4 * i], m[4 * i + 1], m[4 * i + 2], m[4 * i + 3]};
}

// Any s: one lane per row, the row updated in place in memory, sums in
// index order as the reference.
__global__ __launch_bounds__(kBlock) void gdn_step_generic_kernel(GdnStepArgs a) {
  const int row = blockIdx.x * kBlock + threadIdx.x;
  if (row >= a.h_v * a.s) return;
  const int h = row / a.s, j = row % a.s;
  const int kh = h % a.h_k;
  float *mr = a.state + static_cast<size_t>(row) * a.s;
  for (size_t t = 0; t < a.n_tok; ++t) {
    const float *kv = a.k + (t * a.h_k + kh) * a.s;
    const float *qv = a.q + (t * a.h_k + kh) * a.s;
    const float eg = expf(a.gate[t * a.h_v + h]);
    float sum = 0.0f;
    for (int i = 0; i < a.s; ++i) {
      mr[i] *= eg;
      sum += mr[i] * kv[i];
    }
    const float delta = (a.v[(t * a.h_v + h) * a.s + j] - sum) * a.beta[t * a.h_v + h];
    float so = 0.0f;
    for (int i = 0; i < a.s; ++i) {
      mr[i] += kv[i] * delta;
      so += mr[i] * qv[i];
    }
    a.attn[(t * a.h_v + h) * a.s + j] = so * a.scale;
  }
}

// ---- chunked path (matrix cores) -----------------------------------------
//
// Long batches (prefill) take the recurrence 64 tokens at a time in its
// closed form per chunk.  For one v-head, a row m of the state (m_0 at the
// chunk start), the chunk's tokens t = 0..63 with decays a_t = expf(gate_t),
// A_t = a_0 ... a_t and D_ts = A_t / A_s (s <= t), unrolling the per-token
// steps gives
//   x_t     = a_t m_(t-1).k_t = A_t (m_0.k_t) + sum_(s<t) D_ts (k_s.k_t) delta_s
//   delta_t = beta_t (v_t - x_t)
// so the chunk's deltas solve the unit lower triangular system
//   (I + L) delta = beta (v - A (K m_0)),   L_ts = beta_t D_ts (k_t.k_s), s < t,
// whose matrix depends on the head's gates, betas and keys only -- not on
// the state, so it is inverted once per (chunk, v-head) for all 128 rows.
// With T' = (I + L)^-1 diag(beta) and P_ts = D_ts (q_t.k_s) (s <= t):
//   delta = T' (v - A (K m_0))
//   attn  = (A (Q m_0) + P delta) / sqrt(s)
//   m_64  = A_63 m_0 + sum_s (A_63 / A_s) delta_s k_s.
// The same algebra the per-token steps perform, rounded differently (the
// products summed in other orders); measured within ~2e-6 of the per-token
// f32 recurrence (relative to the tensor's largest magnitude) on keys from
// independent to nearly identical, betas up to 1 and decays from none to
// underflow.
//
// gdn_chunk_prep_kernel (all chunks in parallel; a workgroup per (chunk,
// q/k head), or per (chunk, v-head) for short batches) forms K K^T and
// Q K^T on v_mfma_f32_16x16x4_f32, then for each v-head, its four waves
// sharing the work: the decays (prefix sums of the gates in f64, so a large
// early gate costs no precision in later differences), P and L, the inverse
// (16 x 16 diagonal blocks by forward substitution, a lane per column; the
// other blocks by f32 MFMA products) and T', stored in the order the walk's
// MFMA A operands read them.  gdn_chunk_walk_kernel
// (one workgroup per (v-head, 16 state rows)) keeps its rows' state in
// registers as MFMA operands and walks the chunks in order: K m_0 and Q m_0
// (wave w: tokens 16w..16w+15), delta through T' (LDS exchange of the
// right-hand sides), the outputs through P, and the new state (wave w: 32
// of the 128 columns), all on f32 MFMA.
constexpr int kCk = 64;                         // tokens per chunk
constexpr int kCkFrag = kCk * kCk;              // floats of a 64 x 64 matrix
constexpr int kCkPer = 2 * kCkFrag + 2 * kCk;   // per (chunk, v-head): T', P, A, e
constexpr int kCkPitch = 132;                   // prep: staged K / Q rows (floats)
constexpr int kCkBuf = 65;                      // prep: pitch of the 64 x 64 matrices in LDS
constexpr int kCkKPitch = 144;                  // walk: staged K rows
constexpr int kCkMPitch = 132;                  // walk: staged state rows
// batches from which the chunked path runs: measured equal to the per-token
// kernel at 128 tokens (38 us), faster above (256: 55 against 71 us; 512:
// 100 against 139)
constexpr size_t kChunkMin = 128;
constexpr float kGateFloor = -200.0f;           // expf below this is 0 in f32
static_assert(3 * kCk * kCkBuf <= 2 * kCk * kCkPitch, "K K^T, Q K^T and L fit the staging area");

typedef float f32x4m __attribute__((ext_vector_type(4)));

struct GdnChunkArgs {
  const float *q, *k, *v, *gate, *beta;
  float *state, *attn;
  float *scr;  // [n_chunks][h_v][kCkPer]
  size_t n_tok;
  int h_k, h_v, n_chunks;
  float scale;
  int xcd_map;
  int prep_per;  // prep workgroups per (chunk, q/k head): 1, or one per v-head
};

__device__ __forceinline__ f32x4m mfma_f32(float a, float b, f32x4m c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// T' and P are stored in MFMA A-fragment order: element (r, c) of row tile
// wt = r / 16 belongs to lane l = r % 16 + 16 (c % 4) at step ks = c / 4 and
// sits at ((wt * 64 + l) * 16 + ks), so each lane of the walk reads its 16
// values of a tile as four 16-byte loads.

// Block (bi, bj), bi >= bj, of the inverse in the 64 x 64 buffer of L:
// diagonal blocks in place, T_ij (i > j) in the upper block (j, i), which L
// leaves free.
__device__ __forceinline__ float *tblock(float *buf, int bi, int bj) {
  return bi == bj ? buf + 16 * bi * (kCkBuf + 1) : buf + 16 * bj * kCkBuf + 16 * bi;
}

// Tiles k = w + 4 u (u < N) of the lower triangle of K K^T and Q K^T (tile
// k: row tile ti, column tile nt <= ti), accumulated over the 128 dims and
// written to LDS at pitch kCkBuf once every wave has read the staged rows
// (one block barrier: every wave runs exactly one instantiation, so each
// arrives at it once).  N is a template parameter so the accumulators stay
// in registers across the loop (no per-step branches).
template <int N>
__device__ __forceinline__ void prep_qk_tiles(const float *sK, const float *sQ, float *sKK,
                                              float *sQK, int w, int lr, int lg) {
  f32x4m accK[N], accQ[N];
  int ra[N], rb[N], ti[N], nt[N];
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const int k = w + 4 * u;
    ti[u] = k < 1 ? 0 : (k < 3 ? 1 : (k < 6 ? 2 : 3));
    nt[u] = k - ti[u] * (ti[u] + 1) / 2;
    ra[u] = (16 * ti[u] + lr) * kCkPitch + lg;
    rb[u] = (16 * nt[u] + lr) * kCkPitch + lg;
    accK[u] = accQ[u] = f32x4m{0.0f, 0.0f, 0.0f, 0.0f};
  }
#pragma unroll 8
  for (int ks = 0; ks < kFast / 4; ++ks) {
#pragma unroll
    for (int u = 0; u < N; ++u) {
      const float b = sK[rb[u] + 4 * ks];
      accK[u] = mfma_f32(sK[ra[u] + 4 * ks], b, accK[u]);
      accQ[u] = mfma_f32(sQ[ra[u] + 4 * ks], b, accQ[u]);
    }
  }
  __syncthreads();  // sKK and sQK overlay the staged K and Q
#pragma unroll
  for (int u = 0; u < N; ++u)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      sKK[(16 * ti[u] + 4 * lg + rr) * kCkBuf + 16 * nt[u] + lr] = accK[u][rr];
      sQK[(16 * ti[u] + 4 * lg + rr) * kCkBuf + 16 * nt[u] + lr] = accQ[u][rr];
    }
}

// Workgroup (chunk c, q/k head kh, part): with `per` = 1 it prepares every
// v-head of kh (K K^T and Q K^T formed once for all of them); with per > 1
// (short batches, to fill the chip) part n prepares v-head kh + n h_k only.
// The four waves share each v-head: wave w forms rows 16 w .. 16 w + 15 of P
// and L (lane (lr, lg): row 16 w + lr, columns 16 lg .. 16 lg + 15),
// inverts diagonal block w, takes pair w of each distance of the
// off-diagonal blocks and stores row tile w of T'.  Its LDS (K, Q, K K^T,
// Q K^T, L, all in the 67 KB that first holds the staged K and Q) lets two
// workgroups share a CU.
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(2, 2))) void
gdn_chunk_prep_kernel(GdnChunkArgs a) {
  // K, Q (pitch kCkPitch); then K K^T, Q K^T and L / the inverse (pitch 65:
  // lane t reading row t hits bank t + s)
  __shared__ __attribute__((aligned(16))) float sStage[2 * kCk * kCkPitch];
  __shared__ double sG[kCk];
  __shared__ float sB[kCk];
  __shared__ float sS[4][16 * 17];  // per-wave block products in transit
  const int per = a.prep_per;
  const int bid = static_cast<int>(blockIdx.x);
  const int c = bid / (a.h_k * per), kh = (bid / per) % a.h_k, part = bid % per;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (scalar branches)
  const int l = threadIdx.x & 63, lr = l & 15, lg = l >> 4;
  const size_t t0 = static_cast<size_t>(c) * kCk;
  float *sK = sStage, *sQ = sStage + kCk * kCkPitch;
  float *sKK = sStage, *sQK = sStage + kCk * kCkBuf;
  // stage the chunk's k and q rows of this head (zeros past the batch)
#pragma unroll
  for (int i = 0; i < kCk * 32 / kBlock; ++i) {
    const int e = i * kBlock + threadIdx.x, t = e >> 5, c4 = e & 31;
    f32x4m kv = {0.0f, 0.0f, 0.0f, 0.0f}, qv = kv;
    if (t0 + t < a.n_tok) {
      const size_t off = ((t0 + t) * a.h_k + kh) * kFast + 4 * c4;
      kv = *reinterpret_cast<const f32x4m *>(a.k + off);
      qv = *reinterpret_cast<const f32x4m *>(a.q + off);
    }
    *reinterpret_cast<f32x4m *>(sK + t * kCkPitch + 4 * c4) = kv;
    *reinterpret_cast<f32x4m *>(sQ + t * kCkPitch + 4 * c4) = qv;
  }
  __syncthreads();
  // K K^T and Q K^T on the 10 tiles with s <= t: tiles k = w, w + 4, w + 8
  // (of those below 10) to wave w
  if (w < 2)
    prep_qk_tiles<3>(sK, sQ, sKK, sQK, w, lr, lg);
  else
    prep_qk_tiles<2>(sK, sQ, sKK, sQK, w, lr, lg);
  __syncthreads();
  float *buf = sStage + 2 * kCk * kCkBuf;  // 64 x 64 at pitch kCkBuf: L, then the inverse
  const int n_vh = (a.h_v - kh + a.h_k - 1) / a.h_k;  // v-heads h = kh + n h_k
  const int t = 16 * w + lr;                            // this lane's row of P and L
  for (int n = part; n < n_vh; n += per) {              // the same count in every wave
    const int hv = kh + n * a.h_k;
    float *out = a.scr + (static_cast<size_t>(c) * a.h_v + hv) * kCkPer;
    if (w == 0) {
      // decays: A_t = expf(G_t), e_t = expf(G_63 - G_t), G the prefix sums
      // of the gates (f64) -- lane l = token l
      float g = 0.0f, b = 0.0f;
      if (t0 + l < a.n_tok) {
        g = a.gate[(t0 + l) * a.h_v + hv];
        b = a.beta[(t0 + l) * a.h_v + hv];
      }
      g = g < kGateFloor ? kGateFloor : g;  // -inf too (NaN stays NaN)
      double G = static_cast<double>(g);
#pragma unroll
      for (int d = 1; d < kCk; d <<= 1) {
        const double o = __shfl_up(G, d, kCk);
        if (l >= d) G += o;
      }
      const double Glast = __shfl(G, kCk - 1, kCk);
      sG[l] = G;
      sB[l] = b;
      out[2 * kCkFrag + l] = expf(static_cast<float>(G));
      out[2 * kCkFrag + kCk + l] = expf(static_cast<float>(Glast - G));
    }
    __syncthreads();
    // P and L on this lane's 16 entries (D_ts = expf(G_t - G_s), s <= t);
    // P goes out in A-fragment order: entries 16 lg + m + 4 j (j = 0..3) are
    // the consecutive steps 4 lg + j of lane t % 16 + 16 m
    {
      const double Gt = sG[t];
      const float bt = sB[t];
      float pv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int s = 16 * lg + i;
        const float arg = static_cast<float>(Gt - sG[s]);
        const float d = s <= t ? exp_hw(arg < 0.0f ? arg : 0.0f) : 0.0f;
        pv[i] = s <= t ? d * sQK[t * kCkBuf + s] : 0.0f;
        buf[t * kCkBuf + s] = s < t ? bt * d * sKK[t * kCkBuf + s] : 0.0f;
      }
#pragma unroll
      for (int m = 0; m < 4; ++m)
        *reinterpret_cast<f32x4m *>(out + kCkFrag + (w * 64 + lr + 16 * m) * 16 + 4 * lg) =
            f32x4m{pv[m], pv[m + 4], pv[m + 8], pv[m + 12]};
    }
    __syncthreads();
    // (I + L)^-1 blockwise (16 x 16 blocks).  Diagonal block w: lane lr of
    // lane group 0 takes column lr by forward substitution (when row r is
    // final its multiple goes into every later row), then overwrites L_ww.
    float x[16];
    float *dg = buf + 16 * w * (kCkBuf + 1);
    if (lg == 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] = r == lr ? 1.0f : 0.0f;
#pragma unroll
      for (int r = 0; r < 15; ++r)
#pragma unroll
        for (int r2 = r + 1; r2 < 16; ++r2) x[r2] = fmaf(-dg[r2 * kCkBuf + r], x[r], x[r2]);
    }
    __syncthreads();
    if (lg == 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) dg[r * kCkBuf + lr] = x[r];
    }
    __syncthreads();
    // Off-diagonal blocks, one distance at a time, pair (w + dist, w) on
    // wave w:  T_ij = -T_ii (sum_(j <= m < i) L_im T_mj)  (f32 MFMA); T_ij
    // (i > j) is kept in the upper block (j, i), which L leaves free.
    for (int dist = 1; dist < 4; ++dist) {
      const int bi = w + dist, bj = w;
      if (bi < 4) {
        f32x4m S = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int m = bj; m < bi; ++m) {
          const float *la = buf + (16 * bi + lr) * kCkBuf + 16 * m + lg;  // L_(bi, m), A operand
          const float *tt = tblock(buf, m, bj) + lg * kCkBuf + lr;       // T_(m, bj), B operand
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) S = mfma_f32(la[4 * ks], tt[4 * ks * kCkBuf], S);
        }
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) sS[w][(4 * lg + rr) * 17 + lr] = S[rr];
      }
      __syncthreads();
      if (bi < 4) {
        f32x4m tij = {0.0f, 0.0f, 0.0f, 0.0f};
        const float *ta = tblock(buf, bi, bi) + lr * kCkBuf + lg;  // T_ii, A operand
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) tij = mfma_f32(ta[4 * ks], sS[w][(4 * ks + lg) * 17 + lr], tij);
        float *dst = tblock(buf, bi, bj);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) dst[(4 * lg + rr) * kCkBuf + lr] = -tij[rr];
      }
      __syncthreads();
    }
    // T' = (I + L)^-1 diag(beta), row tile w in A-fragment order: lane l =
    // r % 16 + 16 (c % 4) holds steps ks = c / 4 of row r = 16 w + l % 16
    {
      f32x4m *d = reinterpret_cast<f32x4m *>(out + (w * 64 + l) * 16);
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        f32x4m v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int col = 4 * (4 * i4 + e) + lg;
          v[e] = (col >> 4) <= w ? tblock(buf, w, col >> 4)[lr * kCkBuf + (col & 15)] * sB[col]
                                 : 0.0f;
        }
        d[i4] = v;
      }
    }
    __syncthreads();
  }
}

// Workgroup p -> (v-head, 16-row slab).  With xcd_map the 8 slabs of every
// v-head of one q/k head land on one XCD (workgroup p runs on XCD p % 8), so
// that XCD's L2 serves their re-reads of the head's k and q rows and of the
// prepared matrices.  Only placement changes, never results.
__device__ __forceinline__ int walk_tile(const GdnChunkArgs &a) {
  const int p = static_cast<int>(blockIdx.x);
  constexpr int bph = kFast / 16;
  if (!a.xcd_map) return p;
  const int g = (a.h_v / a.h_k) * bph;
  const int x = p % 8, sl = p / 8;
  const int kh = (sl / g) * 8 + x;
  const int local = sl % g;
  return (kh + (local / bph) * a.h_k) * bph + local % bph;
}

// The token rows of chunk c (k and q at A-operand row 16 w + lr, v at the
// D rows 16 w + 4 lg + rr of state row j); zeros past the batch.
__device__ __forceinline__ void walk_load_tokens(const GdnChunkArgs &a, int c, int h, int kh, int j,
                                                 int w, int lr, int lg, f32x4m (&kr)[8],
                                                 f32x4m (&qr)[8], float (&vr)[4]) {
  const size_t t0 = static_cast<size_t>(c) * kCk;
  const size_t tok = t0 + 16 * w + lr;
  if (tok < a.n_tok) {
    const size_t off = (tok * a.h_k + kh) * kFast + 4 * lg;
#pragma unroll
    for (int ib = 0; ib < 8; ++ib) {
      kr[ib] = *reinterpret_cast<const f32x4m *>(a.k + off + 16 * ib);
      qr[ib] = *reinterpret_cast<const f32x4m *>(a.q + off + 16 * ib);
    }
  } else {
#pragma unroll
    for (int ib = 0; ib < 8; ++ib) kr[ib] = qr[ib] = f32x4m{0.0f, 0.0f, 0.0f, 0.0f};
  }
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const size_t tt = t0 + 16 * w + 4 * lg + rr;
    vr[rr] = tt < a.n_tok ? a.v[(tt * a.h_v + h) * kFast + j] : 0.0f;
  }
}

// The chunk's rows are loaded while the previous chunk runs (issued after
// its K m_0 / Q m_0 products, when those registers are free), and the
// prepared matrices at the top of the chunk, ahead of the products that
// precede their use: each chunk then waits on at most one memory round trip.
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(2, 2))) void
gdn_chunk_walk_kernel(GdnChunkArgs a) {
  __shared__ __attribute__((aligned(16))) float sK[kCk * kCkKPitch];
  __shared__ __attribute__((aligned(16))) float sR[kCk * 16];
  __shared__ __attribute__((aligned(16))) float sD[kCk * 16];
  __shared__ __attribute__((aligned(16))) float sM[16 * kCkMPitch];
  __shared__ float sE[kCk];
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (scalar branches)
  const int l = threadIdx.x & 63, lr = l & 15, lg = l >> 4;
  const int tile = walk_tile(a);
  const int h = tile / (kFast / 16), kh = h % a.h_k;
  const int j = (tile % (kFast / 16)) * 16 + lr;  // the state row of this lane's columns
  float *mrow = a.state + (static_cast<size_t>(h) * kFast + j) * kFast;
  // M[ib][r] = m_0[j][16 ib + 4 lg + r]: the B operand of step (ib, r) of
  // K m_0^T and the D fragment of column tile ib of the new state
  f32x4m M[8];
#pragma unroll
  for (int ib = 0; ib < 8; ++ib) M[ib] = *reinterpret_cast<const f32x4m *>(mrow + 16 * ib + 4 * lg);
  f32x4m kr[8], qr[8];
  float vr[4];
  walk_load_tokens(a, 0, h, kh, j, w, lr, lg, kr, qr, vr);
  for (int c = 0; c < a.n_chunks; ++c) {
    const size_t t0 = static_cast<size_t>(c) * kCk;
    const float *scr = a.scr + (static_cast<size_t>(c) * a.h_v + h) * kCkPer;
    const f32x4m *tf = reinterpret_cast<const f32x4m *>(scr + (w * 64 + l) * 16);
    const f32x4m *pf = reinterpret_cast<const f32x4m *>(scr + kCkFrag + (w * 64 + l) * 16);
    f32x4m tfr[4], pfr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      tfr[i] = tf[i];
      pfr[i] = pf[i];
    }
    const f32x4m At = *reinterpret_cast<const f32x4m *>(scr + 2 * kCkFrag + 16 * w + 4 * lg);
    const float alast = scr[2 * kCkFrag + kCk - 1];
    if (w == 0) sE[l] = scr[2 * kCkFrag + kCk + l];
#pragma unroll
    for (int ib = 0; ib < 8; ++ib)
      *reinterpret_cast<f32x4m *>(sK + (16 * w + lr) * kCkKPitch + 16 * ib + 4 * lg) = kr[ib];
    // K m_0^T and Q m_0^T, two accumulators each (independent MFMA chains)
    f32x4m X0 = {0.0f, 0.0f, 0.0f, 0.0f}, X1 = X0, Y0 = X0, Y1 = X0;
#pragma unroll
    for (int ib = 0; ib < 8; ib += 2)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        X0 = mfma_f32(kr[ib][r], M[ib][r], X0);
        Y0 = mfma_f32(qr[ib][r], M[ib][r], Y0);
        X1 = mfma_f32(kr[ib + 1][r], M[ib + 1][r], X1);
        Y1 = mfma_f32(qr[ib + 1][r], M[ib + 1][r], Y1);
      }
    const f32x4m X = X0 + X1, Y = Y0 + Y1;
    // right-hand sides v - A (K m_0): tokens 16 w + 4 lg + rr, row j
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) sR[(16 * w + 4 * lg + rr) * 16 + lr] = vr[rr] - At[rr] * X[rr];
    if (c + 1 < a.n_chunks) walk_load_tokens(a, c + 1, h, kh, j, w, lr, lg, kr, qr, vr);
    __syncthreads();
    // delta rows of tile w = T' (lower triangular: steps below 4 (w + 1))
    f32x4m D = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < 16; ++ks)
      if (ks < 4 * (w + 1)) D = mfma_f32(tfr[ks >> 2][ks & 3], sR[(4 * ks + lg) * 16 + lr], D);
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) sD[(16 * w + 4 * lg + rr) * 16 + lr] = D[rr];
    __syncthreads();
    // outputs A (Q m_0) + P delta
    f32x4m O = At * Y;
#pragma unroll
    for (int ks = 0; ks < 16; ++ks)
      if (ks < 4 * (w + 1)) O = mfma_f32(pfr[ks >> 2][ks & 3], sD[(4 * ks + lg) * 16 + lr], O);
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const size_t tt = t0 + 16 * w + 4 * lg + rr;
      if (tt < a.n_tok) a.attn[(tt * a.h_v + h) * kFast + j] = O[rr] * a.scale;
    }
    // new state, column tiles 2w and 2w + 1: A_63 m_0 + (e K)^T delta
#pragma unroll
    for (int ib = 0; ib < 8; ++ib) {
      if ((ib >> 1) == w) {
        f32x4m acc = alast * M[ib];
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) {
          const int s = 4 * ks + lg;
          acc = mfma_f32(sE[s] * sK[s * kCkKPitch + 16 * ib + lr], sD[s * 16 + lr], acc);
        }
        *reinterpret_cast<f32x4m *>(sM + lr * kCkMPitch + 16 * ib + 4 * lg) = acc;
      }
    }
    __syncthreads();
#pragma unroll
    for (int ib = 0; ib < 8; ++ib)
      M[ib] = *reinterpret_cast<const f32x4m *>(sM + lr * kCkMPitch + 16 * ib + 4 * lg);
  }
#pragma unroll
  for (int ib = 0; ib < 8; ++ib)
    if ((ib >> 1) == w) *reinterpret_cast<f32x4m *>(mrow + 16 * ib + 4 * lg) = M[ib];
}

}  // namespace
}  // namespace bh

using namespace bh;

extern "C" int bh_gdn_step(const float *q, const float *k, const float *v, const float *gate,
                           const float *beta, float *state, float *attn, size_t n_tok,
                           size_t h_k, size_t h_v, size_t s, bh_stream stream) {
  if (h_k == 0 || h_v == 0 || s == 0)
    return fail(BH_ERR_SHAPE, "gdn_step: h_k, h_v and s must be positive");
  if (h_v * s > 0x7fffffffu || h_k * s > 0x7fffffffu)
    return fail(BH_ERR_SHAPE, "gdn_step: state too large");
  if (n_tok == 0) return ok();
  if (!q || !k || !v || !gate || !beta || !state || !attn)
    return fail(BH_ERR_ARG, "gdn_step: null pointer");
  GdnStepArgs a{q, k, v, gate, beta, state, attn, n_tok, static_cast<int>(h_k),
                static_cast<int>(h_v), static_cast<int>(s),
                1.0f / sqrtf(static_cast<float>(s)),  // src/gdn.rs:31, f32 on the host
                (h_k % 8 == 0 && h_v % h_k == 0) ? 1 : 0};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool fast =
      s == static_cast<size_t>(kFast) && aligned16(q) && aligned16(k) && aligned16(state);
  if (fast && n_tok >= kChunkMin && aligned16(v) && aligned16(attn)) {
    const size_t n_chunks = (n_tok + kCk - 1) / kCk;
    size_t bytes = 0;
    if (n_chunks > 0x7fffffffu || !mul_size(n_chunks, h_v, kCkPer * sizeof(float), &bytes))
      return fail(BH_ERR_SHAPE, "gdn_step: batch too long");
    float *scr = static_cast<float *>(device_scratch(bytes, kScratchGdn, st));
    if (scr == nullptr) return BH_ERR_HIP;
    // one prep workgroup per (chunk, v-head) while (chunk, q/k head) would
    // leave most CUs idle; each fills a CU (its LDS)
    const size_t rep = (h_v + h_k - 1) / h_k;
    const int per = n_chunks * h_k >= 2 * device_cu_count() ? 1 : static_cast<int>(rep);
    GdnChunkArgs ca{q, k, v, gate, beta, state, attn, scr, n_tok, static_cast<int>(h_k),
                    static_cast<int>(h_v), static_cast<int>(n_chunks), a.scale, a.xcd_map, per};
    BH_LAUNCH(gdn_chunk_prep_kernel, static_cast<unsigned>(n_chunks * h_k * per), kBlock, 0, st,
              ca);
    BH_LAUNCH(gdn_chunk_walk_kernel, static_cast<unsigned>(h_v * (kFast / 16)), kBlock, 0, st, ca);
  } else if (fast) {
    const unsigned grid = static_cast<unsigned>(h_v * s / kRowsPerBlock);
    if (n_tok <= kDirectMax)
      BH_LAUNCH(gdn_step128_direct_kernel, grid, kBlock, 0, st, a);
    else
      BH_LAUNCH(gdn_step128_kernel<kStagedLanes>,
                static_cast<unsigned>(h_v * s / StagedShape<kStagedLanes>::kRows), kBlock, 0, st, a);
  } else {
    const unsigned grid = static_cast<unsigned>((h_v * s + kBlock - 1) / kBlock);
    BH_LAUNCH(gdn_step_generic_kernel, grid, kBlock, 0, st, a);
  }
  return ok();
}
