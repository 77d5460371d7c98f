// Shared host and device helpers of the bonsai HIP library (gfx950 only).
//
// Host side: status/last-error plumbing and launch checking.
// Device side: wave64 / workgroup reductions for "row groups" of G lanes and
// the scalar functions of the reference (src/kernels.rs:148-164,
// src/gguf.rs:881-911) written so that the GPU result matches the x86 build
// of the reference.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/bonsai_hip.h"

namespace bh {

// ---------------------------------------------------------------------------
// Host: status plumbing
// ---------------------------------------------------------------------------

// Records `msg` as this thread's last error and returns `code`.
int fail(int code, const std::string &msg);
// Clears the last error and returns BH_OK.
int ok();
// Converts the result of a launch (hipGetLastError) into a status.
int check_launch(const char *what);
// Converts an arbitrary HIP call result into a status.
int check_hip(hipError_t e, const char *what);

inline hipStream_t as_stream(bh_stream s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// Smallest power of two >= v (v >= 1).
inline int pow2ceil(size_t v) {
  int p = 1;
  while (static_cast<size_t>(p) < v) p <<= 1;
  return p;
}

// Per-device scratch owned by the library, one buffer per client so
// different entry points never share one.  Calls of the same client on one
// device must not overlap in time.  A buffer grows on demand (at least
// twofold) and the buffer it replaces is kept until the process ends, so a
// graph captured earlier keeps valid addresses.  Growth while `stream` is
// capturing is refused (it would allocate inside the capture).  Returns
// nullptr with the status recorded on failure.
constexpr int kScratchSoftmax = 0;  // split-row softmax partials
constexpr int kScratchMatmul = 1;   // PQ2_0 product: f16 x fragments, token scales
constexpr int kScratchAttention = 2;  // attention: chunk partials or probabilities
constexpr int kScratchGather = 3;     // gather + RMSNorm: the row scales
constexpr int kScratchGdn = 4;        // gated delta-net chunks: prepared matrices
constexpr int kScratchKvSplit = 5;    // attention: f32 cache split into f16 hi / lo
constexpr int kScratchSlots = 6;
void *device_scratch(size_t bytes, int slot, hipStream_t stream);
// Current size of this device's buffer for `slot` (0 before the first use).
size_t scratch_bytes(int slot);
// Compute units of the current device (queried once per device; 256 if the
// query fails).
size_t device_cu_count();

// a * b (* c), or false when the product does not fit in size_t.
inline bool mul_size(size_t a, size_t b, size_t *out) { return !__builtin_mul_overflow(a, b, out); }
inline bool mul_size(size_t a, size_t b, size_t c, size_t *out) {
  size_t t;
  return mul_size(a, b, &t) && mul_size(t, c, out);
}


// ---------------------------------------------------------------------------
// Device: reductions
// ---------------------------------------------------------------------------

struct SumOp {
  template <class T> __device__ T operator()(T a, T b) const { return a + b; }
};
// max that ignores NaN in the candidate, like the reference's `if v > max`.
// RMSNorm row scale 1 / sqrt(ss / n + eps) (src/kernels.rs:69-70) with the
// mean as a multiply by the f32 reciprocal of n (exact for powers of two,
// <= 1 ulp otherwise) and the hardware reciprocal square root (<= 1 ulp):
// a few ulps from the correctly rounded divide and square root, far inside
// the 1e-5 bar, and about twenty instructions shorter on the path between a
// row's loads and its stores (measured: 21.9 -> 20.9 us on config 2's
// attention pre-block).
__device__ __forceinline__ float rms_scale(float ss, float inv_n, float eps) {
  return __builtin_amdgcn_rsqf(ss * inv_n + eps);
}

struct MaxOp {
  __device__ float operator()(float a, float b) const { return b > a ? b : a; }
};

// Reduction over aligned groups of G consecutive lanes (G a power of two
// <= 64) without LDS: DPP quad swaps, half-row and row mirrors inside each
// 16-lane row, then the gfx950 row-pair and half-wave swaps
// (v_permlane16_swap, v_permlane32_swap).  32-bit values move as they are,
// 64-bit values as two halves.  The swap steps compute op(lower, upper) on
// both sides of the pair; the DPP steps compute op(own, partner), which is
// the same bits on both sides for commutative ops (sums; max over non-NaN
// partials).  All lanes of the wave must be active.
template <int CTRL, class T>
__device__ __forceinline__ T dpp_move(T x) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit lanes");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                             0xF, 0xF, false));
  } else {
    const int2 h = __builtin_bit_cast(int2, x);
    int2 r;
    r.x = __builtin_amdgcn_update_dpp(0, h.x, CTRL, 0xF, 0xF, false);
    r.y = __builtin_amdgcn_update_dpp(0, h.y, CTRL, 0xF, 0xF, false);
    return __builtin_bit_cast(T, r);
  }
}
// Returns {value of the lower half of the pair, value of the upper half}.
template <int SPAN, class T>
__device__ __forceinline__ void lane_swap(T x, T &lo, T &hi) {
  if constexpr (sizeof(T) == 4) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto r = SPAN == 16 ? __builtin_amdgcn_permlane16_swap(u, u, false, false)
                              : __builtin_amdgcn_permlane32_swap(u, u, false, false);
    lo = __builtin_bit_cast(T, static_cast<unsigned>(r[0]));
    hi = __builtin_bit_cast(T, static_cast<unsigned>(r[1]));
  } else {
    const uint2 h = __builtin_bit_cast(uint2, x);
    const auto a = SPAN == 16 ? __builtin_amdgcn_permlane16_swap(h.x, h.x, false, false)
                              : __builtin_amdgcn_permlane32_swap(h.x, h.x, false, false);
    const auto b = SPAN == 16 ? __builtin_amdgcn_permlane16_swap(h.y, h.y, false, false)
                              : __builtin_amdgcn_permlane32_swap(h.y, h.y, false, false);
    lo = __builtin_bit_cast(T, make_uint2(a[0], b[0]));
    hi = __builtin_bit_cast(T, make_uint2(a[1], b[1]));
  }
}
template <int G, class T, class Op>
__device__ __forceinline__ T lane_group_reduce(T x, Op op) {
  static_assert(G >= 1 && G <= 64 && (G & (G - 1)) == 0, "group of 1..64 lanes");
  if constexpr (G >= 2) x = op(x, dpp_move<0xB1>(x));    // quad_perm [1,0,3,2]
  if constexpr (G >= 4) x = op(x, dpp_move<0x4E>(x));    // quad_perm [2,3,0,1]
  if constexpr (G >= 8) x = op(x, dpp_move<0x141>(x));   // row_half_mirror
  if constexpr (G >= 16) x = op(x, dpp_move<0x140>(x));  // row_mirror
  if constexpr (G >= 32) {
    T lo, hi;
    lane_swap<16>(x, lo, hi);
    x = op(lo, hi);
  }
  if constexpr (G >= 64) {
    T lo, hi;
    lane_swap<32>(x, lo, hi);
    x = op(lo, hi);
  }
  return x;
}
template <int G>
__device__ __forceinline__ float lane_group_sum(float x) {
  return lane_group_reduce<G>(x, SumOp{});
}

// Reduce `v` over a group of G consecutive lanes (G a power of two <= 1024).
// Groups of up to 64 lanes live in one wave and reduce with cross-lane
// shuffles only; larger groups span G/64 waves of the block and combine the
// per-wave values through `lds` (blockDim.x/64 entries), in wave order, so
// every lane of the group gets the same bits.  Every thread of the block must
// call this (it contains a barrier when G > 64).
template <int G, class T, class Op>
__device__ __forceinline__ T group_reduce(T v, Op op, T *lds) {
  constexpr int W = G < 64 ? G : 64;
  v = lane_group_reduce<W>(v, op);
  if constexpr (G > 64) {
    constexpr int WPG = G / 64;
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) lds[wave] = v;
    __syncthreads();
    const int first = (wave / WPG) * WPG;
    T r = lds[first];
#pragma unroll
    for (int i = 1; i < WPG; ++i) r = op(r, lds[first + i]);
    v = r;
  }
  return v;
}

// Streaming 16-byte load / store, marked non-temporal (data touched once).
// Measured on gfx950: non-temporal stores lift the row kernels by 5-15%
// (rms rows T=8192: 57 -> 48 us); non-temporal loads help the q/k and GDN
// kernels but slow the norm rows, and a split softmax's first pass keeps
// ordinary loads so its second pass re-reads the logits from the cache.
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 load_stream(const float4 *p) {
  const f32x4 v = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
#ifndef BH_STORE_SC1
#define BH_STORE_SC1 0
#endif
__device__ __forceinline__ void store_stream(float4 *p, float4 v) {
  f32x4 t = {v.x, v.y, v.z, v.w};
#if BH_STORE_SC1
  asm volatile("global_store_dwordx4 %0, %1, off sc1 nt" ::"v"(p), "v"(t) : "memory");
#else
  __builtin_nontemporal_store(t, reinterpret_cast<f32x4 *>(p));
#endif
}

// ---------------------------------------------------------------------------
// Device: scalar functions of the reference
// ---------------------------------------------------------------------------

// kernels::silu (src/kernels.rs:148-150)
__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }
// kernels::sigmoid (src/kernels.rs:162-164)
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }
// kernels::softplus (src/kernels.rs:153-159): ln(1 + e^x), identity above 20
__device__ __forceinline__ float softplus(float x) {
  return x > 20.0f ? x : logf(1.0f + expf(x));
}

// e^x through the hardware base-2 exponential (v_exp_f32, ~1 ulp) with the
// rounding error of x * log2(e) carried by FMA (a two-part log2(e)) and put
// back to first order: e^x = 2^t * 2^err ~ 2^t * (1 + err * ln 2).  Relative
// error a few 1e-7 for x <= 0 (what a softmax feeds it), against expf's
// ~1e-7; -inf gives exactly 0, NaN stays NaN.  Used where a kernel is bound
// by the exponentials and the result only needs the reference's tolerance.
__device__ __forceinline__ float exp_hw(float x) {
  constexpr float kL2E = 1.44269502162933349609375f;   // log2(e) rounded to f32
  constexpr float kL2ELo = 1.925963033500011e-08f;     // log2(e) - kL2E
  constexpr float kLn2 = 0.693147180559945309f;
  const float t = x * kL2E;
  float err = __builtin_fmaf(x, kL2E, -t);
  err = __builtin_fmaf(x, kL2ELo, err);
  const float r = __builtin_amdgcn_exp2f(t);
  return x == -INFINITY ? 0.0f : r * __builtin_fmaf(err, kLn2, 1.0f);
}

// silu with the hardware exponential (exp_hw) and reciprocal: within a few
// ulps of silu() -- for kernels whose outputs carry the 1e-5 tolerance, not
// for the bit-exact unary entry point.  Infinite and NaN inputs give what
// silu() gives (-inf: NaN; +inf: +inf).
__device__ __forceinline__ float silu_fast(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + exp_hw(-x));
}
// sigmoid the same way (within a few ulps of sigmoid())
__device__ __forceinline__ float sigmoid_fast(float x) {
  return __builtin_amdgcn_rcpf(1.0f + exp_hw(-x));
}

// gguf::half_to_f32 (src/gguf.rs:881-911) in integer arithmetic: exact for
// every one of the 65536 patterns, NaN payloads kept (no quieting).
__device__ __forceinline__ uint32_t half_bits_to_f32_bits(uint32_t h) {
  const uint32_t sign = (h >> 15) & 1u;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t man = h & 0x3ffu;
  if (exp == 0u) {
    if (man == 0u) return sign << 31;
    // subnormal: shift the mantissa up until bit 10 is set
    const uint32_t nbits = 32u - __clz(man);  // 1..10
    const uint32_t k = 11u - nbits;
    const uint32_t e = 113u - k;
    return (sign << 31) | (e << 23) | (((man << k) & 0x3ffu) << 13);
  }
  if (exp == 0x1fu) return (sign << 31) | 0x7f800000u | (man << 13);
  return (sign << 31) | ((exp + 112u) << 23) | (man << 13);
}

// One PQ2_0 weight: (code - 1) * scale with the IEEE product an x86 SSE
// multiply gives (src/kernels.rs:226).  The finite case is a single exact
// multiply; the two non-finite scale cases are spelled out because the GPU
// and SSE return different NaN bit patterns: a NaN scale comes back quieted
// with its payload, and 0 * inf is SSE's default NaN 0xFFC00000.
__device__ __forceinline__ float pq2_weight(uint32_t code, float scale, bool finite) {
  const float v = static_cast<float>(static_cast<int>(code) - 1) * scale;
  if (finite) return v;
  const uint32_t sb = __float_as_uint(scale);
  if ((sb & 0x7fffffu) != 0u) return __uint_as_float(sb | 0x00400000u);  // NaN
  if (code == 1u) return __uint_as_float(0xffc00000u);                   // 0*inf
  return v;                                                              // +-inf
}

}  // namespace bh

// Launch helper: bounds-checked grid, returns a status from the enclosing fn.
#define BH_LAUNCH(kernel, grid, block, shmem, stream, ...)                   \
  do {                                                                       \
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(block), shmem, stream,       \
                       __VA_ARGS__);                                         \
    int _st = ::bh::check_launch(#kernel);                                   \
    if (_st != BH_OK) return _st;                                            \
  } while (0)
