// Causal conv1d window helpers shared by the standalone conv kernel
// (conv.hip) and the fused GDN prep (elementwise.hip).  Semantics: see
// conv.hip (src/forward.rs:508-533).
#pragma once

#include <hip/hip_runtime.h>

#include "common.hpp"

namespace bh {

constexpr int kMaxConvK = 64;

struct ConvIn {
  const float *x;      // [n_tok][ch] conv inputs (the qkv projections)
  const float *state;  // [ch][k-1] cached inputs, oldest first
  const float *w;      // [ch][k] taps
  int ch, k;
};

// Pre-activation of token t, channel c: sum_j w[c][j] * s_{t-k+1+j} in f32,
// j ascending (s_p = x[p][c], or the cache for p < 0).
__device__ __forceinline__ float conv_at(const ConvIn &cv, size_t t, int c) {
  float acc = 0.0f;
  for (int j = 0; j < cv.k; ++j) {
    const long p = static_cast<long>(t) - (cv.k - 1) + j;
    const float s = p >= 0 ? cv.x[static_cast<size_t>(p) * cv.ch + c]
                           : cv.state[static_cast<size_t>(c) * (cv.k - 1) + (p + cv.k - 1)];
    acc += cv.w[static_cast<size_t>(c) * cv.k + j] * s;
  }
  return acc;
}

// The same for channels c..c+3 (c a multiple of 4; x rows and w 16-byte
// aligned), K taps known at compile time.
template <int K>
__device__ __forceinline__ float4 conv_window4(const ConvIn &cv, size_t t, int c) {
  float wv[4][K];
  const float4 *w4 = reinterpret_cast<const float4 *>(cv.w + static_cast<size_t>(c) * K);
#pragma unroll
  for (int f = 0; f < K; ++f) {  // the 4K taps of channels c..c+3, contiguous
    const float4 q = w4[f];
    const float e[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int u = 0; u < 4; ++u) wv[(4 * f + u) / K][(4 * f + u) % K] = e[u];
  }
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const long p = static_cast<long>(t) - (K - 1) + j;
    float4 s;
    if (p >= 0) {
      s = reinterpret_cast<const float4 *>(cv.x + static_cast<size_t>(p) * cv.ch)[c / 4];
    } else {
      const float *st = cv.state + static_cast<size_t>(c) * (K - 1) + (p + K - 1);
      s = make_float4(st[0], st[K - 1], st[2 * (K - 1)], st[3 * (K - 1)]);
    }
    acc.x += wv[0][j] * s.x;
    acc.y += wv[1][j] * s.y;
    acc.z += wv[2][j] * s.z;
    acc.w += wv[3][j] * s.w;
  }
  return acc;
}

// Component-wise select of two float4 values.  Selecting between a load and
// an array element with ?: can compile to a load through a selected pointer,
// which moves the array to scratch memory; selecting values does not.
__device__ __forceinline__ float4 sel4(bool c, float4 a, float4 b) {
  return make_float4(c ? a.x : b.x, c ? a.y : b.y, c ? a.z : b.z, c ? a.w : b.w);
}

// Argument checks shared by the conv entry points (BH_OK or a status).
int conv_check(const ConvIn &cv, const float *out, const char *who);
// The state shift after a pass over n_tok tokens (second launch on `st`).
int conv_state_update(const ConvIn &cv, size_t n_tok, hipStream_t st);

}  // namespace bh
