// Causal conv1d + SiLU over the GDN qkv channels, for any number of tokens.
//
// Reference: src/forward.rs:508-533 (one token): per channel c, win = the
// channel's k-1 cached inputs (oldest first) and the current input, acc =
// sum_j w[c*k + j] * win[j] in f32 with j ascending, out = silu(acc); the
// cache then drops its oldest sample and appends the current input.
//
// Over n_tok tokens the recurrence only shifts inputs, so every output is
// independent: with s_p = x[p][c] for p >= 0 and s_p = state[c][p + k - 1]
// for p < 0, out[t][c] = silu(sum_j w[c][j] * s_{t-k+1+j}) and the new state
// is s_{n_tok-k+1 ..  n_tok-1}.  One pass computes all outputs in parallel
// (the same products and additions, in the same order, as the per-token
// loop); a second, per-channel pass shifts the state, so an in-place state
// buffer is read completely before it is rewritten.
#include <hip/hip_runtime.h>

#include <string>

#include "common.hpp"
#include "conv.hpp"

namespace bh {
namespace {

constexpr int kBlock = 256;

// out[t][c..c+3] for k = 4, channels 16-byte aligned: a lane runs RUN
// consecutive tokens of its 4 channels with the taps and the 4-row input
// window in registers; the RUN input rows are loaded together before the
// first use.  The lanes of the first run (the only ones that read the cache)
// also write the new cache of their channels after reading the old one --
// s_{n_tok-3 .. n_tok-1}, taken from x or, for a batch of fewer than 3
// tokens, from the old cache they already hold -- so no second launch is
// needed and an in-place cache is safe (each cache entry is read and
// rewritten by the same lane).
template <int RUN>
__global__ __launch_bounds__(kBlock) void conv1d_silu4_kernel(ConvIn cv, float *out, size_t n4,
                                                              size_t n_tok, float *new_state) {
  const size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= n4) return;
  const size_t t0 = static_cast<size_t>(blockIdx.y) * RUN;
  const int c = static_cast<int>(i) * 4;
  const int nt = n_tok - t0 < static_cast<size_t>(RUN) ? static_cast<int>(n_tok - t0) : RUN;
  const float4 *x4 = reinterpret_cast<const float4 *>(cv.x) + i;
  const size_t row4 = static_cast<size_t>(cv.ch) / 4;
  float4 xr[RUN];
#pragma unroll
  for (int tt = 0; tt < RUN; ++tt)
    xr[tt] = load_stream(x4 + (t0 + (tt < nt ? tt : nt - 1)) * row4);
  float wv[4][4];  // [channel q][tap j]
  const float4 *w4 = reinterpret_cast<const float4 *>(cv.w + static_cast<size_t>(c) * 4);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 f = w4[q];
    wv[q][0] = f.x;
    wv[q][1] = f.y;
    wv[q][2] = f.z;
    wv[q][3] = f.w;
  }
  float4 win[4];
  if (t0 != 0) {  // runs start at 0 or at RUN >= 3: the window is three input rows
#pragma unroll
    for (int j = 0; j < 3; ++j) win[j] = x4[(t0 - 3 + j) * row4];
  } else {  // the first run: the window is the cache (oldest first)
    const float *st = cv.state + static_cast<size_t>(c) * 3;
#pragma unroll
    for (int j = 0; j < 3; ++j) win[j] = make_float4(st[j], st[3 + j], st[6 + j], st[9 + j]);
    if (new_state != nullptr) {
      // new cache entry e of channel c+q = s_{n_tok-3+e}: input row n_tok-3+e,
      // or for a batch of fewer than 3 tokens an old entry this lane holds.
      // Selects are per component on values: a select between a load and an
      // array element would become a load through a selected pointer and
      // move the window to scratch memory.
      auto entry = [&](int e) {
        const long p = static_cast<long>(n_tok) - 3 + e;
        const float4 xv = x4[static_cast<size_t>(p >= 0 ? p : 0) * row4];
        const float4 ov = sel4(p == -2, win[1], win[2]);
        return sel4(p >= 0, xv, ov);
      };
      const float4 n0 = entry(0), n1 = entry(1), n2 = entry(2);
      float *nst = new_state + static_cast<size_t>(c) * 3;
      nst[0] = n0.x; nst[1] = n1.x; nst[2] = n2.x;
      nst[3] = n0.y; nst[4] = n1.y; nst[5] = n2.y;
      nst[6] = n0.z; nst[7] = n1.z; nst[8] = n2.z;
      nst[9] = n0.w; nst[10] = n1.w; nst[11] = n2.w;
    }
  }
#pragma unroll
  for (int tt = 0; tt < RUN; ++tt) {
    if (tt < nt) {
      win[3] = xr[tt];
      // src/forward.rs:518-522: acc = sum_j w[c][j] * win[j], j ascending
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        acc.x += wv[0][j] * win[j].x;
        acc.y += wv[1][j] * win[j].y;
        acc.z += wv[2][j] * win[j].z;
        acc.w += wv[3][j] * win[j].w;
      }
      store_stream(reinterpret_cast<float4 *>(out + (t0 + tt) * cv.ch) + i,
                   make_float4(silu_fast(acc.x), silu_fast(acc.y), silu_fast(acc.z),
                               silu_fast(acc.w)));
#pragma unroll
      for (int j = 0; j < 3; ++j) win[j] = win[j + 1];
    }
  }
}

// Any k / layout: one output per lane.
__global__ __launch_bounds__(kBlock) void conv1d_silu_kernel(ConvIn cv, float *out, size_t total) {
  const size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= total) return;
  const size_t t = i / cv.ch;
  const int c = static_cast<int>(i - t * cv.ch);
  out[i] = silu(conv_at(cv, t, c));
}

// New state, one channel per lane (src/forward.rs:526-532 applied n_tok times).
__global__ __launch_bounds__(kBlock) void conv_state_kernel(const float *x, float *state, int ch,
                                                            int k, size_t n_tok) {
  const int c = blockIdx.x * kBlock + threadIdx.x;
  if (c >= ch || k < 2) return;
  const int n_prev = k - 1;
  float *st = state + static_cast<size_t>(c) * n_prev;
  // entry i becomes s_{n_tok - n_prev + i}; a cached source index (n_tok + i)
  // is always above i, so ascending order reads each old entry before it is
  // overwritten
  for (int i = 0; i < n_prev; ++i) {
    const long p = static_cast<long>(n_tok) - n_prev + i;
    st[i] = p >= 0 ? x[static_cast<size_t>(p) * ch + c] : st[n_tok + i];
  }
}

}  // namespace

int conv_check(const ConvIn &cv, const float *out, const char *who) {
  if (cv.k < 1 || cv.k > kMaxConvK)
    return fail(BH_ERR_SHAPE, std::string(who) + ": conv kernel size " + std::to_string(cv.k) +
                                  " must be in 1.." + std::to_string(kMaxConvK));
  if (cv.x == nullptr || cv.w == nullptr || out == nullptr || (cv.k > 1 && cv.state == nullptr))
    return fail(BH_ERR_ARG, std::string(who) + ": null pointer");
  if (out == cv.x)
    return fail(BH_ERR_ARG, std::string(who) +
                                ": the output must not alias the conv input (later tokens read it)");
  return BH_OK;
}

int conv_state_update(const ConvIn &cv, size_t n_tok, hipStream_t st) {
  if (cv.k < 2 || n_tok == 0) return ok();
  const unsigned grid = static_cast<unsigned>((cv.ch + kBlock - 1) / kBlock);
  BH_LAUNCH(conv_state_kernel, grid, kBlock, 0, st, cv.x, const_cast<float *>(cv.state), cv.ch,
            cv.k, n_tok);
  return ok();
}

}  // namespace bh

using namespace bh;

extern "C" int bh_conv1d_silu(const float *x, float *state, const float *w, size_t n_tok,
                              size_t ch, size_t k, float *out, bh_stream stream) {
  if (ch > 0x7fffffffu) return fail(BH_ERR_SHAPE, "conv1d_silu: too many channels");
  ConvIn cv{x, state, w, static_cast<int>(ch), static_cast<int>(k)};
  if (k < 1 || k > static_cast<size_t>(kMaxConvK))
    return fail(BH_ERR_SHAPE, "conv1d_silu: conv kernel size " + std::to_string(k) +
                                  " must be in 1.." + std::to_string(kMaxConvK));
  if (n_tok == 0 || ch == 0) return ok();
  if (int e = conv_check(cv, out, "conv1d_silu")) return e;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t total = n_tok * ch;
  constexpr int kRun = 8;  // tokens per lane ([4096, 10240]: 63.4 us; 4: 70.1, 16: 66.8)
  const size_t runs = (n_tok + kRun - 1) / kRun;
  if (k == 4 && ch % 4 == 0 && aligned16(x) && aligned16(out) && aligned16(w) && runs <= 65535) {
    const size_t n4 = ch / 4;
    BH_LAUNCH(conv1d_silu4_kernel<kRun>, dim3(static_cast<unsigned>((n4 + kBlock - 1) / kBlock),
                                              static_cast<unsigned>(runs)),
              kBlock, 0, st, cv, out, n4, n_tok, state);
    return ok();  // the kernel advanced the cache
  } else {
    if ((total + kBlock - 1) / kBlock > 0x7fffffffu)
      return fail(BH_ERR_SHAPE, "conv1d_silu: too many elements");
    BH_LAUNCH(conv1d_silu_kernel, static_cast<unsigned>((total + kBlock - 1) / kBlock), kBlock, 0,
              st, cv, out, total);
  }
  return conv_state_update(cv, n_tok, st);
}
