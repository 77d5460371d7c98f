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

// out[t][c..c+3] for k = 4, channels 16-byte aligned.
__global__ __launch_bounds__(kBlock) void conv1d_silu4_kernel(ConvIn cv, float *out, size_t n4,
                                                              size_t total) {
  const size_t i = static_cast<size_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= total) return;
  const size_t t = i / n4;
  const int c = static_cast<int>(i - t * n4) * 4;
  const float4 acc = conv_window4<4>(cv, t, c);
  store_stream(reinterpret_cast<float4 *>(out + t * cv.ch) + c / 4,
               make_float4(silu(acc.x), silu(acc.y), silu(acc.z), silu(acc.w)));
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
  if (k == 4 && ch % 4 == 0 && aligned16(x) && aligned16(out) && aligned16(w)) {
    const size_t n4 = ch / 4, t4 = n_tok * n4;
    BH_LAUNCH(conv1d_silu4_kernel, static_cast<unsigned>((t4 + kBlock - 1) / kBlock), kBlock, 0,
              st, cv, out, n4, t4);
  } else {
    if ((total + kBlock - 1) / kBlock > 0x7fffffffu)
      return fail(BH_ERR_SHAPE, "conv1d_silu: too many elements");
    BH_LAUNCH(conv1d_silu_kernel, static_cast<unsigned>((total + kBlock - 1) / kBlock), kBlock, 0,
              st, cv, out, total);
  }
  return conv_state_update(cv, n_tok, st);
}
