// bonsai_kernels.hpp -- C++ mirror of the reference's kernel interface over
// the bonsai HIP library's C ABI (include/bonsai_hip.h).
//
// The reference engine is Rust; its hot-path kernels are free functions in
// src/kernels.rs and src/rope.rs that take slices and return Vec<f32> or
// Result<Vec<f32>, String>.  This header keeps those names, argument meanings
// and error behaviour so host code (and the tests in tests/cpp/) read like
// the reference:
//
//   kernels::rms_norm(x, w, eps)                -> std::vector<float>
//   kernels::rms_norm_inplace(x, w, eps)
//   kernels::rms_norm_rows(x, w, row_len, eps)  -> Result<std::vector<float>>
//   kernels::l2_norm_rows(x, row_len, eps)      -> Result<std::vector<float>>
//   kernels::silu / softplus / sigmoid(float)   -> float
//   kernels::map_inplace(x, Act)
//   kernels::softmax_rows(x, row_len)           -> Result<std::vector<float>>
//   kernels::pq2_row_bytes(ne0)                 -> size_t
//   kernels::decode_pq2_0_row(raw, ne0)         -> std::vector<float>
//   kernels::dot_pq2_0_row(payload, ne0, row, x)            -> Result<float>
//   kernels::pq2_matvec_range(payload, ne0, base, n, x, y)  -> Result<void>
//   kernels::pq2_matmul_n(payload, ne0, base, n, x, n_tok, y) -> Result<void>
//   rope::rope_imrope(head, p_t, p_h, p_w, p_e, n_dims, sections, freq_base)
//   prefill::batch_embed(payload, ne0, n_rows, tokens) -> Result<std::vector<float>>
//   gdn::gdn_step(q, k, v, gate, beta, state, attn)
//   gdn::zero_state()                                  -> std::vector<float>
//
// Every call runs on the current HIP device (host memory in, host memory
// out, synchronous), through the bh_host_* entry points.  A HIP failure is
// reported as an Err like a shape error (the reference has no such case).
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "../../include/bonsai_hip.h"

namespace bonsai {

// Result<T, String> of the reference: either a value or an error message.
template <class T>
class Result {
 public:
  static Result ok(T v) { return Result(std::move(v), std::string(), true); }
  static Result err(std::string e) { return Result(T(), std::move(e), false); }
  bool is_ok() const { return ok_; }
  bool is_err() const { return !ok_; }
  // unwrap(): the value, or throws std::runtime_error with the message
  const T &unwrap() const {
    if (!ok_) throw std::runtime_error("called unwrap() on an Err: " + err_);
    return val_;
  }
  const std::string &error() const { return err_; }

 private:
  Result(T v, std::string e, bool ok) : val_(std::move(v)), err_(std::move(e)), ok_(ok) {}
  T val_;
  std::string err_;
  bool ok_;
};

namespace detail {
inline void check_or_throw(int st) {
  if (st != BH_OK) throw std::runtime_error(bh_last_error());
}
}  // namespace detail

namespace kernels {

enum class Act { Silu = BH_SILU, Sigmoid = BH_SIGMOID, Softplus = BH_SOFTPLUS };

// src/kernels.rs:59 (w must hold x.size() values; the reference indexes it)
inline std::vector<float> rms_norm(const std::vector<float> &x, const std::vector<float> &w,
                                   float eps) {
  std::vector<float> out(x.size());
  if (w.size() < x.size()) throw std::out_of_range("rms_norm: weight shorter than x");
  detail::check_or_throw(bh_host_rms_norm(x.data(), x.size(), w.data(), eps, out.data()));
  return out;
}

// src/kernels.rs:80
inline void rms_norm_inplace(std::vector<float> &x, const std::vector<float> &w, float eps) {
  x = rms_norm(x, w, eps);
}

// src/kernels.rs:97
inline Result<std::vector<float>> rms_norm_rows(const std::vector<float> &x,
                                                const std::vector<float> &w, size_t row_len,
                                                float eps) {
  std::vector<float> out(x.size());
  const int st = bh_host_rms_norm_rows(x.data(), x.size(), w.data(), w.size(), row_len, eps,
                                       out.data());
  if (st != BH_OK) return Result<std::vector<float>>::err(bh_last_error());
  return Result<std::vector<float>>::ok(std::move(out));
}

// src/kernels.rs:126
inline Result<std::vector<float>> l2_norm_rows(const std::vector<float> &x, size_t row_len,
                                               float eps) {
  std::vector<float> out(x.size());
  const int st = bh_host_l2_norm_rows(x.data(), x.size(), row_len, eps, out.data());
  if (st != BH_OK) return Result<std::vector<float>>::err(bh_last_error());
  return Result<std::vector<float>>::ok(std::move(out));
}

// src/kernels.rs:167
inline void map_inplace(std::vector<float> &x, Act f) {
  detail::check_or_throw(bh_host_map_inplace(x.data(), x.size(), static_cast<int>(f)));
}

inline float apply(Act f, float v) {
  std::vector<float> one{v};
  map_inplace(one, f);
  return one[0];
}

// src/kernels.rs:148, 153, 162 (one value through the device kernel)
inline float silu(float x) { return apply(Act::Silu, x); }
inline float softplus(float x) { return apply(Act::Softplus, x); }
inline float sigmoid(float x) { return apply(Act::Sigmoid, x); }

// src/kernels.rs:175
inline Result<std::vector<float>> softmax_rows(const std::vector<float> &x, size_t row_len) {
  std::vector<float> out(x.size());
  const int st = bh_host_softmax_rows(x.data(), x.size(), row_len, out.data());
  if (st != BH_OK) return Result<std::vector<float>>::err(bh_last_error());
  return Result<std::vector<float>>::ok(std::move(out));
}

// src/kernels.rs:209
inline size_t pq2_row_bytes(size_t ne0) { return bh_pq2_row_bytes(ne0); }

// src/kernels.rs:214
inline std::vector<float> decode_pq2_0_row(const std::vector<uint8_t> &raw, size_t ne0) {
  std::vector<float> out(ne0);
  detail::check_or_throw(bh_host_decode_pq2_0_row(raw.data(), raw.size(), ne0, out.data()));
  return out;
}

// src/kernels.rs:233-262
inline Result<float> dot_pq2_0_row(const std::vector<uint8_t> &payload, size_t ne0, uint64_t row,
                                   const std::vector<float> &x) {
  float out = 0.0f;
  const int st = bh_host_dot_pq2_0_row(payload.data(), payload.size(), ne0, row, x.data(),
                                       x.size(), &out);
  if (st != BH_OK) return Result<float>::err(bh_last_error());
  return Result<float>::ok(out);
}

// src/kernels.rs:283-333: y[r] = row(base_row + r) . x for r < n_rows (y may
// be longer; only the first n_rows entries are written)
inline Result<bool> pq2_matvec_range(const std::vector<uint8_t> &payload, size_t ne0,
                                     uint64_t base_row, size_t n_rows,
                                     const std::vector<float> &x, std::vector<float> &y) {
  const int st = bh_host_pq2_matvec_range(payload.data(), payload.size(), ne0, base_row, n_rows,
                                          x.data(), x.size(), y.data(), y.size());
  if (st != BH_OK) return Result<bool>::err(bh_last_error());
  return Result<bool>::ok(true);
}

// src/kernels.rs:340-423: x [n_tok][ne0], y [n_tok][n_rows]
inline Result<bool> pq2_matmul_n(const std::vector<uint8_t> &payload, size_t ne0,
                                 uint64_t base_row, size_t n_rows, const std::vector<float> &x,
                                 size_t n_tok, std::vector<float> &y) {
  const int st = bh_host_pq2_matmul_n(payload.data(), payload.size(), ne0, base_row, n_rows,
                                      x.data(), x.size(), n_tok, y.data(), y.size());
  if (st != BH_OK) return Result<bool>::err(bh_last_error());
  return Result<bool>::ok(true);
}

}  // namespace kernels

namespace rope {

// src/rope.rs:9 (in place on one head vector)
inline void rope_imrope(std::vector<float> &head, int64_t p_t, int64_t p_h, int64_t p_w,
                        int64_t p_e, size_t n_dims, std::array<int32_t, 4> sections,
                        float freq_base) {
  detail::check_or_throw(bh_host_rope_imrope(head.data(), head.size(), p_t, p_h, p_w, p_e,
                                             n_dims, sections.data(), freq_base));
}

}  // namespace rope

namespace prefill {

// src/prefill.rs:143 over a PQ2_0 token_embd payload of n_rows rows: the
// tile [tokens.size()][ne0], or the row_f32 range error of src/weights.rs:337
inline Result<std::vector<float>> batch_embed(const std::vector<uint8_t> &payload, size_t ne0,
                                              size_t n_rows, const std::vector<uint32_t> &tokens) {
  std::vector<float> out(tokens.size() * ne0);
  const int st = bh_host_batch_embed(payload.data(), payload.size(), ne0, n_rows, tokens.data(),
                                     tokens.size(), out.data());
  if (st != BH_OK) return Result<std::vector<float>>::err(bh_last_error());
  return Result<std::vector<float>>::ok(std::move(out));
}

}  // namespace prefill

namespace gdn {

// src/gdn.rs:17 (s = 128, h_k = 16, h_v = 48; one token): state advanced in
// place, attn written.  The reference indexes its slices; a short one throws
// std::out_of_range here.
inline void gdn_step(const std::vector<float> &q, const std::vector<float> &k,
                     const std::vector<float> &v, const std::vector<float> &gate,
                     const std::vector<float> &beta, std::vector<float> &state,
                     std::vector<float> &attn) {
  const int st = bh_host_gdn_step(q.data(), q.size(), k.data(), k.size(), v.data(), v.size(),
                                  gate.data(), gate.size(), beta.data(), beta.size(),
                                  state.data(), state.size(), attn.data(), attn.size());
  if (st == BH_ERR_SHAPE) throw std::out_of_range(bh_last_error());
  detail::check_or_throw(st);
}

// src/gdn.rs:80
inline std::vector<float> zero_state() { return std::vector<float>(48 * 128 * 128, 0.0f); }

}  // namespace gdn

}  // namespace bonsai
