// Host-slice mirrors of the reference signatures (bh_host_*).
//
// Each one takes the Rust function's arguments as host pointers + lengths,
// checks them the way the Rust does (same error text), copies the inputs to
// the current device, runs the device entry point on a private stream,
// copies the result back and synchronises.  They exist so a Rust FFI module
// can keep the exact shapes of src/kernels.rs / src/rope.rs / src/prefill.rs
// while the arithmetic runs on the GPU.
#include <hip/hip_runtime.h>

#include <cstring>
#include <string>
#include <vector>

#include "common.hpp"

namespace bh {
namespace {

// Device buffer owned for the duration of one host call.
class DevBuf {
 public:
  DevBuf() = default;
  DevBuf(const DevBuf &) = delete;
  DevBuf &operator=(const DevBuf &) = delete;
  ~DevBuf() {
    if (p_ != nullptr) (void)hipFree(p_);
  }
  int alloc(size_t bytes) {
    if (bytes == 0) bytes = 16;
    return check_hip(hipMalloc(&p_, bytes), "hipMalloc");
  }
  template <class T>
  T *as() const {
    return static_cast<T *>(p_);
  }

 private:
  void *p_ = nullptr;
};

class Stream {
 public:
  Stream() { err_ = check_hip(hipStreamCreate(&s_), "hipStreamCreate"); }
  ~Stream() {
    if (s_ != nullptr) (void)hipStreamDestroy(s_);
  }
  int status() const { return err_; }
  hipStream_t get() const { return s_; }
  bh_stream handle() const { return reinterpret_cast<bh_stream>(s_); }

 private:
  hipStream_t s_ = nullptr;
  int err_ = BH_OK;
};

int upload(DevBuf &d, const void *src, size_t bytes, hipStream_t s) {
  if (int e = d.alloc(bytes)) return e;
  if (bytes == 0) return BH_OK;
  return check_hip(hipMemcpyAsync(d.as<void>(), src, bytes, hipMemcpyHostToDevice, s),
                   "hipMemcpyAsync H2D");
}

int download(void *dst, const DevBuf &d, size_t bytes, hipStream_t s) {
  if (bytes != 0) {
    if (int e = check_hip(hipMemcpyAsync(dst, d.as<void>(), bytes, hipMemcpyDeviceToHost, s),
                          "hipMemcpyAsync D2H"))
      return e;
  }
  return check_hip(hipStreamSynchronize(s), "hipStreamSynchronize");
}

}  // namespace
}  // namespace bh

using namespace bh;

extern "C" int bh_host_rms_norm(const float *x, size_t n, const float *w, float eps, float *out) {
  if (n == 0) return ok();
  Stream s;
  if (s.status()) return s.status();
  DevBuf dx, dw, dout;
  if (int e = upload(dx, x, n * 4, s.get())) return e;
  if (int e = upload(dw, w, n * 4, s.get())) return e;
  if (int e = dout.alloc(n * 4)) return e;
  if (int e = bh_rms_norm(dx.as<float>(), dw.as<float>(), n, eps, dout.as<float>(), s.handle()))
    return e;
  if (int e = download(out, dout, n * 4, s.get())) return e;
  return ok();
}

extern "C" int bh_host_rms_norm_rows(const float *x, size_t x_len, const float *w, size_t w_len,
                                     size_t row_len, float eps, float *out) {
  // shape errors first, with the reference's messages (src/kernels.rs:98-108)
  if (w_len != row_len)
    return fail(BH_ERR_SHAPE, "rms_norm_rows: weight len " + std::to_string(w_len) +
                                  " != row_len " + std::to_string(row_len));
  if (row_len == 0 || x_len % row_len != 0)
    return fail(BH_ERR_SHAPE, "rms_norm_rows: x len " + std::to_string(x_len) +
                                  " not divisible by row_len " + std::to_string(row_len));
  if (x_len == 0) return ok();
  Stream s;
  if (s.status()) return s.status();
  DevBuf dx, dw, dout;
  if (int e = upload(dx, x, x_len * 4, s.get())) return e;
  if (int e = upload(dw, w, w_len * 4, s.get())) return e;
  if (int e = dout.alloc(x_len * 4)) return e;
  if (int e = bh_rms_norm_rows(dx.as<float>(), x_len, dw.as<float>(), w_len, row_len, eps,
                               dout.as<float>(), s.handle()))
    return e;
  if (int e = download(out, dout, x_len * 4, s.get())) return e;
  return ok();
}

extern "C" int bh_host_l2_norm_rows(const float *x, size_t x_len, size_t row_len, float eps,
                                    float *out) {
  if (row_len == 0 || x_len % row_len != 0)
    return fail(BH_ERR_SHAPE, "l2_norm_rows: x len " + std::to_string(x_len) +
                                  " not divisible by row_len " + std::to_string(row_len));
  if (x_len == 0) return ok();
  Stream s;
  if (s.status()) return s.status();
  DevBuf dx, dout;
  if (int e = upload(dx, x, x_len * 4, s.get())) return e;
  if (int e = dout.alloc(x_len * 4)) return e;
  if (int e = bh_l2_norm_rows(dx.as<float>(), x_len, row_len, eps, dout.as<float>(), s.handle()))
    return e;
  if (int e = download(out, dout, x_len * 4, s.get())) return e;
  return ok();
}

extern "C" int bh_host_map_inplace(float *x, size_t n, int mode) {
  if (mode != BH_SILU && mode != BH_SIGMOID && mode != BH_SOFTPLUS)
    return fail(BH_ERR_ARG, "map_inplace: mode must be silu, sigmoid or softplus");
  if (n == 0) return ok();
  Stream s;
  if (s.status()) return s.status();
  DevBuf dx;
  if (int e = upload(dx, x, n * 4, s.get())) return e;
  if (int e = bh_unary(mode, dx.as<float>(), nullptr, n, dx.as<float>(), s.handle())) return e;
  if (int e = download(x, dx, n * 4, s.get())) return e;
  return ok();
}

extern "C" int bh_host_softmax_rows(const float *x, size_t x_len, size_t row_len, float *out) {
  if (row_len == 0 || x_len % row_len != 0)
    return fail(BH_ERR_SHAPE, "softmax_rows: x len " + std::to_string(x_len) +
                                  " not divisible by row_len " + std::to_string(row_len));
  if (x_len == 0) return ok();
  Stream s;
  if (s.status()) return s.status();
  DevBuf dx, dout;
  if (int e = upload(dx, x, x_len * 4, s.get())) return e;
  if (int e = dout.alloc(x_len * 4)) return e;
  if (int e = bh_softmax_rows(dx.as<float>(), x_len, row_len, 1.0f, dout.as<float>(), s.handle()))
    return e;
  if (int e = download(out, dout, x_len * 4, s.get())) return e;
  return ok();
}

extern "C" int bh_host_rope_imrope(float *head, size_t head_len, int64_t p_t, int64_t p_h,
                                   int64_t p_w, int64_t p_e, size_t n_dims,
                                   const int32_t sections[4], float freq_base) {
  // the reference debug-asserts n_dims <= head.len() and n_dims even (src/rope.rs:19-20)
  if (n_dims % 2 != 0 || n_dims > head_len)
    return fail(BH_ERR_SHAPE, "rope_imrope: n_dims " + std::to_string(n_dims) +
                                  " must be even and <= head len " + std::to_string(head_len));
  if (head_len == 0) return ok();
  // positions travel as int32 on the device; `p as f32` of a position beyond
  // the int32 range is not representable there
  const int64_t ps[4] = {p_t, p_h, p_w, p_e};
  int32_t pos[4];
  for (int i = 0; i < 4; ++i) {
    if (ps[i] < INT32_MIN || ps[i] > INT32_MAX)
      return fail(BH_ERR_RANGE, "rope_imrope: position outside the int32 range");
    pos[i] = static_cast<int32_t>(ps[i]);
  }
  Stream s;
  if (s.status()) return s.status();
  DevBuf dh, dp;
  if (int e = upload(dh, head, head_len * 4, s.get())) return e;
  if (int e = upload(dp, pos, sizeof(pos), s.get())) return e;
  if (int e = bh_rope_imrope(dh.as<float>(), 1, 1, head_len, dp.as<int32_t>(), n_dims, sections,
                             freq_base, s.handle()))
    return e;
  if (int e = download(head, dh, head_len * 4, s.get())) return e;
  return ok();
}

extern "C" int bh_host_decode_pq2_0_row(const uint8_t *raw, size_t raw_len, size_t ne0,
                                        float *out) {
  const size_t rb = bh_pq2_row_bytes(ne0);
  if (raw_len < rb)
    return fail(BH_ERR_SHAPE, "decode_pq2_0_row: raw len " + std::to_string(raw_len) +
                                  " < row bytes " + std::to_string(rb));
  if (ne0 == 0) return ok();
  Stream s;
  if (s.status()) return s.status();
  DevBuf draw, did, dout;
  const uint32_t id = 0;
  if (int e = upload(draw, raw, rb, s.get())) return e;
  if (int e = upload(did, &id, sizeof(id), s.get())) return e;
  if (int e = dout.alloc(ne0 * 4)) return e;
  if (int e = bh_pq2_embed_gather(draw.as<uint8_t>(), ne0, 1, did.as<uint32_t>(), 1,
                                  dout.as<float>(), nullptr, s.handle()))
    return e;
  if (int e = download(out, dout, ne0 * 4, s.get())) return e;
  return ok();
}

namespace {
// (base_row + n_rows) * rb, or false when it does not fit in size_t.
bool rows_end_bytes(uint64_t base_row, size_t n_rows, size_t rb, size_t *out) {
  const unsigned __int128 v = (static_cast<unsigned __int128>(base_row) + n_rows) * rb;
  if (v > static_cast<unsigned __int128>(SIZE_MAX)) return false;
  *out = static_cast<size_t>(v);
  return true;
}
}  // namespace

extern "C" int bh_host_batch_embed(const uint8_t *payload, size_t payload_len, size_t ne0,
                                   size_t n_rows, const uint32_t *tokens, size_t n_tok,
                                   float *out) {
  const size_t rb = bh_pq2_row_bytes(ne0);
  size_t tab_bytes = 0;
  if (!rows_end_bytes(0, n_rows, rb, &tab_bytes))
    return fail(BH_ERR_SHAPE, "batch_embed: n_rows * row bytes overflows");
  if (payload_len < tab_bytes)
    return fail(BH_ERR_SHAPE, "batch_embed: payload len " + std::to_string(payload_len) +
                                  " < n_rows * row bytes " + std::to_string(tab_bytes));
  size_t out_bytes = 0;
  if (!mul_size(n_tok, ne0, 4, &out_bytes))
    return fail(BH_ERR_SHAPE, "batch_embed: output size overflows");
  // Weights::row_f32 range check (src/weights.rs:337-341), first bad token wins
  for (size_t k = 0; k < n_tok; ++k) {
    if (tokens[k] >= n_rows)
      return fail(BH_ERR_RANGE, "Weights: row_f32(token_embd.weight): row " +
                                    std::to_string(tokens[k]) + " out of range (n_rows " +
                                    std::to_string(n_rows) + ")");
  }
  if (n_tok == 0 || ne0 == 0) return ok();
  Stream s;
  if (s.status()) return s.status();
  DevBuf dtab, dids, dout;
  if (int e = upload(dtab, payload, tab_bytes, s.get())) return e;
  if (int e = upload(dids, tokens, n_tok * 4, s.get())) return e;
  if (int e = dout.alloc(out_bytes)) return e;
  if (int e = bh_pq2_embed_gather(dtab.as<uint8_t>(), ne0, n_rows, dids.as<uint32_t>(), n_tok,
                                  dout.as<float>(), nullptr, s.handle()))
    return e;
  if (int e = download(out, dout, out_bytes, s.get())) return e;
  return ok();
}

namespace {
// Uploads rows [base_row, base_row + n_rows) of a host payload and runs
// bh_pq2_matmul_n on them; the caller has done the reference's checks.
int host_matmul_rows(const uint8_t *payload, size_t ne0, uint64_t base_row, size_t n_rows,
                     const float *x, size_t n_tok, float *y) {
  if (n_rows == 0 || n_tok == 0) return ok();
  const size_t rb = bh_pq2_row_bytes(ne0);
  Stream s;
  if (s.status()) return s.status();
  DevBuf dw, dx, dy;
  if (int e = upload(dw, payload + base_row * rb, n_rows * rb, s.get())) return e;
  if (int e = upload(dx, x, n_tok * ne0 * 4, s.get())) return e;
  if (int e = dy.alloc(n_tok * n_rows * 4)) return e;
  if (int e = bh_pq2_matmul_n(dw.as<uint8_t>(), n_rows * rb, ne0, 0, n_rows, dx.as<float>(),
                              n_tok * ne0, n_tok, dy.as<float>(), n_tok * n_rows, s.handle()))
    return e;
  return download(y, dy, n_tok * n_rows * 4, s.get());
}

}  // namespace

extern "C" int bh_host_dot_pq2_0_row(const uint8_t *payload, size_t payload_len, size_t ne0,
                                     uint64_t row, const float *x, size_t x_len, float *out) {
  // src/kernels.rs:239-256
  if (x_len != ne0)
    return fail(BH_ERR_SHAPE, "dot_pq2_0_row: x length " + std::to_string(x_len) + " != ne0 " +
                                  std::to_string(ne0));
  const size_t rb = bh_pq2_row_bytes(ne0);
  size_t end = 0;
  if (!rows_end_bytes(row, 1, rb, &end))
    return fail(BH_ERR_SHAPE, "dot_pq2_0_row: row " + std::to_string(row) +
                                  " byte range overflows, payload is " +
                                  std::to_string(payload_len));
  const size_t start = end - rb;
  if (end > payload_len)
    return fail(BH_ERR_SHAPE, "dot_pq2_0_row: row " + std::to_string(row) + " needs bytes " +
                                  std::to_string(start) + ".." + std::to_string(end) +
                                  ", payload is " + std::to_string(payload_len));
  if (ne0 == 0) {
    *out = 0.0f;
    return ok();
  }
  return host_matmul_rows(payload, ne0, row, 1, x, 1, out);
}

extern "C" int bh_host_pq2_matvec_range(const uint8_t *payload, size_t payload_len, size_t ne0,
                                        uint64_t base_row, size_t n_rows, const float *x,
                                        size_t x_len, float *y, size_t y_len) {
  // src/kernels.rs:291-307
  if (x_len != ne0)
    return fail(BH_ERR_SHAPE, "pq2_matvec_range: x length " + std::to_string(x_len) +
                                  " != ne0 " + std::to_string(ne0));
  if (y_len < n_rows) return fail(BH_ERR_SHAPE, "pq2_matvec_range: y too small");
  const size_t rb = bh_pq2_row_bytes(ne0);
  size_t byte_len = 0;
  if (!rows_end_bytes(base_row, n_rows, rb, &byte_len))
    return fail(BH_ERR_SHAPE, "pq2_matvec_range: row range byte length overflows");
  if (byte_len > payload_len)
    return fail(BH_ERR_SHAPE, "pq2_matvec_range: rows " + std::to_string(base_row) + ".." +
                                  std::to_string(base_row + n_rows) + " need " +
                                  std::to_string(byte_len) + " bytes, payload is " +
                                  std::to_string(payload_len));
  return host_matmul_rows(payload, ne0, base_row, n_rows, x, 1, y);
}

extern "C" int bh_host_pq2_matmul_n(const uint8_t *payload, size_t payload_len, size_t ne0,
                                    uint64_t base_row, size_t n_rows, const float *x,
                                    size_t x_len, size_t n_tok, float *y, size_t y_len) {
  // src/kernels.rs:349-364
  if (x_len != n_tok * ne0)
    return fail(BH_ERR_SHAPE, "pq2_matmul_n: x length " + std::to_string(x_len) + " != n_tok " +
                                  std::to_string(n_tok) + " * ne0 " + std::to_string(ne0));
  if (y_len < n_tok * n_rows) return fail(BH_ERR_SHAPE, "pq2_matmul_n: y too small");
  const size_t rb = bh_pq2_row_bytes(ne0);
  size_t need = 0;
  if (!rows_end_bytes(base_row, n_rows, rb, &need))
    return fail(BH_ERR_SHAPE, "pq2_matmul_n: overflow");
  if (need > payload_len) return fail(BH_ERR_SHAPE, "pq2_matmul_n: row range exceeds payload");
  return host_matmul_rows(payload, ne0, base_row, n_rows, x, n_tok, y);
}

extern "C" int bh_host_gdn_step(const float *q, size_t q_len, const float *k, size_t k_len,
                                const float *v, size_t v_len, const float *gate, size_t gate_len,
                                const float *beta, size_t beta_len, float *state, size_t state_len,
                                float *attn, size_t attn_len) {
  // src/gdn.rs:26-28 fixes the shape; the reference indexes its slices
  // (panicking when one is short), this entry point reports it instead
  constexpr size_t S = 128, HK = 16, HV = 48;
  const struct {
    const char *name;
    size_t len, need;
  } args[] = {{"q", q_len, HK * S},
              {"k", k_len, HK * S},
              {"v", v_len, HV * S},
              {"gate", gate_len, HV},
              {"beta", beta_len, HV},
              {"state", state_len, HV * S * S},
              {"attn", attn_len, HV * S}};
  for (const auto &a : args)
    if (a.len < a.need)
      return fail(BH_ERR_SHAPE, std::string("gdn_step: ") + a.name + " len " +
                                    std::to_string(a.len) + " < " + std::to_string(a.need));
  Stream s;
  if (s.status()) return s.status();
  DevBuf dq, dk, dv, dg, db, dst, dattn;
  if (int e = upload(dq, q, HK * S * 4, s.get())) return e;
  if (int e = upload(dk, k, HK * S * 4, s.get())) return e;
  if (int e = upload(dv, v, HV * S * 4, s.get())) return e;
  if (int e = upload(dg, gate, HV * 4, s.get())) return e;
  if (int e = upload(db, beta, HV * 4, s.get())) return e;
  if (int e = upload(dst, state, HV * S * S * 4, s.get())) return e;
  if (int e = dattn.alloc(HV * S * 4)) return e;
  if (int e = bh_gdn_step(dq.as<float>(), dk.as<float>(), dv.as<float>(), dg.as<float>(),
                          db.as<float>(), dst.as<float>(), dattn.as<float>(), 1, HK, HV, S,
                          s.handle()))
    return e;
  if (int e = download(state, dst, HV * S * S * 4, s.get())) return e;
  if (int e = download(attn, dattn, HV * S * 4, s.get())) return e;
  return ok();
}
