// Closed form of a run of identical sequential f32 additions.
//
// The reference's rms_norm sums the squares of a row one after another in
// f32 (src/kernels.rs:65-68).  On a PQ2_0 row whose codes are ternary
// (0, 1, 2: weights -d, 0, +d) every square of a 128-weight block is either
// d*d or +0, and adding +0 to a non-negative sum leaves it unchanged, so a
// block's part of that sequence is "add x = d*d to s, n times".  This header
// evaluates such a run without n dependent additions and returns the same
// bits as the loop.
//
// Why it is exact.  Let s lie in the binade [2^E, 2^(E+1)) with unit in the
// last place u = 2^(E-23), s = S*u (2^23 <= S < 2^24), and x = (q + f)*u
// with integer q >= 0 and 0 <= f < 1.  While the exact s_i + x stays below
// 2^(E+1), round-to-nearest-even gives s_(i+1) = s_i + m*u with
//   m = q       if f < 1/2,
//   m = q + 1   if f > 1/2,
//   and, for f = 1/2 (a tie), the even one of S_i + q, S_i + q + 1: once S_i
//   is even that is S_i + q + (q & 1) for every later step (the result is
//   even again), so an odd S_i takes one real addition first.
// Step i (from 0) keeps the binade exactly when i*m < C = 2^24 - S - q
// (f < 1 makes the fractional part irrelevant), so k = ceil(C / m) steps
// are one multiply-add on the integer mantissa; the step that leaves the
// binade is a real f32 addition, and the loop starts over in the next
// binade.  A run crosses at most a few binades, so a 128-weight block costs
// a handful of integer operations instead of up to 128 dependent adds.
// When m = 0 (x below half an ulp of s) the sum no longer moves.
#pragma once

#include <cstdint>

// Reciprocal used for the step count: the hardware approximation on the GPU
// (within 1 ulp), IEEE division on the host.  Either is corrected to the
// exact integer quotient.
#ifndef BH_SEQ_RCP
#if defined(__HIP_DEVICE_COMPILE__)
#define BH_SEQ_RCP(v) __builtin_amdgcn_rcpf(v)
#else
#define BH_SEQ_RCP(v) (1.0f / (v))
#endif
#endif

namespace bh {

// a * b for a, b < 2^24 whose product fits 32 bits: the GPU's full-rate
// 24-bit multiply (the 32-bit one is quarter rate).
__host__ __device__ inline uint32_t seq_mul24(uint32_t a, uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __umul24(a, b);
#else
  return a * b;
#endif
}

__host__ __device__ inline uint32_t seq_f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ inline float seq_u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// The value of `for (i = 0; i < n; ++i) s = s + x;` in f32 (round to nearest
// even) for s >= +0 and x a positive normal f32.  A non-finite s stays what
// the loop would make it (s + x).
__host__ __device__ inline float repeat_add_f32(float s, float x, uint32_t n) {
  while (n > 0) {
    const uint32_t sb = seq_f2u(s);
    if (sb >= 0x7f800000u) return s + x;  // inf or NaN: unchanged by further adds
    if (sb == 0u) {                       // +0 + x = x
      s = x;
      --n;
      continue;
    }
    const uint32_t xb = seq_f2u(x);
    const int es = static_cast<int>(sb >> 23);  // biased exponents (both normal)
    const int ex = static_cast<int>(xb >> 23);
    if (ex >= es) {  // x at least the binade of s: no run within a binade
      s = s + x;
      --n;
      continue;
    }
    const int sh = es - ex;  // 1..: x / u = MX / 2^sh
    if (sh >= 25) return s;  // x < u/2: every further add rounds back to s
    const uint32_t S = (sb & 0x7fffffu) | 0x800000u;
    const uint32_t MX = (xb & 0x7fffffu) | 0x800000u;
    const uint32_t q = MX >> sh;
    const uint32_t rem = MX & ((1u << sh) - 1u);
    const uint32_t half = 1u << (sh - 1);
    uint32_t m;
    if (rem == half) {
      if (S & 1u) {  // a tie from an odd mantissa: one real add makes it even
        s = s + x;
        --n;
        continue;
      }
      m = q + (q & 1u);
    } else {
      m = q + (rem > half ? 1u : 0u);
    }
    if (m == 0u) return s;
    const int32_t C = (1 << 24) - static_cast<int32_t>(S) - static_cast<int32_t>(q);
    if (C <= 0) {  // the next add leaves the binade
      s = s + x;
      --n;
      continue;
    }
    // all n steps fit when (n - 1) * m < C (n <= 2^24, m <= 2^23 + 1: the
    // product fits 64 bits); otherwise ceil(C / m) of them do
    const uint32_t k = static_cast<uint64_t>(n - 1u) * m < static_cast<uint64_t>(C)
                           ? n
                           : (static_cast<uint32_t>(C) - 1u) / m + 1u;
    const uint32_t Sn = S + k * m;  // <= 2^24: at most the binade's upper end
    s = Sn == (1u << 24) ? seq_u2f(static_cast<uint32_t>(es + 1) << 23)
                         : seq_u2f((static_cast<uint32_t>(es) << 23) | (Sn & 0x7fffffu));
    n -= k;
  }
  return s;
}

// One step of the same evaluation without branches, for a wave whose lanes
// each walk their own row: applies the run's steps that stay in the current
// binade of s, then (if any remain) the one step that leaves it as a real
// f32 addition, and returns the steps still to do.  Repeating it until n is 0
// gives repeat_add_f32's result.  1 <= n <= 256 (a 128-weight block's run
// fits): every product of a step count and m then fits the 24-bit multiply,
// the quotient ceil(C / m) is needed only when it is below n, and the f32
// reciprocal gets it within one of the exact value, which one integer
// comparison each way corrects.
__host__ __device__ inline uint32_t repeat_add_step_f32(float &s, float x, uint32_t n) {
  // Written as selects only: the GPU walks one row per lane and a branch per
  // case would serialise the lanes.  x / u is formed exactly by a power-of-two
  // scaling; m is then x / u rounded half to even (for f != 1/2 that is the
  // nearest integer, for a tie it is q + (q & 1)) and q its floor.
  const uint32_t sb = seq_f2u(s);
  const int es = static_cast<int>(sb >> 23);
  const float xu_raw = __builtin_ldexpf(x, 150 - es);  // x / u, exact
  const float xu = xu_raw < 16777216.0f ? xu_raw : 16777216.0f;  // x >= 2^E: no run
  const float qf = __builtin_floorf(xu);
  const float mf = __builtin_rintf(xu);
  const bool tie = xu - qf == 0.5f;
  const uint32_t q = static_cast<uint32_t>(qf);
  const uint32_t m = static_cast<uint32_t>(mf);
  const uint32_t S = (sb & 0x7fffffu) | 0x800000u;
  const int32_t C = (1 << 24) - static_cast<int32_t>(S) - static_cast<int32_t>(q);
  const bool special = sb - 1u >= 0x7f7fffffu;  // +0, inf or NaN
  const bool nofit = special | (xu >= 8388608.0f) | (tie & ((S & 1u) != 0u)) | (C <= 0);
  // K = floor((C - 1) / m), needed only when the whole run does not fit
  const uint32_t c1 = C > 0 ? static_cast<uint32_t>(C) - 1u : 0u;
  const float kf = static_cast<float>(c1) * BH_SEQ_RCP(mf > 1.0f ? mf : 1.0f);
  uint32_t K = static_cast<uint32_t>(kf < 256.0f ? kf : 256.0f);
  K -= static_cast<uint32_t>(seq_mul24(K, m) > c1);
  K += static_cast<uint32_t>(seq_mul24(K + 1u, m) <= c1);
  const bool fits = seq_mul24(n - 1u, m) <= c1;
  const uint32_t k = nofit ? 0u : (fits ? n : K + 1u);
  // s + k*m ulps: adding to the bit pattern carries into the exponent field
  // exactly when the mantissa reaches 2^24 (the binade's upper end)
  const float run = seq_u2f(sb + seq_mul24(k, m));
  const bool more = n > k;
  s = more ? run + x : run;
  return (special && sb != 0u) || !more ? 0u : n - k - 1u;
}

}  // namespace bh
