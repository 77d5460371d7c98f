// CPU check of bh::repeat_add_f32 (csrc/seqsum.hpp) against the plain loop of
// sequential f32 additions it replaces.  Built with g++ by tests/test_seqsum.py
// (x86-64 SSE arithmetic: IEEE f32, round to nearest even, no contraction).
#define __host__
#define __device__
// The GPU's reciprocal is within 1 ulp; the step count must come out exact
// whichever way it errs, so the test is built with the IEEE reciprocal and
// with it moved one ulp down or up (-DRCP_ULP=-1 / 1).
#include <cmath>
#ifndef RCP_ULP
#define RCP_ULP 0
#endif
static inline float test_rcp(float v) {
  float r = 1.0f / v;
  if (RCP_ULP < 0) r = std::nextafter(r, 0.0f);
  if (RCP_ULP > 0) r = std::nextafter(r, 2.0f * r);
  return r;
}
#define BH_SEQ_RCP(v) test_rcp(v)
#include "../../ternary-bonsai-inference_amd/csrc/seqsum.hpp"

#include <cstdint>
#include <cstdio>
#include <cstring>

namespace {

uint64_t g_state = 0x9e3779b97f4a7c15ull;
uint64_t next() {  // splitmix64
  uint64_t z = (g_state += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
uint32_t below(uint32_t n) { return static_cast<uint32_t>(next() % n); }

float bits(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
uint32_t ubits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

float loop_add(float s, float x, uint32_t n) {
  volatile float acc = s;  // one rounding per addition, as the reference
  for (uint32_t i = 0; i < n; ++i) acc = acc + x;
  return acc;
}

// A positive normal f32 with biased exponent e and a mantissa drawn to hit
// the interesting cases (powers of two, all-ones, low-bit patterns).
float pick(int e) {
  uint32_t man;
  switch (below(6)) {
    case 0: man = 0; break;
    case 1: man = 0x7fffffu; break;
    case 2: man = below(16); break;
    case 3: man = 0x7fffffu - below(16); break;
    default: man = static_cast<uint32_t>(next()) & 0x7fffffu;
  }
  if (e < 1) e = 1;
  if (e > 254) e = 254;
  return bits((static_cast<uint32_t>(e) << 23) | man);
}

int g_fail = 0;
long g_cases = 0;
void check(float s, float x, uint32_t n) {
  ++g_cases;
  const float want = loop_add(s, x, n);
  const float got = bh::repeat_add_f32(s, x, n);
  float st = s;
  uint32_t left = n, steps = 0;
  while (left > 0 && steps < 100000) {  // runs of at most 256 at a time
    const uint32_t part = left < 256 ? left : 256;
    left = left - part + bh::repeat_add_step_f32(st, x, part);
    ++steps;
  }
  if (ubits(want) != ubits(got) || ubits(want) != ubits(st)) {
    if (g_fail < 10)
      std::printf("MISMATCH s=%08x x=%08x n=%u: loop %08x closed form %08x steps %08x\n", ubits(s),
                  ubits(x), n, ubits(want), ubits(got), ubits(st));
    ++g_fail;
  }
}

// f16 value of bits h (finite), widened exactly
float half_val(uint32_t h) {
  const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
  float v = e == 0 ? static_cast<float>(m) * bits(0x33800000u)  // m * 2^-24
                   : bits(((e + 112u) << 23) | (m << 13));
  return v;
}

}  // namespace

int main() {
  // random runs: s from 0 or any binade, x from a few binades above s down
  // to far below its half ulp, n up to 5000
  for (int it = 0; it < 120000; ++it) {
    const int es = 20 + static_cast<int>(below(200));
    const float s = below(10) == 0 ? 0.0f : pick(es);
    const float x = pick(es + 3 - static_cast<int>(below(32)));
    const uint32_t n = below(4) == 0 ? below(5) : below(5000);
    check(s, x, n);
  }
  // ties: x a power of two equal to half an ulp of s, or q + 1/2 ulps
  for (int it = 0; it < 40000; ++it) {
    const int es = 40 + static_cast<int>(below(150));
    const float s = pick(es);
    const int sh = 1 + static_cast<int>(below(24));
    const uint32_t man = (below(2) ? 0u : (static_cast<uint32_t>(next()) & 0x7fffffu)) |
                         (1u << (sh - 1 < 23 ? sh - 1 : 0));
    const float x = bits((static_cast<uint32_t>(es - sh) << 23) | (man & 0x7fffffu));
    check(s, x, below(3000));
  }
  // s just below a binade boundary
  for (int it = 0; it < 40000; ++it) {
    const int es = 40 + static_cast<int>(below(150));
    const float s = bits((static_cast<uint32_t>(es) << 23) | (0x7fffffu - below(64)));
    const float x = pick(es - static_cast<int>(below(26)));
    check(s, x, below(300));
  }
  // whole ternary rows: 40 blocks of 128 weights, f16 scales, the sum of
  // squares run by runs against the element loop
  for (int it = 0; it < 20000; ++it) {
    float s_loop = 0.0f, s_run = 0.0f;
    const uint32_t base = below(31);
    for (int b = 0; b < 40; ++b) {
      uint32_t h = (below(8) == 0 ? below(0x7c00u) : ((base + below(3)) << 10) | below(1024));
      if (((h >> 10) & 0x1f) == 0x1f) h = 0x7bff;
      const float d = half_val(h);
      const float x = d * d;
      uint32_t n = 0;
      for (int j = 0; j < 128; ++j) {
        const int code = static_cast<int>(below(3));
        const volatile float w = static_cast<float>(code - 1) * d;
        const volatile float sq = w * w;
        s_loop = s_loop + sq;
        n += code != 1;
      }
      if (x != 0.0f) {
        const float s_prev = s_run;
        s_run = bh::repeat_add_f32(s_run, x, n);
        float st = s_prev;
        for (uint32_t left = n; left > 0;) left = bh::repeat_add_step_f32(st, x, left);
        if (ubits(st) != ubits(s_run)) {
          if (g_fail < 10) std::printf("ROW STEP MISMATCH %08x %08x\n", ubits(st), ubits(s_run));
          ++g_fail;
        }
      }
    }
    ++g_cases;
    if (ubits(s_loop) != ubits(s_run)) {
      if (g_fail < 10) std::printf("ROW MISMATCH loop %08x runs %08x\n", ubits(s_loop), ubits(s_run));
      ++g_fail;
    }
  }
  // non-finite sums stay non-finite
  check(bits(0x7f800000u), 1.0f, 3);
  check(bits(0x7fc00001u), 1.0f, 3);
  std::printf("%ld cases, %d mismatches\n", g_cases, g_fail);
  return g_fail != 0;
}
