// Planar-quantized KV cache: the fixed tables shared by the store kernel
// (kvquant.hip) and the attention kernels (attention.hip).
//
// Reference: src/kvquant.rs (PlanarQuant; BONSAI_KV=planarN / planarNk).  A
// kv-head vector x of hd = 256 floats is stored as its norm n = |x| (f32,
// the squares summed in index order) and, for the rotated unit vector
// R (x / n) -- every pair (2i, 2i+1) turned by a fixed Givens angle
// (c_i, s_i) -- the index of the nearest of 2^bits Lloyd-Max centroids per
// coordinate, packed LSB first at `bits` bits each (32 * bits bytes).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>

namespace bh {

constexpr int kPlanarHd = 256;  // head size of the planar kernels (the model's)

// Passed to the kernels by value (2 KB of kernel arguments): no device
// allocation, nothing to keep alive across graph replays.
struct PlanarTables {
  float cent[256];  // 2^bits centroids, ascending (the rest unused)
  float gc[kPlanarHd / 2];
  float gs[kPlanarHd / 2];
};

// The tables of (hd, bits), computed once per pair on the host (thread-safe).
// False for hd != 256 or bits outside 1..8.
bool planar_tables(size_t hd, unsigned bits, PlanarTables *out);

inline size_t planar_packed_len(size_t hd, unsigned bits) {
  return ((hd + 1) / 2 * 2 * bits + 7) / 8;
}

}  // namespace bh
