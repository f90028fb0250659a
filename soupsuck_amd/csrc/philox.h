// Counter-based random bits for the LoRA dropout mask: Philox4x32-10
// (J. K. Salmon, M. A. Moraes, R. O. Dror, D. E. Shaw, "Parallel random
// numbers: as easy as 1, 2, 3", SC'11; round multipliers 0xD2511F53 /
// 0xCD9E8D57 and key increments 0x9E3779B9 / 0xBB67AE85 from that paper).
//
// Mask of an activation X [rows, cols] (row-major element e = row * cols +
// col) for a call with 64-bit seed s and drop probability p:
//   key = (s mod 2^32, s / 2^32); counter = (e / 4 mod 2^32, e / 4 / 2^32, 0, 0);
//   u   = word (e mod 4) of Philox4x32-10(counter, key);
//   keep(e) = u < thr,  thr = floor((1 - p) * 2^32);
//   dropped X = keep ? fp32(x) * inv : 0,  inv = fp32(1 / (1 - p)).
// A kernel regenerates any element's bit from (s, e) alone, so the mask is
// never stored: the forward's Z, the backward's dA and the dX update each
// recompute the bits of the elements they touch.  oracle/philox.py restates
// the same definition.
#pragma once

#include "common.h"

namespace ss {

struct DropoutArgs {
  uint64_t seed;
  uint32_t thr;
  float inv;
  int on;
};

__device__ __forceinline__ u32x4 philox4x32_10(u32x4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    const uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
    c = u32x4{(uint32_t)(p1 >> 32) ^ c[1] ^ k0, (uint32_t)p1, (uint32_t)(p0 >> 32) ^ c[3] ^ k1,
              (uint32_t)p0};
  }
  return c;
}

// Keep bits (bit j = element e4 * 4 + j) of the aligned group of four
// elements starting at element 4 * e4.
__device__ __forceinline__ uint32_t keep4(const DropoutArgs& d, uint64_t e4) {
  const u32x4 u = philox4x32_10(u32x4{(uint32_t)e4, (uint32_t)(e4 >> 32), 0u, 0u},
                                (uint32_t)d.seed, (uint32_t)(d.seed >> 32));
  return (uint32_t)(u[0] < d.thr) | ((uint32_t)(u[1] < d.thr) << 1) |
         ((uint32_t)(u[2] < d.thr) << 2) | ((uint32_t)(u[3] < d.thr) << 3);
}

// Keep bits of the 8 consecutive elements e .. e + 7 (e % 4 == 0).
__device__ __forceinline__ uint32_t keep8(const DropoutArgs& d, uint64_t e) {
  return keep4(d, e >> 2) | (keep4(d, (e >> 2) + 1) << 4);
}

// fp32 value of dropped X for one element.
__device__ __forceinline__ float dropped(const DropoutArgs& d, float x, bool keep) {
  return keep ? x * d.inv : 0.0f;
}

}  // namespace ss
