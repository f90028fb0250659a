// Block-level bodies of the NF4 decode (A2/A3), shared by the stand-alone
// dequant kernels of nf4_dequant.hip and the fused preparation launch of the
// QLoRA projection (decode next to the rank-16 products).  Both expect
// blockDim.x = 256.
#pragma once

#include "common.h"

namespace ss {

template <bool NESTED>
__device__ __forceinline__ float block_scale(const uint8_t* __restrict__ qabs,
                                             const float* __restrict__ absmax,
                                             const float* __restrict__ absmax2,
                                             const float* __restrict__ code2, float offset,
                                             int64_t block) {
  if constexpr (NESTED) {
    return nested_scale(qabs, absmax2, code2, offset, block);
  } else {
    return absmax[block];
  }
}

constexpr int kDecodeTLd = 64 + 8;
// LDS of a decode block: the 16-entry code table, then (transposed decode)
// a [64 k][64 + 8 n] fp16 tile.
constexpr int kDecodeSmem = 64 + 64 * kDecodeTLd * 2;

// Block vb of nblocks of the row-major decode: 8 elements (one dword of codes)
// per thread and step, grid-stride over `groups` 8-element groups.  (Four
// groups per thread from one 16-byte load measured slower for the stand-alone
// decode: 14.3 against 10.7 us at 8960 x 1536.)
template <bool NESTED>
__device__ __forceinline__ void decode_vec_block(
    const uint32_t* __restrict__ packed, const uint8_t* __restrict__ qabs,
    const float* __restrict__ absmax, const float* __restrict__ absmax2,
    const float* __restrict__ code2, const float* __restrict__ offset_ptr,
    half8* __restrict__ out, int64_t groups, int64_t vb, int64_t nblocks, unsigned char* smem) {
  float* lut = reinterpret_cast<float*>(smem);
  if (threadIdx.x < 16) lut[threadIdx.x] = kNF4[threadIdx.x];
  __syncthreads();
  const float offset = NESTED ? offset_ptr[0] : 0.0f;
  const int64_t stride = nblocks * blockDim.x;
  for (int64_t g = vb * blockDim.x + threadIdx.x; g < groups; g += stride) {
    const uint32_t word = __builtin_nontemporal_load(packed + g);
    const float scale = block_scale<NESTED>(qabs, absmax, absmax2, code2, offset, g >> 3);
    half8 v;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t byte = (word >> (8 * b)) & 0xffu;
      v[2 * b] = f32_to_f16(lut[byte >> 4] * scale);
      v[2 * b + 1] = f32_to_f16(lut[byte & 15u] * scale);
    }
    out[g] = v;
  }
}

// Tile vb of the transposed decode out[k][n] = W[n][k] (W [rows, cols], cols
// % 64 == 0): a 64 x 64 tile through LDS with padded rows, so both the code
// reads and the fp16 writes are coalesced.
__device__ __forceinline__ void decode_t_block(
    const uint8_t* __restrict__ packed, const uint8_t* __restrict__ qabs,
    const float* __restrict__ absmax2, const float* __restrict__ code2,
    const float* __restrict__ offset_ptr, half_t* __restrict__ out, int64_t rows, int64_t cols,
    int64_t vb, unsigned char* smem) {
  constexpr int LD = kDecodeTLd;
  float* lut = reinterpret_cast<float*>(smem);
  half_t* tile = reinterpret_cast<half_t*>(smem + 64);  // [k][n]
  if (threadIdx.x < 16) lut[threadIdx.x] = kNF4[threadIdx.x];
  __syncthreads();
  const float offset = offset_ptr[0];
  const int64_t ntiles = cdiv(rows, 64);
  const int64_t n0 = (vb % ntiles) * 64;
  const int64_t k0 = (vb / ntiles) * 64;
  const int nl = threadIdx.x & 63;
  const int part = threadIdx.x >> 6;
  const int64_t n = n0 + nl;
  half_t vals[16];
  if (n < rows) {
    const int64_t e = n * cols + k0 + part * 16;
    const uint2 w = *reinterpret_cast<const uint2*>(packed + (e >> 1));
    const float scale = nested_scale(qabs, absmax2, code2, offset, e >> 6);
    const uint32_t words[2] = {w.x, w.y};
#pragma unroll
    for (int wi = 0; wi < 2; ++wi)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t byte = (words[wi] >> (8 * b)) & 0xffu;
        vals[8 * wi + 2 * b] = f32_to_f16(lut[byte >> 4] * scale);
        vals[8 * wi + 2 * b + 1] = f32_to_f16(lut[byte & 15u] * scale);
      }
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) vals[j] = (half_t)0.0f;
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) tile[(part * 16 + j) * LD + nl] = vals[j];
  __syncthreads();
  // 64 k-rows x 8 chunks of 8 n; two chunks per thread.
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int chunk = threadIdx.x + 256 * c;
    const int kr = chunk >> 3;
    const int nc = (chunk & 7) * 8;
    const int64_t k = k0 + kr;
    const int64_t nn = n0 + nc;
    const half8 v = *reinterpret_cast<const half8*>(tile + kr * LD + nc);
    half_t* dst = out + k * rows + nn;
    if (nn + 8 <= rows && rows % 8 == 0) {
      *reinterpret_cast<half8*>(dst) = v;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (nn + j < rows) dst[j] = v[j];
    }
  }
}

constexpr int kDecodeT2Ld = 64 + 8;
// LDS of the wide transposed decode: the code table, then a [128 k][64 + 8 n]
// fp16 tile.
constexpr int kDecodeT2Smem = 64 + 128 * kDecodeT2Ld * 2;

// Tile vb of the transposed decode with 64 n x 128 k tiles (cols % 128 ==
// 0): thread (part = tid / 64, row = tid % 64) decodes 32 consecutive columns
// of one weight row (half a 64-block: one scale) from one 16-byte code load
// and writes them transposed into LDS (the 64 lanes of a wave touch 64
// consecutive halves); the tile leaves as four 16-byte row stores of W^T per
// thread.  Twice the bytes in flight per thread of decode_t_block.
__device__ __forceinline__ void decode_t2_block(
    const uint8_t* __restrict__ packed, const uint8_t* __restrict__ qabs,
    const float* __restrict__ absmax2, const float* __restrict__ code2,
    const float* __restrict__ offset_ptr, half_t* __restrict__ out, int64_t rows, int64_t cols,
    int64_t vb, unsigned char* smem) {
  constexpr int LD = kDecodeT2Ld;
  float* lut = reinterpret_cast<float*>(smem);
  half_t* tile = reinterpret_cast<half_t*>(smem + 64);  // [k][n]
  if (threadIdx.x < 16) lut[threadIdx.x] = kNF4[threadIdx.x];
  __syncthreads();
  const float offset = offset_ptr[0];
  const int64_t ntiles = cdiv(rows, 64);
  const int64_t n0 = (vb % ntiles) * 64;
  const int64_t k0 = (vb / ntiles) * 128;
  const int nl = threadIdx.x & 63;
  const int part = threadIdx.x >> 6;
  const int64_t n = n0 + nl;
  half_t vals[32];
  if (n < rows) {
    const int64_t e = n * cols + k0 + part * 32;
    const u32x4 w = *reinterpret_cast<const u32x4*>(packed + (e >> 1));
    const float scale = nested_scale(qabs, absmax2, code2, offset, e >> 6);
#pragma unroll
    for (int wi = 0; wi < 4; ++wi)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t byte = (w[wi] >> (8 * b)) & 0xffu;
        vals[8 * wi + 2 * b] = f32_to_f16(lut[byte >> 4] * scale);
        vals[8 * wi + 2 * b + 1] = f32_to_f16(lut[byte & 15u] * scale);
      }
  } else {
#pragma unroll
    for (int j = 0; j < 32; ++j) vals[j] = (half_t)0.0f;
  }
#pragma unroll
  for (int j = 0; j < 32; ++j) tile[(part * 32 + j) * LD + nl] = vals[j];
  __syncthreads();
  // 128 k-rows x 8 chunks of 8 n; four chunks per thread.
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int chunk = threadIdx.x + 256 * c;
    const int kr = chunk >> 3;
    const int nc = (chunk & 7) * 8;
    const int64_t k = k0 + kr;
    const int64_t nn = n0 + nc;
    const half8 v = *reinterpret_cast<const half8*>(tile + kr * LD + nc);
    half_t* dst = out + k * rows + nn;
    if (nn + 8 <= rows && rows % 8 == 0) {
      *reinterpret_cast<half8*>(dst) = v;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (nn + j < rows) dst[j] = v[j];
    }
  }
}

}  // namespace ss
