// Block-level bodies of the NF4 decode (A2/A3) of the stand-alone dequant
// kernels (nf4_dequant.hip), which the decode-first GEMM path also launches.
// The transposed tiles expect blockDim.x = 256.
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

// Both NF4 values of a code byte e in one 8-byte LDS read: pair[e] =
// {NF4[e >> 4], NF4[e & 15]}.  Against a 16-entry table this halves the LDS
// reads and drops the nibble split from the decode.
constexpr int kPairBytes = 256 * 8;

__device__ __forceinline__ const float2* load_pairs(unsigned char* smem) {
  float2* pair = reinterpret_cast<float2*>(smem);
  for (int i = threadIdx.x; i < 256; i += blockDim.x) pair[i] = float2{kNF4[i >> 4], kNF4[i & 15]};
  return pair;
}

// v[at + i] = fp16(NF4[c_i] * scale) for the 8 codes c_i of word: element 2j
// is the high nibble of byte j, element 2j + 1 its low nibble.
template <class V>
__device__ __forceinline__ void decode_word(const float2* __restrict__ pair, uint32_t word,
                                            float scale, V& v, int at) {
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const float2 pr = pair[(word >> (8 * b)) & 0xffu];
    v[at + 2 * b] = f32_to_f16(pr.x * scale);
    v[at + 2 * b + 1] = f32_to_f16(pr.y * scale);
  }
}

constexpr int kDecodeTLd = 64 + 8;
// LDS of a decode block: the code-pair table, then (transposed decode) a
// [64 k][64 + 8 n] fp16 tile.
constexpr int kDecodeSmem = kPairBytes + 64 * kDecodeTLd * 2;

// Row-major decode: 8 elements (one dword of codes) per lane and group.  A
// wave covers U * 64 consecutive groups per step -- U coalesced dword loads
// per lane (with their qabs / absmax2 loads) issued before any arithmetic,
// then U 16-byte stores, each wave-wide store 1 KiB contiguous -- and the
// waves of the grid stride over the groups.  The code-pair table and the
// 256-entry code2 table sit in LDS, so the scale costs no dependent global
// load.  U = 8 keeps 2 KiB of codes in flight per wave (large weights), U = 2
// gives more waves to small ones (measured on MI355X: 18944 x 3584 in 32.3 us,
// 5.3 TB/s, against 42.4 us with one group per lane and step).
constexpr int kDecodeRowsSmem = kPairBytes + 256 * 4;

template <bool NESTED, int U>
__device__ __forceinline__ void decode_rows_block(
    const uint32_t* __restrict__ packed, const uint8_t* __restrict__ qabs,
    const float* __restrict__ absmax, const float* __restrict__ absmax2,
    const float* __restrict__ code2, const float* __restrict__ offset_ptr,
    half8* __restrict__ out, int64_t groups, int64_t vb, int64_t nblocks, unsigned char* smem) {
  const float2* pair = load_pairs(smem);
  float* c2 = reinterpret_cast<float*>(smem + kPairBytes);
  if constexpr (NESTED)
    for (int i = threadIdx.x; i < 256; i += blockDim.x) c2[i] = code2[i];
  __syncthreads();
  const float offset = NESTED ? offset_ptr[0] : 0.0f;
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t waves_per_block = blockDim.x / kWave;
  const int64_t wave = vb * waves_per_block + threadIdx.x / kWave;
  const int64_t step = nblocks * waves_per_block * (U * kWave);
  for (int64_t base = wave * (U * kWave); base < groups; base += step) {
    uint32_t word[U], q[U];
    float am[U];  // absmax2 (nested) or the block's absmax (flat)
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int64_t g = base + j * kWave + lane;
      const int64_t gs = g < groups ? g : 0;  // clamped, never stored
      word[j] = __builtin_nontemporal_load(packed + gs);
      if constexpr (NESTED) {
        q[j] = qabs[gs >> 3];
        am[j] = absmax2[gs >> 11];
      } else {
        q[j] = 0;
        am[j] = absmax[gs >> 3];
      }
    }
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int64_t g = base + j * kWave + lane;
      float scale = am[j];
      if constexpr (NESTED) {
        // fp32(fp32(code2[q] * absmax2) + offset), two roundings.
        const float product = c2[q[j]] * am[j];
        scale = product + offset;
      }
      half8 v;
      decode_word(pair, word[j], scale, v, 0);
      if (g < groups) out[g] = v;
    }
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
  const float2* pair = load_pairs(smem);
  half_t* tile = reinterpret_cast<half_t*>(smem + kPairBytes);  // [k][n]
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
      decode_word(pair, words[wi], scale, vals, 8 * wi);
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
// LDS of the wide transposed decode: the code-pair table, then a
// [128 k][64 + 8 n] fp16 tile.
constexpr int kDecodeT2Smem = kPairBytes + 128 * kDecodeT2Ld * 2;

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
  const float2* pair = load_pairs(smem);
  half_t* tile = reinterpret_cast<half_t*>(smem + kPairBytes);  // [k][n]
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
      decode_word(pair, w[wi], scale, vals, 8 * wi);
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
