// Standalone NF4 decode (nested A2 and flat A3), bit-exact.
//
// Reference: solution/kernels/nf4.py:41-59 (nf4_decode_kernel), formula at
// :7-10.  HBM-bound: 0.5 B read + 2 B written per element (+1/64 B qabs).
//
// Vector path (decode_rows_block): each lane decodes 8 consecutive elements
// per group -- one packed dword (4 bytes) in, one 16-byte fp16 store out --
// with U groups per lane in flight, so a wave moves U x 256 B of nibbles and
// writes 1 KiB contiguous per store.  The NF4 and code2 tables sit in LDS.
// 8 consecutive elements always share one 64-block (8 divides 64), so each
// group needs a single scale.
// Generic path: one element per lane, any alignment / tail.

#include "decode_blocks.h"

namespace ss {

template <bool NESTED, int U>
__global__ __launch_bounds__(256) void nf4_dequant_vec_kernel(
    const uint32_t* __restrict__ packed, const uint8_t* __restrict__ qabs,
    const float* __restrict__ absmax, const float* __restrict__ absmax2,
    const float* __restrict__ code2, const float* __restrict__ offset_ptr,
    half8* __restrict__ out, int64_t groups) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[kDecodeRowsSmem];
  decode_rows_block<NESTED, U>(packed, qabs, absmax, absmax2, code2, offset_ptr, out, groups,
                               blockIdx.x, gridDim.x, smem);
}

template <bool NESTED>
__global__ __launch_bounds__(256) void nf4_dequant_scalar_kernel(
    const uint8_t* __restrict__ packed, const uint8_t* __restrict__ qabs,
    const float* __restrict__ absmax, const float* __restrict__ absmax2,
    const float* __restrict__ code2, const float* __restrict__ offset_ptr,
    half_t* __restrict__ out, int64_t begin, int64_t n) {
  const float offset = NESTED ? offset_ptr[0] : 0.0f;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = begin + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint32_t byte = packed[i >> 1];
    const uint32_t nib = (i & 1) ? (byte & 15u) : (byte >> 4);
    const float scale = block_scale<NESTED>(qabs, absmax, absmax2, code2, offset, i >> 6);
    out[i] = f32_to_f16(kNF4[nib] * scale);
  }
}

// Transposed decode: out[k][n] = Wdec[n][k] for W [rows, cols] with cols % 64
// == 0, so that the backward GEMM dX = dY . W reads W^T with k contiguous.
// One 256-thread workgroup per 64 x 64 tile (WIDE: 64 x 128 tiles, 32
// columns per thread from one 16-byte code load, decode_t2_block): thread
// (part = tid / 64, row = tid % 64) decodes consecutive columns of one weight
// row (one scale) and writes them transposed into LDS, where the 64 lanes of a
// wave touch 64 consecutive halves; the tile then leaves as 16-byte row
// stores of W^T.
template <bool WIDE>
__global__ __launch_bounds__(256) void nf4_dequant_t_kernel(
    const uint8_t* __restrict__ packed, const uint8_t* __restrict__ qabs,
    const float* __restrict__ absmax2, const float* __restrict__ code2,
    const float* __restrict__ offset_ptr, half_t* __restrict__ out, int64_t rows, int64_t cols) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[WIDE ? kDecodeT2Smem : kDecodeSmem];
  if constexpr (WIDE)
    decode_t2_block(packed, qabs, absmax2, code2, offset_ptr, out, rows, cols, blockIdx.x, smem);
  else
    decode_t_block(packed, qabs, absmax2, code2, offset_ptr, out, rows, cols, blockIdx.x, smem);
}

static int grid_for(int64_t work, int threads) {
  // Enough waves to cover every CU several times; the loops are grid-stride.
  int64_t blocks = cdiv(work, threads);
  const int64_t cap = 256 * 32;
  return (int)(blocks < cap ? (blocks > 0 ? blocks : 1) : cap);
}

template <bool NESTED>
static int launch_dequant(const uint8_t* packed, const uint8_t* qabs, const float* absmax,
                          const float* absmax2, const float* code2, const float* offset,
                          uint16_t* out, int64_t n, hipStream_t stream) {
  if (n == 0) return SS_OK;
  half_t* o = reinterpret_cast<half_t*>(out);
  const bool aligned = (reinterpret_cast<uintptr_t>(packed) % 4 == 0) &&
                       (reinterpret_cast<uintptr_t>(out) % 16 == 0);
  int64_t done = 0;
  if (aligned) {
    const int64_t groups = n / 8;
    if (groups > 0) {
      // 8 groups per lane and step from 2^20 groups (8M elements) on, else 2;
      // at most 4096 workgroups, grid-stride beyond.
      const bool wide = groups >= ((int64_t)1 << 20);
      const int64_t per_block = (wide ? 8 : 2) * 256;
      const int64_t blocks = cdiv(groups, per_block) < 4096 ? cdiv(groups, per_block) : 4096;
      auto kern = wide ? nf4_dequant_vec_kernel<NESTED, 8> : nf4_dequant_vec_kernel<NESTED, 2>;
      hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, stream,
                         reinterpret_cast<const uint32_t*>(packed), qabs, absmax, absmax2, code2,
                         offset, reinterpret_cast<half8*>(o), groups);
      SS_CHECK_LAUNCH("nf4_dequant_vec_kernel");
    }
    done = groups * 8;
  }
  if (done < n) {
    hipLaunchKernelGGL(nf4_dequant_scalar_kernel<NESTED>, dim3(grid_for(n - done, 256)), dim3(256),
                       0, stream, packed, qabs, absmax, absmax2, code2, offset, o, done, n);
    SS_CHECK_LAUNCH("nf4_dequant_scalar_kernel");
  }
  return SS_OK;
}

}  // namespace ss

extern "C" int ss_nf4_dequant_nested(const uint8_t* packed, const uint8_t* qabs,
                                     const float* absmax2, const float* code2,
                                     const float* offset, uint16_t* out, int64_t n,
                                     void* stream) {
  SS_CHECK_ARG(n >= 0, "ss_nf4_dequant_nested: n=%lld must be >= 0", (long long)n);
  if (n == 0) return SS_OK;
  SS_CHECK_ARG(packed && qabs && absmax2 && code2 && offset && out,
               "ss_nf4_dequant_nested: null pointer");
  return ss::launch_dequant<true>(packed, qabs, nullptr, absmax2, code2, offset, out, n,
                                  (hipStream_t)stream);
}

extern "C" int ss_nf4_dequant_nested_t(const uint8_t* packed, const uint8_t* qabs,
                                       const float* absmax2, const float* code2,
                                       const float* offset, uint16_t* out, int64_t rows,
                                       int64_t cols, void* stream) {
  const char* fn = "ss_nf4_dequant_nested_t";
  SS_CHECK_ARG(rows >= 0 && cols >= 0, "%s: negative size", fn);
  if (rows == 0 || cols == 0) return SS_OK;
  SS_CHECK_ARG(packed && qabs && absmax2 && code2 && offset && out, "%s: null pointer", fn);
  if (cols % 64 != 0 || reinterpret_cast<uintptr_t>(packed) % 8 != 0 ||
      reinterpret_cast<uintptr_t>(out) % 16 != 0) {
    ss::set_error("%s: needs cols %% 64 == 0, 8-byte aligned packed and 16-byte aligned out", fn);
    return SS_ERR_UNSUPPORTED;
  }
  // 64 x 128 tiles (16-byte code loads) when the columns allow, else 64 x 64.
  const bool wide = cols % 128 == 0 && reinterpret_cast<uintptr_t>(packed) % 16 == 0;
  const int64_t tiles = ss::cdiv(rows, 64) * (wide ? cols / 128 : cols / 64);
  hipLaunchKernelGGL(wide ? ss::nf4_dequant_t_kernel<true> : ss::nf4_dequant_t_kernel<false>,
                     dim3((unsigned)tiles), dim3(256), 0, (hipStream_t)stream, packed, qabs,
                     absmax2, code2, offset, reinterpret_cast<ss::half_t*>(out), rows, cols);
  SS_CHECK_LAUNCH("nf4_dequant_t_kernel");
  return SS_OK;
}

extern "C" int ss_nf4_dequant_flat(const uint8_t* packed, const float* absmax, uint16_t* out,
                                   int64_t n, void* stream) {
  SS_CHECK_ARG(n >= 0, "ss_nf4_dequant_flat: n=%lld must be >= 0", (long long)n);
  if (n == 0) return SS_OK;
  SS_CHECK_ARG(packed && absmax && out, "ss_nf4_dequant_flat: null pointer");
  return ss::launch_dequant<false>(packed, nullptr, absmax, nullptr, nullptr, nullptr, out, n,
                                   (hipStream_t)stream);
}
