// fp16 2-D transpose, dst[c][r] = src[r][c] (rows x cols of src), through
// 64 x 64 LDS tiles so that both the reads and the writes are coalesced
// 16-byte accesses.  Used by the fused cross-entropy backward to present the
// vocabulary-chunk products to the dense NT MFMA kernel (both operands
// contiguous along the reduced dimension).

#include "common.h"

namespace ss {
namespace {

constexpr int kTT = 64;
constexpr int kTLd = kTT + 8;  // LDS row pitch (halves): 144 B rows keep column reads spread

// One 64 x 64 tile per workgroup of 256 threads: each thread reads two
// 8-element row chunks, writes them to LDS, and after the barrier writes two
// 8-element chunks of the transposed tile.  VEC: rows of src and dst start
// 16-byte aligned, so every chunk lying wholly inside the matrix is one
// 16-byte access; chunks at a ragged edge go element by element.
template <bool VEC>
__global__ __launch_bounds__(256) void transpose_f16_kernel(const half_t* __restrict__ src,
                                                            int64_t lds, int64_t rows,
                                                            int64_t cols,
                                                            half_t* __restrict__ dst,
                                                            int64_t ldd) {
  __shared__ half_t tile[kTT * kTLd];
  const int64_t ctiles = cdiv(cols, kTT);
  const int64_t r0 = (blockIdx.x / ctiles) * kTT;
  const int64_t c0 = (blockIdx.x % ctiles) * kTT;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int chunk = threadIdx.x + 256 * h;  // 64 rows x 8 chunks
    const int rr = chunk >> 3;
    const int cc = (chunk & 7) * 8;
    const int64_t r = r0 + rr;
    half8 v = half8{};
    if (VEC && r < rows && c0 + cc + 8 <= cols) {
      v = *reinterpret_cast<const half8*>(src + r * lds + c0 + cc);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (r < rows && c0 + cc + e < cols) v[e] = src[r * lds + c0 + cc + e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[(cc + e) * kTLd + rr] = v[e];
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int chunk = threadIdx.x + 256 * h;  // 64 dst rows (src cols) x 8 chunks
    const int cr = chunk >> 3;
    const int rc = (chunk & 7) * 8;
    const int64_t c = c0 + cr;
    if (c >= cols) continue;
    const half8 v = *reinterpret_cast<const half8*>(&tile[cr * kTLd + rc]);
    if (VEC && r0 + rc + 8 <= rows) {
      *reinterpret_cast<half8*>(dst + c * ldd + r0 + rc) = v;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (r0 + rc + e < rows) dst[c * ldd + r0 + rc + e] = v[e];
    }
  }
}

}  // namespace
}  // namespace ss

using namespace ss;

extern "C" int ss_transpose_f16(const uint16_t* src, int64_t lds, int64_t rows, int64_t cols,
                                uint16_t* dst, int64_t ldd, void* stream) {
  const char* fn = "ss_transpose_f16";
  SS_CHECK_ARG(rows >= 0 && cols >= 0, "%s: negative size", fn);
  if (rows == 0 || cols == 0) return SS_OK;
  SS_CHECK_ARG(src && dst, "%s: null pointer", fn);
  SS_CHECK_ARG(lds >= cols && ldd >= rows, "%s: leading dimension too small", fn);
  const bool vec = reinterpret_cast<uintptr_t>(src) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(dst) % 16 == 0 && lds % 8 == 0 && ldd % 8 == 0;
  const int64_t tiles = cdiv(rows, kTT) * cdiv(cols, kTT);
  auto kern = vec ? transpose_f16_kernel<true> : transpose_f16_kernel<false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<const half_t*>(src), lds, rows, cols,
                     reinterpret_cast<half_t*>(dst), ldd);
  SS_CHECK_LAUNCH("transpose_f16_kernel");
  return SS_OK;
}
