// Right-padding removal: packed gather and zero-filling scatter (A16).
//
// Reference: solution/unpad.py:149-161 (_pack = index_select of rows,
// _scatter = zeros + index_copy) and :184-199 (row-major indices).  Pure
// row copies, bit-exact, HBM-bound: gather moves 2 * T * row_bytes, scatter
// writes B*S*row_bytes and reads T*row_bytes.  Each lane copies 16 B
// (vector path) so one wave moves 1 KiB contiguous per access.

#include "common.h"

namespace ss {

template <typename V>
__global__ __launch_bounds__(256) void gather_kernel(const V* __restrict__ src, V* __restrict__ dst,
                                                     const int64_t* __restrict__ indices,
                                                     int64_t tokens, int64_t row_vecs,
                                                     int64_t src_rows) {
  const int64_t total = tokens * row_vecs;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t t = i / row_vecs;
    const int64_t v = i - t * row_vecs;
    const int64_t r = indices[t];
    // An index outside the source (never produced by the length-derived
    // indices) yields a zero row instead of an out-of-bounds read.
    dst[i] = (r >= 0 && r < src_rows) ? src[r * row_vecs + v] : V{};
  }
}

template <typename V>
__global__ __launch_bounds__(256) void scatter_kernel(const V* __restrict__ src, V* __restrict__ dst,
                                                      const int32_t* __restrict__ inverse,
                                                      int64_t rows, int64_t row_vecs,
                                                      int64_t tokens) {
  const int64_t total = rows * row_vecs;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / row_vecs;
    const int64_t v = i - r * row_vecs;
    const int32_t j = inverse[r];
    V out;
    if (j >= 0 && j < tokens) {
      out = src[(int64_t)j * row_vecs + v];
    } else {
      out = V{};
    }
    dst[i] = out;
  }
}

__global__ __launch_bounds__(256) void fill_kernel(int32_t* __restrict__ p, int64_t n, int32_t v) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

__global__ __launch_bounds__(256) void invert_kernel(const int64_t* __restrict__ indices,
                                                     int64_t tokens, int32_t* __restrict__ inverse,
                                                     int64_t rows) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < tokens; t += stride) {
    const int64_t r = indices[t];
    if (r >= 0 && r < rows) inverse[r] = (int32_t)t;
  }
}

static unsigned grid_for(int64_t work) {
  const int64_t blocks = cdiv(work, 256);
  return (unsigned)(blocks < 16384 ? (blocks > 0 ? blocks : 1) : 16384);
}

static bool al(const void* p, int a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

}  // namespace ss

using namespace ss;

extern "C" int ss_unpad_gather(const void* padded, int64_t padded_rows, void* packed,
                               const int64_t* indices, int64_t tokens, int64_t row_bytes,
                               void* stream) {
  SS_CHECK_ARG(tokens >= 0 && row_bytes >= 0, "ss_unpad_gather: negative size");
  SS_CHECK_ARG(row_bytes % 2 == 0, "ss_unpad_gather: row_bytes must be even");
  if (tokens == 0 || row_bytes == 0) return SS_OK;
  SS_CHECK_ARG(padded && packed && indices, "ss_unpad_gather: null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (row_bytes % 16 == 0 && al(padded, 16) && al(packed, 16)) {
    const int64_t rv = row_bytes / 16;
    hipLaunchKernelGGL(gather_kernel<uint4>, dim3(grid_for(tokens * rv)), dim3(256), 0, s,
                       (const uint4*)padded, (uint4*)packed, indices, tokens, rv, padded_rows);
  } else {
    const int64_t rv = row_bytes / 2;
    hipLaunchKernelGGL(gather_kernel<uint16_t>, dim3(grid_for(tokens * rv)), dim3(256), 0, s,
                       (const uint16_t*)padded, (uint16_t*)packed, indices, tokens, rv,
                       padded_rows);
  }
  SS_CHECK_LAUNCH("gather_kernel");
  return SS_OK;
}

extern "C" int ss_unpad_inverse(const int64_t* indices, int64_t tokens, int32_t* inverse,
                                int64_t rows, void* stream) {
  SS_CHECK_ARG(tokens >= 0 && rows >= 0 && tokens <= rows, "ss_unpad_inverse: bad sizes");
  SS_CHECK_ARG(rows < 2147483647LL, "ss_unpad_inverse: rows must fit int32");
  if (rows == 0) return SS_OK;
  SS_CHECK_ARG(inverse && (tokens == 0 || indices), "ss_unpad_inverse: null pointer");
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(fill_kernel, dim3(grid_for(rows)), dim3(256), 0, s, inverse, rows, -1);
  SS_CHECK_LAUNCH("fill_kernel");
  if (tokens > 0) {
    hipLaunchKernelGGL(invert_kernel, dim3(grid_for(tokens)), dim3(256), 0, s, indices, tokens,
                       inverse, rows);
    SS_CHECK_LAUNCH("invert_kernel");
  }
  return SS_OK;
}

extern "C" int ss_unpad_scatter(const void* packed, int64_t tokens, void* padded,
                                const int32_t* inverse, int64_t rows, int64_t row_bytes,
                                void* stream) {
  SS_CHECK_ARG(rows >= 0 && row_bytes >= 0, "ss_unpad_scatter: negative size");
  SS_CHECK_ARG(row_bytes % 2 == 0, "ss_unpad_scatter: row_bytes must be even");
  if (rows == 0 || row_bytes == 0) return SS_OK;
  SS_CHECK_ARG(tokens >= 0, "ss_unpad_scatter: negative tokens");
  SS_CHECK_ARG(padded && inverse && (tokens == 0 || packed), "ss_unpad_scatter: null pointer");
  hipStream_t s = (hipStream_t)stream;
  if (row_bytes % 16 == 0 && al(padded, 16) && (packed == nullptr || al(packed, 16))) {
    const int64_t rv = row_bytes / 16;
    hipLaunchKernelGGL(scatter_kernel<uint4>, dim3(grid_for(rows * rv)), dim3(256), 0, s,
                       (const uint4*)packed, (uint4*)padded, inverse, rows, rv, tokens);
  } else {
    const int64_t rv = row_bytes / 2;
    hipLaunchKernelGGL(scatter_kernel<uint16_t>, dim3(grid_for(rows * rv)), dim3(256), 0, s,
                       (const uint16_t*)packed, (uint16_t*)padded, inverse, rows, rv, tokens);
  }
  SS_CHECK_LAUNCH("scatter_kernel");
  return SS_OK;
}
