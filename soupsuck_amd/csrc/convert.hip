// Lossless fp32 -> fp16 storage conversion of a frozen table (the tied
// embedding / lm_head of Qwen2), with the exactness check in the same pass.
//
// Reference: solution/embedding.py:51-64 (_lossless_candidate: copy each
// 32 MiB chunk to fp16 and require torch.equal(half.float(), fp32) for every
// element, else refuse).  Here one HBM pass reads the fp32 table (4 B per
// element), writes the fp16 candidate (2 B) and raises a device flag if any
// element does not round-trip exactly (a NaN never does: NaN != NaN, as in
// torch.equal).  The caller reads the flag once; the candidate is the
// eventual storage, so no chunked fp32 scratch exists.  HBM-bound: 6 B per
// element, 1.40 GB for the 151936 x 1536 Qwen2.5-1.5B table.

#include "common.h"

namespace ss {
namespace {

__device__ __forceinline__ bool exact(float v, half_t h) { return (float)h == v; }

// Vector path: 8 elements per lane and step (two 16-byte loads, one 16-byte
// store), grid-stride.  A lane that sees an inexact element stores 1 to the
// flag with an ordinary vector store; every writer writes the same value.
__global__ __launch_bounds__(256) void f32_to_f16_exact_vec(const float4v* __restrict__ src,
                                                            half8* __restrict__ dst,
                                                            int64_t groups,
                                                            int* __restrict__ flag) {
  bool bad = false;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups; g += stride) {
    const float4v a = __builtin_nontemporal_load(src + 2 * g);
    const float4v b = __builtin_nontemporal_load(src + 2 * g + 1);
    half8 h;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      h[i] = f32_to_f16(a[i]);
      h[4 + i] = f32_to_f16(b[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) bad |= !exact(a[i], h[i]) || !exact(b[i], h[4 + i]);
    dst[g] = h;
  }
  if (bad) flag[0] = 1;
}

__global__ __launch_bounds__(256) void f32_to_f16_exact_scalar(const float* __restrict__ src,
                                                               half_t* __restrict__ dst,
                                                               int64_t begin, int64_t n,
                                                               int* __restrict__ flag) {
  bool bad = false;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = begin + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float v = src[i];
    const half_t h = f32_to_f16(v);
    bad |= !exact(v, h);
    dst[i] = h;
  }
  if (bad) flag[0] = 1;
}

int grid_blocks(int64_t work) {
  const int64_t blocks = cdiv(work, 256);
  const int64_t cap = 256 * 16;
  return (int)(blocks < 1 ? 1 : (blocks < cap ? blocks : cap));
}

}  // namespace
}  // namespace ss

extern "C" int ss_f32_to_f16_exact(const float* src, uint16_t* dst, int64_t n, int* flag,
                                   void* stream) {
  const char* fn = "ss_f32_to_f16_exact";
  SS_CHECK_ARG(n >= 0, "%s: n=%lld must be >= 0", fn, (long long)n);
  if (n == 0) return SS_OK;
  SS_CHECK_ARG(src && dst && flag, "%s: null pointer", fn);
  hipStream_t s = (hipStream_t)stream;
  auto* out = reinterpret_cast<ss::half_t*>(dst);
  int64_t done = 0;
  if (reinterpret_cast<uintptr_t>(src) % 16 == 0 && reinterpret_cast<uintptr_t>(dst) % 16 == 0) {
    const int64_t groups = n / 8;
    if (groups > 0) {
      hipLaunchKernelGGL(ss::f32_to_f16_exact_vec, dim3(ss::grid_blocks(groups)), dim3(256), 0, s,
                         reinterpret_cast<const ss::float4v*>(src),
                         reinterpret_cast<ss::half8*>(out), groups, flag);
      SS_CHECK_LAUNCH("f32_to_f16_exact_vec");
    }
    done = groups * 8;
  }
  if (done < n) {
    hipLaunchKernelGGL(ss::f32_to_f16_exact_scalar, dim3(ss::grid_blocks(n - done)), dim3(256), 0,
                       s, src, out, done, n, flag);
    SS_CHECK_LAUNCH("f32_to_f16_exact_scalar");
  }
  return SS_OK;
}
