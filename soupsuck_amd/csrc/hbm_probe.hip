// HBM read ceiling probe (measurement only, no counterpart in the reference):
// the time a plain streaming read of `bytes` takes on this GPU, the yardstick
// for the weight-streaming NF4 kernels at small T, whose HBM roofline assumes
// the nominal 8 TB/s.  Each workgroup of 256 threads reads 4 KiB chunks
// (16-byte loads, four in flight per thread) grid-stride and folds them with
// XOR into one word per workgroup, so the loads cannot be elided; the words go
// to `sink` (one per workgroup).

#include "common.h"

namespace ss {

__global__ __launch_bounds__(256) void hbm_read_probe_kernel(const u32x4* __restrict__ src,
                                                             int64_t vecs,
                                                             uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  const int64_t stride = (int64_t)gridDim.x * 256 * 4;
  for (int64_t base = (int64_t)blockIdx.x * 256 * 4 + threadIdx.x; base < vecs; base += stride) {
    u32x4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t i = base + 256 * j;
      v[j] = i < vecs ? __builtin_nontemporal_load(src + i) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) acc ^= v[j][0] ^ v[j][1] ^ v[j][2] ^ v[j][3];
  }
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] ^= red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) sink[blockIdx.x] = red[0];
}

}  // namespace ss

extern "C" int ss_hbm_read_probe(const void* src, int64_t bytes, int64_t blocks, uint32_t* sink,
                                 void* stream) {
  const char* fn = "ss_hbm_read_probe";
  SS_CHECK_ARG(bytes >= 0 && blocks >= 1 && blocks <= (1 << 20), "%s: bad size", fn);
  if (bytes == 0) return SS_OK;
  SS_CHECK_ARG(src && sink, "%s: null pointer", fn);
  SS_CHECK_ARG(bytes % 16 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0,
               "%s: bytes and src must be 16-byte multiples", fn);
  hipLaunchKernelGGL(ss::hbm_read_probe_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, reinterpret_cast<const ss::u32x4*>(src), bytes / 16,
                     sink);
  SS_CHECK_LAUNCH("hbm_read_probe_kernel");
  return SS_OK;
}
