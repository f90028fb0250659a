// Typed element access for kernels whose tensors may be fp16 or fp32.
#pragma once

#include "common.h"

namespace ss {

__device__ __forceinline__ float ld_elem(const void* p, int dt, int64_t i) {
  return dt == SS_F16 ? (float)reinterpret_cast<const half_t*>(p)[i]
                      : reinterpret_cast<const float*>(p)[i];
}

__device__ __forceinline__ void st_elem(void* p, int dt, int64_t i, float v) {
  if (dt == SS_F16)
    reinterpret_cast<half_t*>(p)[i] = f32_to_f16(v);
  else
    reinterpret_cast<float*>(p)[i] = v;
}

// Round an fp32 value to the storage precision of dtype dt (identity for fp32).
__device__ __forceinline__ float round_to(int dt, float v) {
  return dt == SS_F16 ? (float)f32_to_f16(v) : v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}

inline bool valid_dtype(int dt) { return dt == SS_F16 || dt == SS_F32; }

inline int promote(int a, int b) { return (a == SS_F32 || b == SS_F32) ? SS_F32 : SS_F16; }

}  // namespace ss
