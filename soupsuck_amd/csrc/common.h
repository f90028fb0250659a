// Shared definitions for the soupsuck_amd HIP kernels (gfx950 / CDNA4).
//
// Every kernel in this library is written for 64-wide wavefronts.  All
// sources are compiled with -ffp-contract=off so that a*b+c stays two
// roundings wherever the reference disables fusion (enable_fp_fusion=False
// on every reference launch), and fp32 -> fp16 conversions are the hardware
// round-to-nearest-even v_cvt_f16_f32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/soupsuck_amd.h"

namespace ss {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float2v __attribute__((ext_vector_type(2)));
// Native 128-bit vector (HIP's uint4 is a class type; selects and copies of it
// can be lowered through memory, so register staging uses this type).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// Sixteen NF4 code points (format data: reference solution/kernels/nf4.py:32-37).
#define SS_NF4_CODE_POINTS                                                                  \
  -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,                \
      -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,           \
      0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f, \
      0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f
__device__ __constant__ static const float kNF4[16] = {SS_NF4_CODE_POINTS};

// fp16(code point) bit patterns (round to nearest even), computed at compile
// time, for decoders that build their tables without a memory load.
struct Nf4HalfBits {
  uint16_t v[16];
};
constexpr Nf4HalfBits nf4_half_bits() {
  constexpr float codes[16] = {SS_NF4_CODE_POINTS};
  Nf4HalfBits h{};
  for (int i = 0; i < 16; ++i) h.v[i] = __builtin_bit_cast(uint16_t, (_Float16)codes[i]);
  return h;
}
constexpr Nf4HalfBits kNF4Half = nf4_half_bits();
// kNF4Half.v[i] for a run-time i, without a memory access (selects).
__device__ __forceinline__ uint32_t nf4_half_bits_of(int i) {
  uint32_t r = 0;
#pragma unroll
  for (int q = 0; q < 16; ++q) r = i == q ? kNF4Half.v[q] : r;
  return r;
}

// fp32 -> fp16 with round-to-nearest-even as its own instruction.  The empty
// asm makes the value opaque to instruction selection, which would otherwise
// fold a preceding fp32 multiply into v_fma_mix*_f16 with a +0 addend: that
// turns a -0 product into +0 and rounds the exact product once instead of
// rounding it to fp32 first.  It emits no instruction.
__device__ __forceinline__ half_t f32_to_f16(float v) {
  asm("" : "+v"(v));
  return (half_t)v;
}

// fp32 scale of one 64-element NF4 block of a nested (double-quantized) state:
// fp32(fp32(code2[qabs[b]] * absmax2[b / 256]) + offset).  Two separate
// roundings; the translation unit is built without contraction.
__device__ __forceinline__ float nested_scale(const uint8_t* __restrict__ qabs,
                                              const float* __restrict__ absmax2,
                                              const float* __restrict__ code2,
                                              float offset, int64_t block) {
  const float code = code2[qabs[block]];
  const float product = code * absmax2[block >> 8];
  return product + offset;
}

__host__ __device__ constexpr int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Compute units of the current device, queried once per device (256 when the
// query fails).  Concurrent first calls store the same value.
inline int device_cu_count() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int v = 0;
    const bool ok =
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess;
    cus[dev] = ok && v > 0 ? v : 256;
  }
  return cus[dev];
}

// Thread-local last-error text for the C ABI.
void set_error(const char* fmt, ...);

}  // namespace ss

#define SS_CHECK_ARG(cond, ...)          \
  do {                                   \
    if (!(cond)) {                       \
      ss::set_error(__VA_ARGS__);        \
      return SS_ERR_INVALID_ARGUMENT;    \
    }                                    \
  } while (0)

#define SS_CHECK_LAUNCH(name)                                               \
  do {                                                                      \
    hipError_t _e = hipGetLastError();                                      \
    if (_e != hipSuccess) {                                                 \
      ss::set_error("%s launch failed: %s", name, hipGetErrorString(_e));   \
      return SS_ERR_LAUNCH;                                                 \
    }                                                                       \
  } while (0)
