// SwiGLU activation of a Qwen2 MLP, forward and both derivatives, on 2-D
// strided fp16/fp32 matrices (rows = tokens, cols = intermediate width).
//
//   p = 1 / (1 + exp(-g)),  act = g * p
//   forward   a  = act * u
//   backward  slope = p + act * (1 - p);  dg = (da * u) * slope;  du = da * act
//
// in fp32 with one rounding per operation (the translation unit is built
// with -ffp-contract=off), the order of solution/kernels/swiglu_fused.py:33-46.
// exp(-g) is 2^(-g log2 e) through v_exp_f32 and the reciprocal is v_rcp_f32
// (both within 1 ulp on their own; the product g log2 e adds a relative error
// of about |g| 2^-24); the fp16 results equal a float64 evaluation within one
// fp16 ulp apart from the cancellation of slope near g = -1.28.
//
// The pass is HBM-bound: 6 bytes per fp16 element forward (g, u read, a
// written), 10 backward (g, u, da read, dg, du written), against about 15
// VALU operations per element.  Contiguous rows take the vector kernel: a
// workgroup (grid x: row tiles, y: column tiles) covers 8 rows x 256
// columns, each thread one 8-element chunk (16-byte loads and stores for
// fp16, two for fp32), all loads issued before the arithmetic (with fp16
// operands the dtype is a template argument, so no run-time dtype branch
// separates them).  Measured at [990, 8960] fp16: 8-row tiles 10.2 / 20.4 us
// (forward / backward) before that change, 16-row
// tiles (two chunks per thread) 11.4 / 23.2 us, 32-row tiles 11.5 / 26.6 us.  Anything
// else (column strides, unaligned rows, widths not a multiple of 8) runs the
// element-wise kernel over the same tiles.

#include "common.h"
#include "elementwise.h"
#include "swiglu.h"

namespace ss {
namespace {

constexpr int kCols = 256;       // columns per workgroup tile
constexpr int kRows = 8;         // rows per workgroup tile
constexpr int kChunk = 8;        // elements per vector access

struct Mat {
  void* p;
  int dt;
  int64_t rs, cs;
};

__device__ __forceinline__ void load8(const Mat& m, int64_t off, float (&v)[kChunk]) {
  if (m.dt == SS_F16) {
    const half8 h = *reinterpret_cast<const half8*>(static_cast<const half_t*>(m.p) + off);
#pragma unroll
    for (int e = 0; e < kChunk; ++e) v[e] = (float)h[e];
  } else {
    const float* f = static_cast<const float*>(m.p) + off;
    const float4v a = *reinterpret_cast<const float4v*>(f);
    const float4v b = *reinterpret_cast<const float4v*>(f + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = a[e];
      v[e + 4] = b[e];
    }
  }
}

__device__ __forceinline__ void store8(const Mat& m, int64_t off, const float (&v)[kChunk]) {
  if (m.dt == SS_F16) {
    half8 h;
#pragma unroll
    for (int e = 0; e < kChunk; ++e) h[e] = f32_to_f16(v[e]);
    *reinterpret_cast<half8*>(static_cast<half_t*>(m.p) + off) = h;
  } else {
    float* f = static_cast<float*>(m.p) + off;
    float4v a, b;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a[e] = v[e];
      b[e] = v[e + 4];
    }
    *reinterpret_cast<float4v*>(f) = a;
    *reinterpret_cast<float4v*>(f + 4) = b;
  }
}

// fp16 operands (F16): plain 16-byte accesses, no run-time dtype branch, so a
// thread's loads go out together instead of each waiting for the previous one.
template <bool F16>
__device__ __forceinline__ void load8t(const Mat& m, int64_t off, float (&v)[kChunk]) {
  if constexpr (F16) {
    const half8 h = *reinterpret_cast<const half8*>(static_cast<const half_t*>(m.p) + off);
#pragma unroll
    for (int e = 0; e < kChunk; ++e) v[e] = (float)h[e];
  } else {
    load8(m, off, v);
  }
}

template <bool F16>
__device__ __forceinline__ void store8t(const Mat& m, int64_t off, const float (&v)[kChunk]) {
  if constexpr (F16) {
    half8 h;
#pragma unroll
    for (int e = 0; e < kChunk; ++e) h[e] = f32_to_f16(v[e]);
    *reinterpret_cast<half8*>(static_cast<half_t*>(m.p) + off) = h;
  } else {
    store8(m, off, v);
  }
}

// Vector kernel: unit column strides, 16-byte aligned rows, cols % 8 == 0;
// F16: every operand fp16.
template <bool BWD, bool F16>
__global__ __launch_bounds__(256) void swiglu_vec_kernel(Mat g, Mat u, Mat da, Mat o0, Mat o1,
                                                         int64_t rows, int64_t cols) {
  const int64_t c = blockIdx.y * (int64_t)kCols + (threadIdx.x & 31) * kChunk;
  const int64_t r0 = blockIdx.x * (int64_t)kRows + (threadIdx.x >> 5);
  if (c >= cols) return;
  constexpr int kU = kRows / 8;
  float gv[kU][kChunk], uv[kU][kChunk], dv[kU][kChunk];
#pragma unroll
  for (int k = 0; k < kU; ++k) {
    const int64_t r = r0 + 8 * k;
    if (r < rows) {
      load8t<F16>(g, r * g.rs + c, gv[k]);
      load8t<F16>(u, r * u.rs + c, uv[k]);
      if (BWD) load8t<F16>(da, r * da.rs + c, dv[k]);
    }
  }
#pragma unroll
  for (int k = 0; k < kU; ++k) {
    const int64_t r = r0 + 8 * k;
    if (r >= rows) continue;
    float a[kChunk], b[kChunk];
#pragma unroll
    for (int e = 0; e < kChunk; ++e) {
      const SwigluTerms t = swiglu_terms(gv[k][e]);
      if (BWD) {
        const float slope = swiglu_slope(t);
        a[e] = (dv[k][e] * uv[k][e]) * slope;
        b[e] = dv[k][e] * t.act;
      } else {
        a[e] = t.act * uv[k][e];
      }
    }
    store8t<F16>(o0, r * o0.rs + c, a);
    if (BWD) store8t<F16>(o1, r * o1.rs + c, b);
  }
}

// Element-wise kernel for any strides and widths.
template <bool BWD>
__global__ __launch_bounds__(256) void swiglu_any_kernel(Mat g, Mat u, Mat da, Mat o0, Mat o1,
                                                         int64_t rows, int64_t cols) {
  const int64_t c = blockIdx.y * (int64_t)kCols + threadIdx.x;
  if (c >= cols) return;
  for (int k = 0; k < kRows; ++k) {
    const int64_t r = blockIdx.x * (int64_t)kRows + k;
    if (r >= rows) break;
    const SwigluTerms t = swiglu_terms(ld_elem(g.p, g.dt, r * g.rs + c * g.cs));
    const float uu = ld_elem(u.p, u.dt, r * u.rs + c * u.cs);
    if (BWD) {
      const float d = ld_elem(da.p, da.dt, r * da.rs + c * da.cs);
      const float slope = swiglu_slope(t);
      st_elem(o0.p, o0.dt, r * o0.rs + c * o0.cs, (d * uu) * slope);
      st_elem(o1.p, o1.dt, r * o1.rs + c * o1.cs, d * t.act);
    } else {
      st_elem(o0.p, o0.dt, r * o0.rs + c * o0.cs, t.act * uu);
    }
  }
}

bool vector_ok(const Mat& m) {
  const int64_t es = m.dt == SS_F16 ? 2 : 4;
  return m.cs == 1 && reinterpret_cast<uintptr_t>(m.p) % 16 == 0 && (m.rs * es) % 16 == 0;
}

int launch(bool bwd, const Mat* mats, int count, int64_t rows, int64_t cols, void* stream,
           const char* fn) {
  bool vec = cols % kChunk == 0;
  for (int i = 0; i < count; ++i) vec = vec && vector_ok(mats[i]);
  const Mat none{nullptr, SS_F16, 0, 0};
  const Mat& g = mats[0];
  const Mat& u = mats[1];
  const Mat& da = bwd ? mats[2] : none;
  const Mat& o0 = bwd ? mats[3] : mats[2];
  const Mat& o1 = bwd ? mats[4] : none;
  const dim3 grid((unsigned)cdiv(rows, kRows), (unsigned)cdiv(cols, kCols));
  bool f16 = true;
  for (int i = 0; i < count; ++i) f16 = f16 && mats[i].dt == SS_F16;
  auto kern = !vec ? (bwd ? swiglu_any_kernel<true> : swiglu_any_kernel<false>)
              : f16 ? (bwd ? swiglu_vec_kernel<true, true> : swiglu_vec_kernel<false, true>)
                    : (bwd ? swiglu_vec_kernel<true, false> : swiglu_vec_kernel<false, false>);
  hipLaunchKernelGGL(kern, grid, dim3(256), 0, (hipStream_t)stream, g, u, da, o0, o1, rows, cols);
  SS_CHECK_LAUNCH(fn);
  return SS_OK;
}

int check_mats(const Mat* mats, int count, int64_t rows, int64_t cols, const char* fn) {
  SS_CHECK_ARG(rows >= 0 && cols >= 0, "%s: negative size", fn);
  SS_CHECK_ARG(cdiv(rows, kRows) <= 0x7fffffff && cdiv(cols, kCols) <= 0xffff,
               "%s: %lld x %lld exceeds the launch grid", fn, (long long)rows, (long long)cols);
  for (int i = 0; i < count; ++i) {
    SS_CHECK_ARG(valid_dtype(mats[i].dt), "%s: dtype of operand %d must be SS_F16 or SS_F32", fn,
                 i);
    if (rows && cols) SS_CHECK_ARG(mats[i].p, "%s: operand %d is null", fn, i);
  }
  return SS_OK;
}

}  // namespace
}  // namespace ss

using namespace ss;

extern "C" int ss_swiglu_fwd(const void* gate, int gate_dtype, int64_t g_rs, int64_t g_cs,
                             const void* up, int up_dtype, int64_t u_rs, int64_t u_cs, void* out,
                             int out_dtype, int64_t o_rs, int64_t o_cs, int64_t rows, int64_t cols,
                             void* stream) {
  const char* fn = "ss_swiglu_fwd";
  const Mat mats[3] = {{const_cast<void*>(gate), gate_dtype, g_rs, g_cs},
                       {const_cast<void*>(up), up_dtype, u_rs, u_cs},
                       {out, out_dtype, o_rs, o_cs}};
  const int rc = check_mats(mats, 3, rows, cols, fn);
  if (rc != SS_OK || rows == 0 || cols == 0) return rc;
  return launch(false, mats, 3, rows, cols, stream, fn);
}

extern "C" int ss_swiglu_bwd(const void* gate, int gate_dtype, int64_t g_rs, int64_t g_cs,
                             const void* up, int up_dtype, int64_t u_rs, int64_t u_cs,
                             const void* grad, int grad_dtype, int64_t d_rs, int64_t d_cs,
                             void* dgate, int dgate_dtype, int64_t dg_rs, int64_t dg_cs, void* dup,
                             int dup_dtype, int64_t du_rs, int64_t du_cs, int64_t rows,
                             int64_t cols, void* stream) {
  const char* fn = "ss_swiglu_bwd";
  const Mat mats[5] = {{const_cast<void*>(gate), gate_dtype, g_rs, g_cs},
                       {const_cast<void*>(up), up_dtype, u_rs, u_cs},
                       {const_cast<void*>(grad), grad_dtype, d_rs, d_cs},
                       {dgate, dgate_dtype, dg_rs, dg_cs},
                       {dup, dup_dtype, du_rs, du_cs}};
  const int rc = check_mats(mats, 5, rows, cols, fn);
  if (rc != SS_OK || rows == 0 || cols == 0) return rc;
  return launch(true, mats, 5, rows, cols, stream, fn);
}
