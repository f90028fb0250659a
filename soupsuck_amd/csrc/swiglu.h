// SwiGLU terms shared by the element-wise kernels (swiglu.hip) and the GEMM
// epilogues that apply the activation to their output (gemm.h glu_apply):
// p = 1 / (1 + exp(-g)) with exp(-g) = 2^(-g log2 e) on v_exp_f32 and the
// reciprocal on v_rcp_f32, act = g p.  Both users must produce the same bits,
// so there is one definition.
#pragma once

#include "common.h"

namespace ss {

struct SwigluTerms {
  float p, act;
};

__device__ __forceinline__ SwigluTerms swiglu_terms(float g) {
  constexpr float kLog2e = 1.4426950408889634f;
  const float e = __builtin_amdgcn_exp2f(g * -kLog2e);
  const float p = __builtin_amdgcn_rcpf(1.0f + e);
  return {p, g * p};
}

// slope = d act / d g = p + act (1 - p), in this order.
__device__ __forceinline__ float swiglu_slope(const SwigluTerms& t) {
  return t.p + t.act * (1.0f - t.p);
}

}  // namespace ss
