// LoRA scale/add epilogue and its gradient (A11).
//
// Reference: solution/kernels/lora_epilogue.py:1-13,24-43.  The scaled
// adapter output is rounded to the adapter dtype BEFORE it is added (and to
// the base dtype when cast_to_result), so a fused multiply-add would change
// bits; this file is built without contraction.  HBM-bound elementwise.

#include "elementwise.h"

namespace ss {

__global__ __launch_bounds__(256) void lora_fwd_kernel(const void* __restrict__ base, int bd,
                                                       const void* __restrict__ adapter, int ad,
                                                       void* __restrict__ out, int od,
                                                       int64_t count, float scale, int cast) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
    const float b = ld_elem(base, bd, i);
    const float a = ld_elem(adapter, ad, i);
    const float product = a * scale;
    float scaled = round_to(ad, product);
    if (cast) scaled = round_to(bd, scaled);
    st_elem(out, od, i, b + scaled);
  }
}

__global__ __launch_bounds__(256) void lora_bwd_kernel(const void* __restrict__ grad, int gd,
                                                       void* __restrict__ d_adapter, int ad,
                                                       int64_t count, float scale) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += stride) {
    const float g = round_to(ad, ld_elem(grad, gd, i));
    st_elem(d_adapter, ad, i, g * scale);
  }
}

static unsigned grid_1d(int64_t count) {
  const int64_t blocks = cdiv(count, 256);
  return (unsigned)(blocks < 8192 ? blocks : 8192);
}

}  // namespace ss

using namespace ss;

extern "C" int ss_lora_epilogue_fwd(const void* base, int base_dtype, const void* adapter,
                                    int adapter_dtype, void* out, int out_dtype, int64_t count,
                                    float scale, int cast_to_result, void* stream) {
  SS_CHECK_ARG(count >= 0, "ss_lora_epilogue_fwd: negative count");
  SS_CHECK_ARG(valid_dtype(base_dtype) && valid_dtype(adapter_dtype) && valid_dtype(out_dtype),
               "ss_lora_epilogue_fwd: dtype must be SS_F16 or SS_F32");
  const int expect = cast_to_result ? base_dtype : promote(base_dtype, adapter_dtype);
  SS_CHECK_ARG(out_dtype == expect, "ss_lora_epilogue_fwd: out dtype %d, expected %d", out_dtype,
               expect);
  if (count == 0) return SS_OK;
  SS_CHECK_ARG(base && adapter && out, "ss_lora_epilogue_fwd: null pointer");
  hipLaunchKernelGGL(lora_fwd_kernel, dim3(grid_1d(count)), dim3(256), 0, (hipStream_t)stream,
                     base, base_dtype, adapter, adapter_dtype, out, out_dtype, count, scale,
                     cast_to_result ? 1 : 0);
  SS_CHECK_LAUNCH("lora_fwd_kernel");
  return SS_OK;
}

extern "C" int ss_lora_epilogue_bwd(const void* grad, int grad_dtype, void* d_adapter,
                                    int adapter_dtype, int64_t count, float scale, void* stream) {
  SS_CHECK_ARG(count >= 0, "ss_lora_epilogue_bwd: negative count");
  SS_CHECK_ARG(valid_dtype(grad_dtype) && valid_dtype(adapter_dtype),
               "ss_lora_epilogue_bwd: dtype must be SS_F16 or SS_F32");
  if (count == 0) return SS_OK;
  SS_CHECK_ARG(grad && d_adapter, "ss_lora_epilogue_bwd: null pointer");
  hipLaunchKernelGGL(lora_bwd_kernel, dim3(grid_1d(count)), dim3(256), 0, (hipStream_t)stream,
                     grad, grad_dtype, d_adapter, adapter_dtype, count, scale);
  SS_CHECK_LAUNCH("lora_bwd_kernel");
  return SS_OK;
}
