// LoRA dropout of the fused QLoRA projection (A10 / A12 with p > 0).
//
// Reference: solution/lora.py:1-40,151-163 -- PEFT's Dropout on an fp32 copy
// of X feeds only the LoRA branch: Z = fp16(fp16(drop(X)) . A^T); backward
// dA = fp16(dZ^T . fp16(drop(X))) and, through the dropout and the casts,
// dX += fp16(fp16(dZ . A) * mask / (1 - p)).  Here the mask is never stored:
// every kernel that touches an element of X recomputes its keep bit from the
// call's seed (philox.h), so forward and backward agree without a [T, K]
// mask tensor.  Z (rank_project_block) and dA (rank_grad_block) apply the
// mask to X as they load it; this file holds the mask export and the
// backward's tail launch: the dA blocks plus an element-wise pass that adds
// the masked rank-16 term to dX, which the dX GEMM then computes without it.

#include "rank16.h"

namespace ss {

__global__ __launch_bounds__(256) void dropout_mask_kernel(DropoutArgs d, uint8_t* __restrict__ out,
                                                           int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g * 4 < n; g += stride) {
    const uint32_t bits = keep4(d, (uint64_t)g);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (g * 4 + j < n) out[g * 4 + j] = (uint8_t)((bits >> j) & 1u);
  }
}

// dX[t, c] = fp16(dX[t, c] + fp16(fp16(sum_r dZ[t, r] A[r, c]) * inv)) where
// kept; 8 columns per thread (k % 8 == 0, 16-byte aligned rows).  A group
// with no kept element is left as it is.
struct DropDx {
  half_t* dx;
  int64_t lddx, t, k;
  const half_t* dz;   // [t, 16]
  const half_t* a;    // [16, k]
  DropoutArgs drop;
};

__device__ __forceinline__ void drop_dx_group(const DropDx& u, int64_t g) {
  const int64_t per_row = u.k / 8;
  const int64_t row = g / per_row;
  const int64_t c0 = (g - row * per_row) * 8;
  const uint32_t bits = keep8(u.drop, (uint64_t)(row * u.k + c0));
  if (!bits) return;
  const half8 z0 = *reinterpret_cast<const half8*>(u.dz + row * 16);
  const half8 z1 = *reinterpret_cast<const half8*>(u.dz + row * 16 + 8);
  half8* dst = reinterpret_cast<half8*>(u.dx + row * u.lddx + c0);
  half8 out = *dst;
  float lora[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) lora[c] = 0.0f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const half8 ar = *reinterpret_cast<const half8*>(u.a + r * u.k + c0);
    const float z = (float)(r < 8 ? z0[r] : z1[r - 8]);
#pragma unroll
    for (int c = 0; c < 8; ++c) lora[c] += z * (float)ar[c];
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    if (!((bits >> c) & 1u)) continue;
    const float v = (float)f32_to_f16((float)f32_to_f16(lora[c]) * u.drop.inv);
    out[c] = f32_to_f16((float)out[c] + v);
  }
  *dst = out;
}

// Blocks [0, da_blocks): dA = fp16(dZ^T . fp16(drop(X))) (rank_grad_block);
// the rest: the dX update, grid-stride over the [t, k / 8] groups.
__global__ __launch_bounds__(256) void qlora_dropout_tail_kernel(RankGradArgs da,
                                                                 int64_t da_blocks, DropDx u) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[kRankGradSmem];
  if ((int64_t)blockIdx.x < da_blocks) {
    const int64_t nblocks = cdiv(da.n, 64);
    rank_grad_block<true, true>(da, blockIdx.x % nblocks, blockIdx.x / nblocks, smem);
    return;
  }
  const int64_t groups = u.t * (u.k / 8);
  const int64_t b = blockIdx.x - da_blocks;
  const int64_t stride = ((int64_t)gridDim.x - da_blocks) * blockDim.x;
  for (int64_t g = b * blockDim.x + threadIdx.x; g < groups; g += stride) drop_dx_group(u, g);
}

DropoutArgs dropout_args(uint64_t seed, float p) {
  DropoutArgs d;
  d.seed = seed;
  // keep(e) = word < thr.  For p below 2^-32, (1 - p) * 2^32 rounds to 2^32, which a
  // uint32 cannot hold: the threshold saturates, so such a p drops with probability 2^-32.
  const double thr = floor((1.0 - (double)p) * 4294967296.0);
  d.thr = thr >= 4294967295.0 ? 0xFFFFFFFFu : (uint32_t)thr;
  d.inv = (float)(1.0 / (1.0 - (double)p));
  d.on = 1;
  return d;
}

// The backward tail: dA (masked X) and the masked rank-16 term of dX.
// Needs vector operands (16-byte aligned dZ, X, A, dX rows; k % 8 == 0).
int launch_dropout_tail(const half_t* dz, const half_t* x, int64_t ldx, const half_t* lora_a,
                        int64_t t, int64_t k, half_t* dx, int64_t lddx, half_t* da,
                        const DropoutArgs& drop, void* rank_ws, size_t rank_ws_bytes,
                        hipStream_t stream) {
  RankGradArgs g;
  bool vec = false;
  const int64_t da_blocks = rank_grad_setup(g, dz, 16, x, ldx, t, k, 1.0f, 0, da, rank_ws,
                                            rank_ws_bytes, 0, vec);
  if (!vec) return SS_ERR_UNSUPPORTED;
  g.drop = drop;
  DropDx u{dx, lddx, t, k, dz, lora_a, drop};
  const int64_t groups = t * (k / 8);
  int64_t upd = cdiv(groups, 256);
  if (upd > 4096) upd = 4096;
  if (upd < 1) upd = 1;
  hipLaunchKernelGGL(qlora_dropout_tail_kernel, dim3((unsigned)(da_blocks + upd)), dim3(256), 0,
                     stream, g, da_blocks, u);
  SS_CHECK_LAUNCH("qlora_dropout_tail_kernel");
  return SS_OK;
}

}  // namespace ss

extern "C" int ss_dropout_mask(uint64_t seed, float p, int64_t rows, int64_t cols, uint8_t* out,
                               void* stream) {
  const char* fn = "ss_dropout_mask";
  SS_CHECK_ARG(rows >= 0 && cols >= 0, "%s: negative size", fn);
  SS_CHECK_ARG(p > 0.0f && p < 1.0f, "%s: p=%g must be in (0, 1)", fn, (double)p);
  const int64_t n = rows * cols;
  if (n == 0) return SS_OK;
  SS_CHECK_ARG(out != nullptr, "%s: null pointer", fn);
  const ss::DropoutArgs d = ss::dropout_args(seed, p);
  int64_t blocks = ss::cdiv(ss::cdiv(n, 4), 256);
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(ss::dropout_mask_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, d, out, n);
  SS_CHECK_LAUNCH("dropout_mask_kernel");
  return SS_OK;
}
