// Rank-16 products of the LoRA branch on MFMA (A10/A12).
//
// Reference: solution/lora.py:151-163 (Z = X.A^T, L = Z.B^T under fp16
// autocast) and solution/lora_pair.py:52-65 (dZ = dL.B, dB = dL^T.Z,
// dA = dZ^T.X).  With rank r = 16 these are "skinny" GEMMs: one operand is
// [T, K] or [T, N] (read once from HBM), the other 16 x K.  They are
// HBM-bound, so both kernels split the long dimension over many waves and
// reduce fp32 partials in a second, tiny pass (deterministic order).
//
// rank_project:  C[M, 16] = A[M, K] . W,  W(k, r) = w_kr ? w[k*ldw + r] : w[r*ldw + k],
//                A optionally replaced by fp16(A * a_scale) (dL = fp16(g * s)).
//                One wave per (16-row block, K chunk); MFMA operands come
//                straight from global memory (16 B per lane for A).
// rank_grad:     C[16, N] = P[T, 16]^T . Q[T, N] (Q optionally fp16(Q * q_scale)),
//                stored [16][N] or transposed [N][16].  One wave per
//                (64-column block, T chunk); Q tiles are loaded coalesced
//                (128 B per row) and transposed through LDS.
// The final pass sums the partials in chunk order and rounds once to fp16.

#include "common.h"

namespace ss {

constexpr int kRank = 16;

__device__ __forceinline__ half8 load_row8(const half_t* __restrict__ p, int64_t row,
                                           int64_t rows, int64_t ld, int64_t k, int64_t kend,
                                           bool vec) {
  half8 v;
  if (row < rows && vec && k + 8 <= kend) {
    v = *reinterpret_cast<const half8*>(p + row * ld + k);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      v[i] = (row < rows && k + i < kend) ? p[row * ld + k + i] : (half_t)0.0f;
  }
  return v;
}

__global__ __launch_bounds__(256) void rank_project_kernel(
    const half_t* __restrict__ a, int64_t lda, int64_t m, int64_t k, const half_t* __restrict__ w,
    int64_t ldw, int w_kr, int scale_a, float a_scale, float* __restrict__ part, int64_t splits,
    int64_t kchunk, int vec) {
  const int lane = threadIdx.x & 63;
  const int64_t mblocks = cdiv(m, 16);
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= mblocks * splits) return;  // the whole wave leaves together
  const int64_t mb = item % mblocks;
  const int64_t s = item / mblocks;
  const int64_t kbeg = s * kchunk;
  const int64_t kend = kbeg + kchunk < k ? kbeg + kchunk : k;
  const int r = lane & 15;
  const int kq = (lane >> 4) * 8;
  const int64_t row = mb * 16 + r;
  float4v acc[2] = {float4v{0.f, 0.f, 0.f, 0.f}, float4v{0.f, 0.f, 0.f, 0.f}};
  int it = 0;
  for (int64_t k0 = kbeg; k0 < kend; k0 += 32, ++it) {
    half8 av = load_row8(a, row, m, lda, k0 + kq, kend, vec);
    if (scale_a) {
#pragma unroll
      for (int i = 0; i < 8; ++i) av[i] = f32_to_f16((float)av[i] * a_scale);
    }
    half8 bv;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t kk = k0 + kq + i;
      bv[i] = kk < kend ? (w_kr ? w[kk * ldw + r] : w[r * ldw + kk]) : (half_t)0.0f;
    }
    acc[it & 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc[it & 1], 0, 0, 0);
  }
  const float4v c = acc[0] + acc[1];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t mm = mb * 16 + (lane >> 4) * 4 + j;
    if (mm < m) part[(s * m + mm) * kRank + r] = c[j];
  }
}

__global__ __launch_bounds__(256) void rank_grad_kernel(
    const half_t* __restrict__ p, int64_t ldp, const half_t* __restrict__ q, int64_t ldq,
    int64_t t, int64_t n, int scale_q, float q_scale, float* __restrict__ part, int64_t splits,
    int64_t tchunk, int vec) {
  constexpr int LDT = 40;  // 32 t values + 8 pad per LDS row (one row per column of Q)
  __shared__ __attribute__((aligned(16))) half_t sq[4][64 * LDT];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t nblocks = cdiv(n, 64);
  const int64_t item = (int64_t)blockIdx.x * 4 + wave;
  if (item >= nblocks * splits) return;  // no block-wide barrier below: waves are independent
  const int64_t nb = item % nblocks;
  const int64_t s = item / nblocks;
  const int64_t n0 = nb * 64;
  const int64_t tbeg = s * tchunk;
  const int64_t tend = tbeg + tchunk < t ? tbeg + tchunk : t;
  half_t* tile = sq[wave];
  const int r = lane & 15;
  const int kq = (lane >> 4) * 8;
  float4v acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = float4v{0.f, 0.f, 0.f, 0.f};
  for (int64_t t0 = tbeg; t0 < tend; t0 += 32) {
    // Q tile [32 t x 64 n]: lane loads 8 columns of one row; 4 passes of 8 rows.
#pragma unroll
    for (int pass = 0; pass < 4; ++pass) {
      const int tl = pass * 8 + (lane >> 3);
      const int nl = (lane & 7) * 8;
      half8 v = load_row8(q, t0 + tl, tend, ldq, n0 + nl, n, vec);
      if (scale_q) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = f32_to_f16((float)v[i] * q_scale);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) tile[(nl + i) * LDT + tl] = v[i];
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_s_waitcnt(0);
    // A operand: P^T (r = lane % 16, t = t0 + kq + i); small and cache resident.
    half8 av;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t tt = t0 + kq + i;
      av[i] = tt < tend ? p[tt * ldp + r] : (half_t)0.0f;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const half8 bv = *reinterpret_cast<const half8*>(tile + (c * 16 + r) * LDT + kq);
      acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc[c], 0, 0, 0);
    }
    __builtin_amdgcn_wave_barrier();
  }
  // lane holds C[r' = 4*(lane/16) + j][n0 + 16c + lane%16]
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int64_t col = n0 + c * 16 + r;
    if (col >= n) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int rr = (lane >> 4) * 4 + j;
      part[(s * kRank + rr) * n + col] = acc[c][j];
    }
  }
}

// out[m][r] (project) = fp16(sum_s part[s][m][r]); out row stride 16.
__global__ __launch_bounds__(256) void rank_project_reduce_kernel(const float* __restrict__ part,
                                                                  int64_t m, int64_t splits,
                                                                  half_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= m * kRank) return;
  float acc = 0.0f;
  for (int64_t s = 0; s < splits; ++s) acc += part[s * m * kRank + i];
  out[i] = f32_to_f16(acc);
}

// grad: out = fp16(sum_s part[s][r][c]) stored [16][n] (transpose = 0) or [n][16].
__global__ __launch_bounds__(256) void rank_grad_reduce_kernel(const float* __restrict__ part,
                                                               int64_t n, int64_t splits,
                                                               int transpose,
                                                               half_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n * kRank) return;
  float acc = 0.0f;
  for (int64_t s = 0; s < splits; ++s) acc += part[s * n * kRank + i];
  const int64_t rr = i / n;
  const int64_t c = i - rr * n;
  out[transpose ? c * kRank + rr : i] = f32_to_f16(acc);
}

// Split count so that the grid has about four waves per CU (1024 waves).
static int64_t pick_splits(int64_t blocks, int64_t len, int64_t step) {
  int64_t s = cdiv(1024, blocks > 0 ? blocks : 1);
  const int64_t max_s = cdiv(len, step);
  if (s > max_s) s = max_s;
  return s < 1 ? 1 : s;
}

static bool al16(const void* p, int64_t ld) {
  return reinterpret_cast<uintptr_t>(p) % 16 == 0 && ld % 8 == 0;
}

}  // namespace ss

using namespace ss;

extern "C" size_t ss_lora_workspace_size(int64_t rows, int64_t cols) {
  // fp32 partials of either kernel for a [rows x 16] or [16 x cols] result:
  // at most cdiv(1024, blocks) splits, blocks >= cdiv(len, 64).
  const int64_t m = rows > cols ? rows : cols;
  const int64_t s = cdiv(1024, cdiv(m > 0 ? m : 1, 64)) + 1;
  return (size_t)(s * (m > 0 ? m : 1) * kRank) * sizeof(float) + 256;
}

extern "C" int ss_lora_project(const uint16_t* a, int64_t lda, int64_t m, int64_t k,
                               const uint16_t* w, int64_t ldw, int w_kr, int scale_a,
                               float a_scale, uint16_t* out, void* workspace,
                               size_t workspace_bytes, void* stream) {
  const char* fn = "ss_lora_project";
  SS_CHECK_ARG(m >= 0 && k >= 0, "%s: negative size", fn);
  if (m == 0) return SS_OK;
  SS_CHECK_ARG(a && w && out && workspace, "%s: null pointer", fn);
  SS_CHECK_ARG(lda >= k && ldw >= (w_kr ? kRank : k), "%s: leading dimension too small", fn);
  const int64_t mblocks = cdiv(m, 16);
  int64_t splits = pick_splits(mblocks, k, 32);
  int64_t kchunk = cdiv(cdiv(k, splits), 32) * 32;
  if (kchunk == 0) kchunk = 32;
  splits = cdiv(k > 0 ? k : 1, kchunk);
  SS_CHECK_ARG((size_t)(splits * m * kRank) * sizeof(float) <= workspace_bytes,
               "%s: workspace too small", fn);
  float* part = reinterpret_cast<float*>(workspace);
  hipStream_t s = (hipStream_t)stream;
  const int64_t waves = mblocks * splits;
  hipLaunchKernelGGL(rank_project_kernel, dim3((unsigned)cdiv(waves, 4)), dim3(256), 0, s,
                     reinterpret_cast<const half_t*>(a), lda, m, k,
                     reinterpret_cast<const half_t*>(w), ldw, w_kr, scale_a, a_scale, part,
                     splits, kchunk, (int)al16(a, lda));
  SS_CHECK_LAUNCH("rank_project_kernel");
  hipLaunchKernelGGL(rank_project_reduce_kernel, dim3((unsigned)cdiv(m * kRank, 256)), dim3(256),
                     0, s, part, m, splits, reinterpret_cast<half_t*>(out));
  SS_CHECK_LAUNCH("rank_project_reduce_kernel");
  return SS_OK;
}

extern "C" int ss_lora_grad(const uint16_t* p, int64_t ldp, const uint16_t* q, int64_t ldq,
                            int64_t t, int64_t n, int scale_q, float q_scale, int transpose,
                            uint16_t* out, void* workspace, size_t workspace_bytes,
                            void* stream) {
  const char* fn = "ss_lora_grad";
  SS_CHECK_ARG(t >= 0 && n >= 0, "%s: negative size", fn);
  if (n == 0) return SS_OK;
  SS_CHECK_ARG(out && workspace && (t == 0 || (p && q)), "%s: null pointer", fn);
  SS_CHECK_ARG(ldp >= kRank && ldq >= n, "%s: leading dimension too small", fn);
  const int64_t nblocks = cdiv(n, 64);
  int64_t splits = pick_splits(nblocks, t, 32);
  int64_t tchunk = cdiv(cdiv(t, splits), 32) * 32;
  if (tchunk == 0) tchunk = 32;
  splits = t > 0 ? cdiv(t, tchunk) : 1;
  SS_CHECK_ARG((size_t)(splits * n * kRank) * sizeof(float) <= workspace_bytes,
               "%s: workspace too small", fn);
  float* part = reinterpret_cast<float*>(workspace);
  hipStream_t s = (hipStream_t)stream;
  const int64_t waves = nblocks * splits;
  hipLaunchKernelGGL(rank_grad_kernel, dim3((unsigned)cdiv(waves, 4)), dim3(256), 0, s,
                     reinterpret_cast<const half_t*>(p), ldp, reinterpret_cast<const half_t*>(q),
                     ldq, t, n, scale_q, q_scale, part, splits, tchunk, (int)al16(q, ldq));
  SS_CHECK_LAUNCH("rank_grad_kernel");
  hipLaunchKernelGGL(rank_grad_reduce_kernel, dim3((unsigned)cdiv(n * kRank, 256)), dim3(256), 0,
                     s, part, n, splits, transpose, reinterpret_cast<half_t*>(out));
  SS_CHECK_LAUNCH("rank_grad_reduce_kernel");
  return SS_OK;
}
