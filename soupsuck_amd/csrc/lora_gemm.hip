// Rank-16 products of the LoRA branch on MFMA (A10/A12).
//
// Reference: solution/lora.py:151-163 (Z = X.A^T, L = Z.B^T under fp16
// autocast) and solution/lora_pair.py:52-65 (dZ = dL.B, dB = dL^T.Z,
// dA = dZ^T.X).  With rank r = 16 these are "skinny" GEMMs: one operand is
// [T, K] or [T, N] (read once from HBM), the other 16 x K.  They are
// HBM-bound and, at training shapes (T ~ 1000), short: launch latency is a
// large share of their time.  Each op is therefore one launch in which a
// workgroup owns a block of outputs and its waves split the reduced
// dimension, combining their fp32 sums through LDS in wave order
// (deterministic).  When few output blocks meet a long reduction (large T
// with a narrow N in rank_grad) the reduction is instead split over many
// workgroups whose fp32 partials a second, tiny pass sums in chunk order.
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

// 8 consecutive elements p[row*ld + k .. +7], zero outside rows x [.., kend).
// VEC: the caller guarantees 16-byte aligned rows and kend % 8 == 0, so a
// chunk is either wholly valid or wholly outside; the load is then branch-free
// (clamped address + select), which keeps every load of a wave in flight.
template <bool VEC>
__device__ __forceinline__ half8 load_row8(const half_t* __restrict__ p, int64_t row,
                                           int64_t rows, int64_t ld, int64_t k, int64_t kend) {
  if constexpr (VEC) {
    const bool ok = row < rows && k < kend;
    const u32x4 raw = *reinterpret_cast<const u32x4*>(p + (ok ? row * ld + k : 0));
    const u32x4 v = ok ? raw : u32x4{0u, 0u, 0u, 0u};
    return __builtin_bit_cast(half8, v);
  } else {
    half8 v;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      v[i] = (row < rows && k + i < kend) ? p[row * ld + k + i] : (half_t)0.0f;
    return v;
  }
}

// Chunk sizes: every wave issues all loads of its chunk before its first MFMA
// (eight 16-byte loads per lane in flight), so a chunk costs about one memory
// round trip.  kMaxSplits bounds the fp32 partials.
constexpr int kProjChunk = 256;  // k per rank_project wave: 8 MFMA steps of 32
constexpr int kGradChunk = 64;   // t per rank_grad step: 2 MFMA steps of 32
constexpr int kMaxSplits = 64;
constexpr int kProjLd = kProjChunk + 8;  // LDS row of the staged W chunk (one rank row)
constexpr int kGradLd = kGradChunk + 8;  // LDS row of the transposed P tile

// Transposed Q tile [64 n][64 t], rows of 128 B with the 16-byte chunk index
// XOR-swizzled by (n ^ n/8) & 7: the transposing 2-byte writes (8 rows 8 apart
// per instruction) and the 16-byte fragment reads (8 consecutive rows) both
// touch 8 distinct chunks, i.e. no LDS bank conflicts.
__device__ __forceinline__ int qtile_index(int n, int t) {
  return n * 64 + ((((t >> 3) ^ n ^ (n >> 3)) & 7) << 3) + (t & 7);
}

// One 256-k chunk [kbeg, kend) of a 16-row block: acc += A'[rows, chunk] . W(chunk, :),
// with W(k, r) staged in the wave's LDS tile as tile[r][k - kbeg].
template <bool VEC>
__device__ __forceinline__ void project_chunk(const half_t* __restrict__ a, int64_t lda,
                                              int64_t m, const half_t* __restrict__ w,
                                              int64_t ldw, int w_kr, float a_scale, int64_t row,
                                              int lane, int64_t kbeg, int64_t kend, half_t* tile,
                                              float4v (&acc)[2]) {
  const int r = lane & 15;
  const int kq = (lane >> 4) * 8;
  half8 av[8];
#pragma unroll
  for (int st = 0; st < 8; ++st) av[st] = load_row8<VEC>(a, row, m, lda, kbeg + st * 32 + kq, kend);
  // Stage W(k, r) for k in [kbeg, kend) as tile[r][k - kbeg] (zero beyond kend).
  if (w_kr) {
    // w is [K][ldw]: one 32-byte row of 16 ranks per k; lane takes 8 ranks of one k.
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int kk = it * 32 + (lane >> 1);
      const int rh = (lane & 1) * 8;
      const half8 v = load_row8<VEC>(w, kbeg + kk, kend, ldw, rh, kRank);
#pragma unroll
      for (int i = 0; i < 8; ++i) tile[(rh + i) * kProjLd + kk] = v[i];
    }
  } else {
    // w is [16][ldw]: each rank row is contiguous in k.
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int c = it * 64 + lane;
      const int rr = c >> 5;
      const int kc = (c & 31) * 8;
      const half8 v = load_row8<VEC>(w + rr * ldw, 0, 1, 0, kbeg + kc, kend);
      *reinterpret_cast<half8*>(tile + rr * kProjLd + kc) = v;
    }
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_s_waitcnt(0);
  // fp16(a * 1.0) == a for every fp16 value, so "no scaling" is a_scale = 1.
#pragma unroll
  for (int st = 0; st < 8; ++st)
#pragma unroll
    for (int i = 0; i < 8; ++i) av[st][i] = f32_to_f16((float)av[st][i] * a_scale);
#pragma unroll
  for (int st = 0; st < 8; ++st) {
    const half8 bv = *reinterpret_cast<const half8*>(tile + r * kProjLd + st * 32 + kq);
    acc[st & 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[st], bv, acc[st & 1], 0, 0, 0);
  }
  __builtin_amdgcn_wave_barrier();
}

// Split form: one wave per (16-row block, K split); fp32 partials part[s][m][16].
template <bool VEC>
__global__ __launch_bounds__(256) void rank_project_kernel(
    const half_t* __restrict__ a, int64_t lda, int64_t m, int64_t k, const half_t* __restrict__ w,
    int64_t ldw, int w_kr, float a_scale, float* __restrict__ part, int64_t splits,
    int64_t kchunk) {
  __shared__ __attribute__((aligned(16))) half_t sw[4][kRank * kProjLd];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t mblocks = cdiv(m, 16);
  const int64_t item = (int64_t)blockIdx.x * 4 + wave;
  if (item >= mblocks * splits) return;  // no block-wide barrier below: waves are independent
  const int64_t mb = item % mblocks;
  const int64_t s = item / mblocks;
  const int64_t send = (s + 1) * kchunk < k ? (s + 1) * kchunk : k;
  const int r = lane & 15;
  const int64_t row = mb * 16 + r;
  float4v acc[2] = {float4v{0.f, 0.f, 0.f, 0.f}, float4v{0.f, 0.f, 0.f, 0.f}};
  for (int64_t kbeg = s * kchunk; kbeg < send; kbeg += kProjChunk) {
    const int64_t kend = kbeg + kProjChunk < send ? kbeg + kProjChunk : send;
    project_chunk<VEC>(a, lda, m, w, ldw, w_kr, a_scale, row, lane, kbeg, kend, sw[wave], acc);
  }
  const float4v c = acc[0] + acc[1];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t mm = mb * 16 + (lane >> 4) * 4 + j;
    if (mm < m) part[(s * m + mm) * kRank + r] = c[j];
  }
}

// One-launch form: workgroup = one 16-row block, blockDim.x / 64 waves; wave w
// takes the 256-k chunks w, w + waves, ...; the waves' sums are added in wave
// order through LDS and rounded once to fp16 (out row stride 16).
constexpr int kRowWaves = 16;

template <bool VEC>
__global__ __launch_bounds__(kRowWaves * 64) void rank_project_rows_kernel(
    const half_t* __restrict__ a, int64_t lda, int64_t m, int64_t k, const half_t* __restrict__ w,
    int64_t ldw, int w_kr, float a_scale, half_t* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) half_t sw[kRowWaves][kRank * kProjLd];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  const int64_t mb = blockIdx.x;
  const int r = lane & 15;
  const int64_t row = mb * 16 + r;
  float4v acc[2] = {float4v{0.f, 0.f, 0.f, 0.f}, float4v{0.f, 0.f, 0.f, 0.f}};
  for (int64_t kbeg = (int64_t)wave * kProjChunk; kbeg < k;
       kbeg += (int64_t)waves * kProjChunk) {
    const int64_t kend = kbeg + kProjChunk < k ? kbeg + kProjChunk : k;
    project_chunk<VEC>(a, lda, m, w, ldw, w_kr, a_scale, row, lane, kbeg, kend, sw[wave], acc);
  }
  // The per-wave tiles are dead once every wave has passed this barrier;
  // their first 16 KiB hold the waves' 16x16 sums.
  __syncthreads();
  float4v* red = reinterpret_cast<float4v*>(&sw[0][0]);
  red[wave * 64 + lane] = acc[0] + acc[1];
  __syncthreads();
  if (wave != 0) return;
  float4v c = red[lane];
  for (int w2 = 1; w2 < waves; ++w2) c += red[w2 * 64 + lane];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t mm = mb * 16 + (lane >> 4) * 4 + j;
    if (mm < m) out[mm * kRank + r] = f32_to_f16(c[j]);
  }
}

// One 64-t chunk [t0, tend) of a 64-column block at n0: acc[c] += P[chunk, :]^T .
// Q'[chunk, n0 + 16c .. +15], Q transposed through the wave's LDS tile.
template <bool VEC>
__device__ __forceinline__ void grad_chunk(const half_t* __restrict__ p, int64_t ldp,
                                           const half_t* __restrict__ q, int64_t ldq, int64_t n,
                                           float q_scale, int64_t n0, int lane, int64_t t0,
                                           int64_t tend, half_t* tile, half_t* ptile,
                                           float4v (&acc)[4]) {
  const int r = lane & 15;
  const int kq = (lane >> 4) * 8;
  // Q tile [64 t x 64 n]: 8 rows of 8 lanes per pass, 16 bytes per lane.
  half8 v[8];
#pragma unroll
  for (int it = 0; it < 8; ++it)
    v[it] = load_row8<VEC>(q, t0 + it * 8 + (lane >> 3), tend, ldq, n0 + (lane & 7) * 8, n);
  // P rows [64 t x 16 r]: lane takes one row (two 16-byte halves).
  const half8 p0 = load_row8<VEC>(p, t0 + lane, tend, ldp, 0, kRank);
  const half8 p1 = load_row8<VEC>(p, t0 + lane, tend, ldp, 8, kRank);
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int tl = it * 8 + (lane >> 3);
    const int nl = (lane & 7) * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // fp16(q * 1.0) == q for every fp16 value, so "no scaling" is q_scale = 1.
      tile[qtile_index(nl + i, tl)] = f32_to_f16((float)v[it][i] * q_scale);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    ptile[i * kGradLd + lane] = p0[i];
    ptile[(8 + i) * kGradLd + lane] = p1[i];
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const half8 av = *reinterpret_cast<const half8*>(ptile + r * kGradLd + kk * 32 + kq);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const half8 bv =
          *reinterpret_cast<const half8*>(tile + qtile_index(c * 16 + r, kk * 32 + kq));
      acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc[c], 0, 0, 0);
    }
  }
  __builtin_amdgcn_wave_barrier();
}

// Split form: one wave per (64-column block, T split); fp32 partials part[s][16][n].
template <bool VEC>
__global__ __launch_bounds__(256) void rank_grad_kernel(
    const half_t* __restrict__ p, int64_t ldp, const half_t* __restrict__ q, int64_t ldq,
    int64_t t, int64_t n, float q_scale, float* __restrict__ part, int64_t splits,
    int64_t tchunk) {
  __shared__ __attribute__((aligned(16))) half_t sq[4][64 * 64];
  __shared__ __attribute__((aligned(16))) half_t sp[4][kRank * kGradLd];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t nblocks = cdiv(n, 64);
  const int64_t item = (int64_t)blockIdx.x * 4 + wave;
  if (item >= nblocks * splits) return;  // no block-wide barrier below: waves are independent
  const int64_t nb = item % nblocks;
  const int64_t s = item / nblocks;
  const int64_t n0 = nb * 64;
  const int64_t send = (s + 1) * tchunk < t ? (s + 1) * tchunk : t;
  float4v acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = float4v{0.f, 0.f, 0.f, 0.f};
  for (int64_t t0 = s * tchunk; t0 < send; t0 += kGradChunk) {
    const int64_t tend = t0 + kGradChunk < send ? t0 + kGradChunk : send;
    grad_chunk<VEC>(p, ldp, q, ldq, n, q_scale, n0, lane, t0, tend, sq[wave], sp[wave], acc);
  }
  // lane holds C[r' = 4*(lane/16) + j][n0 + 16c + lane%16]
  const int r = lane & 15;
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

// One-launch form: workgroup = one 64-column block, blockDim.x / 64 waves;
// wave w takes the 64-t chunks w, w + waves, ...; the waves' sums are added in
// wave order through LDS and rounded once to fp16, stored [16][n] or [n][16].
constexpr int kColWaves = 8;

template <bool VEC>
__global__ __launch_bounds__(kColWaves * 64) void rank_grad_cols_kernel(
    const half_t* __restrict__ p, int64_t ldp, const half_t* __restrict__ q, int64_t ldq,
    int64_t t, int64_t n, float q_scale, int transpose, half_t* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) half_t sq[kColWaves][64 * 64];
  __shared__ __attribute__((aligned(16))) half_t sp[kColWaves][kRank * kGradLd];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  const int64_t n0 = (int64_t)blockIdx.x * 64;
  float4v acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = float4v{0.f, 0.f, 0.f, 0.f};
  for (int64_t t0 = (int64_t)wave * kGradChunk; t0 < t; t0 += (int64_t)waves * kGradChunk) {
    const int64_t tend = t0 + kGradChunk < t ? t0 + kGradChunk : t;
    grad_chunk<VEC>(p, ldp, q, ldq, n, q_scale, n0, lane, t0, tend, sq[wave], sp[wave], acc);
  }
  // The Q tiles are dead once every wave has passed this barrier; their first
  // 32 KiB hold the waves' 16x64 sums.
  __syncthreads();
  float4v* red = reinterpret_cast<float4v*>(&sq[0][0]);
#pragma unroll
  for (int c = 0; c < 4; ++c) red[(wave * 4 + c) * 64 + lane] = acc[c];
  __syncthreads();
  if (wave != 0) return;
  const int r = lane & 15;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float4v v = red[c * 64 + lane];
    for (int w2 = 1; w2 < waves; ++w2) v += red[(w2 * 4 + c) * 64 + lane];
    const int64_t col = n0 + c * 16 + r;
    if (col >= n) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int rr = (lane >> 4) * 4 + j;
      out[transpose ? col * kRank + rr : rr * n + col] = f32_to_f16(v[j]);
    }
  }
}

// Sum of part[s * stride + i] over s in split order; eight loads in flight.
__device__ __forceinline__ float sum_splits(const float* __restrict__ part, int64_t stride,
                                            int64_t i, int64_t splits) {
  float acc = 0.0f;
  int64_t s = 0;
  for (; s + 8 <= splits; s += 8) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = part[(s + j) * stride + i];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += v[j];
  }
  for (; s < splits; ++s) acc += part[s * stride + i];
  return acc;
}

// out[m][r] (project) = fp16(sum_s part[s][m][r]); out row stride 16.
__global__ __launch_bounds__(256) void rank_project_reduce_kernel(const float* __restrict__ part,
                                                                  int64_t m, int64_t splits,
                                                                  half_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= m * kRank) return;
  out[i] = f32_to_f16(sum_splits(part, m * kRank, i, splits));
}

// grad: out = fp16(sum_s part[s][r][c]) stored [16][n] (transpose = 0) or [n][16].
// A workgroup reduces a 16-rank x 16-column block: thread (r, c) reads a
// 64-byte run per rank row; the transposed store goes through LDS so that the
// block writes one contiguous 512-byte run.
__global__ __launch_bounds__(256) void rank_grad_reduce_kernel(const float* __restrict__ part,
                                                               int64_t n, int64_t splits,
                                                               int transpose,
                                                               half_t* __restrict__ out) {
  __shared__ half_t sh[kRank][kRank + 1];
  const int rr = threadIdx.x >> 4;
  const int cl = threadIdx.x & 15;
  const int64_t c0 = (int64_t)blockIdx.x * kRank;
  const int64_t c = c0 + cl;
  const half_t v = c < n ? f32_to_f16(sum_splits(part + rr * n, kRank * n, c, splits))
                         : (half_t)0.0f;
  if (!transpose) {
    if (c < n) out[rr * n + c] = v;
    return;
  }
  sh[cl][rr] = v;
  __syncthreads();
  const int cw = threadIdx.x >> 4;  // column within the block
  const int rw = threadIdx.x & 15;  // rank
  if (c0 + cw < n) out[(c0 + cw) * kRank + rw] = sh[cw][rw];
}

// The one-launch forms are used while they give at least this many
// workgroups, or when the reduction is short enough that a few workgroups
// finish it in a couple of memory round trips (K <= 16 x 256 for project,
// T <= 8 x 8 x 64 for grad); otherwise the split form spreads the reduction.
constexpr int64_t kMinRowBlocks = 32;
constexpr int64_t kMinColBlocks = 32;

// Chunk length along the reduced dimension: a multiple of `unit`, long enough
// that at most kMaxSplits chunks cover `len`.
static int64_t pick_chunk(int64_t len, int64_t unit) {
  const int64_t per = cdiv(len > 0 ? len : 1, kMaxSplits);
  return cdiv(per, unit) * unit;
}

static bool al16(const void* p, int64_t ld) {
  return reinterpret_cast<uintptr_t>(p) % 16 == 0 && ld % 8 == 0;
}

}  // namespace ss

using namespace ss;

extern "C" size_t ss_lora_workspace_size(int64_t rows, int64_t cols) {
  // fp32 partials of either kernel for a [rows x 16] or [16 x cols] result:
  // at most kMaxSplits chunks of the reduced dimension.
  const int64_t m = rows > cols ? rows : cols;
  return (size_t)(kMaxSplits * (m > 0 ? m : 1) * kRank) * sizeof(float) + 256;
}

extern "C" int ss_lora_project(const uint16_t* a, int64_t lda, int64_t m, int64_t k,
                               const uint16_t* w, int64_t ldw, int w_kr, int scale_a,
                               float a_scale, uint16_t* out, void* workspace,
                               size_t workspace_bytes, void* stream) {
  const char* fn = "ss_lora_project";
  SS_CHECK_ARG(m >= 0 && k >= 0, "%s: negative size", fn);
  if (m == 0) return SS_OK;
  SS_CHECK_ARG(a && w && out, "%s: null pointer", fn);
  SS_CHECK_ARG(lda >= k && ldw >= (w_kr ? kRank : k), "%s: leading dimension too small", fn);
  const int64_t mblocks = cdiv(m, 16);
  hipStream_t s = (hipStream_t)stream;
  // Vector loads need 16-byte aligned rows of both operands and K % 8 == 0.
  const bool vec = al16(a, lda) && al16(w, ldw) && k % 8 == 0;
  if (mblocks >= kMinRowBlocks || k <= kRowWaves * kProjChunk) {
    // One launch: a workgroup per 16-row block, up to 16 waves over K.
    const int64_t chunks = cdiv(k > 0 ? k : 1, kProjChunk);
    const int waves = (int)(chunks < kRowWaves ? chunks : kRowWaves);
    auto kern = vec ? rank_project_rows_kernel<true> : rank_project_rows_kernel<false>;
    hipLaunchKernelGGL(kern, dim3((unsigned)mblocks), dim3(64 * waves), 0, s,
                       reinterpret_cast<const half_t*>(a), lda, m, k,
                       reinterpret_cast<const half_t*>(w), ldw, w_kr, scale_a ? a_scale : 1.0f,
                       reinterpret_cast<half_t*>(out));
    SS_CHECK_LAUNCH("rank_project_rows_kernel");
    return SS_OK;
  }
  SS_CHECK_ARG(workspace, "%s: null workspace", fn);
  const int64_t kchunk = pick_chunk(k, kProjChunk);
  const int64_t splits = cdiv(k > 0 ? k : 1, kchunk);
  SS_CHECK_ARG((size_t)(splits * m * kRank) * sizeof(float) <= workspace_bytes,
               "%s: workspace too small", fn);
  float* part = reinterpret_cast<float*>(workspace);
  const int64_t waves = mblocks * splits;
  auto kern = vec ? rank_project_kernel<true> : rank_project_kernel<false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(waves, 4)), dim3(256), 0, s,
                     reinterpret_cast<const half_t*>(a), lda, m, k,
                     reinterpret_cast<const half_t*>(w), ldw, w_kr, scale_a ? a_scale : 1.0f,
                     part, splits, kchunk);
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
  SS_CHECK_ARG(out && (t == 0 || (p && q)), "%s: null pointer", fn);
  SS_CHECK_ARG(t == 0 || (ldp >= kRank && ldq >= n), "%s: leading dimension too small", fn);
  const int64_t nblocks = cdiv(n, 64);
  hipStream_t s = (hipStream_t)stream;
  // Vector loads need 16-byte aligned rows of P and Q and N % 8 == 0.
  const bool vec = al16(q, ldq) && al16(p, ldp) && n % 8 == 0;
  if (nblocks >= kMinColBlocks || t <= kColWaves * kGradChunk * 8) {
    // One launch: a workgroup per 64-column block, up to 8 waves over T.
    const int64_t chunks = cdiv(t > 0 ? t : 1, kGradChunk);
    const int waves = (int)(chunks < kColWaves ? chunks : kColWaves);
    auto kern = vec ? rank_grad_cols_kernel<true> : rank_grad_cols_kernel<false>;
    hipLaunchKernelGGL(kern, dim3((unsigned)nblocks), dim3(64 * waves), 0, s,
                       reinterpret_cast<const half_t*>(p), ldp,
                       reinterpret_cast<const half_t*>(q), ldq, t, n,
                       scale_q ? q_scale : 1.0f, transpose, reinterpret_cast<half_t*>(out));
    SS_CHECK_LAUNCH("rank_grad_cols_kernel");
    return SS_OK;
  }
  SS_CHECK_ARG(workspace, "%s: null workspace", fn);
  const int64_t tchunk = pick_chunk(t, kGradChunk);
  const int64_t splits = t > 0 ? cdiv(t, tchunk) : 1;
  SS_CHECK_ARG((size_t)(splits * n * kRank) * sizeof(float) <= workspace_bytes,
               "%s: workspace too small", fn);
  float* part = reinterpret_cast<float*>(workspace);
  const int64_t waves = nblocks * splits;
  auto kern = vec ? rank_grad_kernel<true> : rank_grad_kernel<false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(waves, 4)), dim3(256), 0, s,
                     reinterpret_cast<const half_t*>(p), ldp, reinterpret_cast<const half_t*>(q),
                     ldq, t, n, scale_q ? q_scale : 1.0f, part, splits, tchunk);
  SS_CHECK_LAUNCH("rank_grad_kernel");
  hipLaunchKernelGGL(rank_grad_reduce_kernel, dim3((unsigned)cdiv(n, kRank)), dim3(256), 0,
                     s, part, n, splits, transpose, reinterpret_cast<half_t*>(out));
  SS_CHECK_LAUNCH("rank_grad_reduce_kernel");
  return SS_OK;
}
