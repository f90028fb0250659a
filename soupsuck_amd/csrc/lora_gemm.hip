// Rank-16 products of the LoRA branch on MFMA (A10/A12).
//
// Reference: solution/lora.py:151-163 (Z = X.A^T, L = Z.B^T under fp16
// autocast) and solution/lora_pair.py:52-65 (dZ = dL.B, dB = dL^T.Z,
// dA = dZ^T.X).  With rank r = 16 these are "skinny" GEMMs: one operand is
// [T, K] or [T, N] (read once from HBM), the other 16 x K.  They are
// HBM-bound and, at training shapes (T ~ 1000), short: launch latency and
// memory round trips are most of their time.  Each op is one launch over
// (output block, reduction split) workgroups sized so that each wave streams
// about one chunk of the reduced dimension (one memory round trip); the
// waves of a workgroup add their sums through LDS, and when the reduction is
// split over several workgroups the last of them to arrive (a per-block
// arrival counter) adds the splits' fp32 sums in split order -- the same sum
// whichever arrives last -- and stores the fp16 result.  The exchange goes
// through device-scope stores and loads (global_store/load sc1: coherent
// across the XCDs' separate L2s, no L2-wide fence), which suits its size
// (1 KiB or 4 KiB per workgroup).  The counters live at the start of the
// caller's workspace: zero on entry, zero again on return.
//
// rank_project:  C[M, 16] = A[M, K] . W,  W(k, r) = w_kr ? w[k*ldw + r] : w[r*ldw + k],
//                A optionally replaced by fp16(A * a_scale) (dL = fp16(g * s)).
//                Workgroup per (16-row block, K split); A rows come straight
//                from global memory into MFMA registers (16 B per lane), W is
//                staged per wave in LDS.
// rank_grad:     C[16, N] = P[T, 16]^T . Q[T, N] (Q optionally fp16(Q * q_scale)),
//                stored [16][N] or transposed [N][16].  Workgroup per
//                (64-column block, T split); Q tiles are loaded coalesced
//                (128 B per row) and transposed through LDS.

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
// round trip.  kMaxSplits bounds the splits of one output block (and the
// fp32 exchange area).
constexpr int kProjChunk = 256;  // k per rank_project wave: 8 MFMA steps of 32
constexpr int kGradChunk = 64;   // t per rank_grad step: 2 MFMA steps of 32
constexpr int kMaxSplits = 16;
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

// Device-scope relaxed accesses for the cross-workgroup exchange of split
// sums (see the header comment).
__device__ __forceinline__ void store_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split exchange of wave 0 of a workgroup that holds `vals` fp32 sums per
// lane for output block `blk`, split `s` of `splits`: returns true in the
// workgroup that arrives last, whose `vals` then hold the sum over all
// splits in split order.  part: [blocks][splits][vals x 64] fp32;
// counters[blk] counts arrivals and is reset by the last arrival.
template <int VALS>
__device__ __forceinline__ bool finish_splits(float (&vals)[VALS], float* __restrict__ part,
                                              int* __restrict__ counters, int64_t blk,
                                              int64_t s, int64_t splits, int lane) {
  float* base = part + blk * splits * (VALS * 64);
#pragma unroll
  for (int v = 0; v < VALS; ++v) store_dev(base + s * (VALS * 64) + v * 64 + lane, vals[v]);
  // This wave's stores are complete before it counts itself.
  __builtin_amdgcn_s_waitcnt(0);
  int seen = 0;
  if (lane == 0)
    seen = __hip_atomic_fetch_add(counters + blk, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  seen = __shfl(seen, 0, kWave);
  if (seen != (int)splits - 1) return false;
  float sum[VALS];
#pragma unroll
  for (int v = 0; v < VALS; ++v) sum[v] = 0.0f;
  for (int64_t x = 0; x < splits; ++x) {
#pragma unroll
    for (int v = 0; v < VALS; ++v)
      sum[v] += x == s ? vals[v] : load_dev(base + x * (VALS * 64) + v * 64 + lane);
  }
#pragma unroll
  for (int v = 0; v < VALS; ++v) vals[v] = sum[v];
  if (lane == 0)
    __hip_atomic_store(counters + blk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// Workgroup = (16-row block blockIdx.x, K split blockIdx.y of gridDim.y),
// blockDim.x / 64 waves.  Split s covers the 256-k chunks [s * cps, (s + 1) *
// cps); wave w takes chunks w, w + waves, ... of it.  The waves' sums are
// added in wave order through LDS, the splits' by finish_splits; out row
// stride 16.
constexpr int kRowWaves = 4;

template <bool VEC>
__global__ __launch_bounds__(kRowWaves * 64) void rank_project_kernel(
    const half_t* __restrict__ a, int64_t lda, int64_t m, int64_t k, const half_t* __restrict__ w,
    int64_t ldw, int w_kr, float a_scale, int64_t cps, half_t* __restrict__ out,
    float* __restrict__ part, int* __restrict__ counters) {
  __shared__ __attribute__((aligned(16))) half_t sw[kRowWaves][kRank * kProjLd];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  const int64_t mb = blockIdx.x;
  const int64_t s = blockIdx.y;
  const int64_t splits = gridDim.y;
  const int r = lane & 15;
  const int64_t row = mb * 16 + r;
  const int64_t kb = s * cps * kProjChunk;
  const int64_t ke = kb + cps * kProjChunk < k ? kb + cps * kProjChunk : k;
  float4v acc[2] = {float4v{0.f, 0.f, 0.f, 0.f}, float4v{0.f, 0.f, 0.f, 0.f}};
  for (int64_t kbeg = kb + (int64_t)wave * kProjChunk; kbeg < ke;
       kbeg += (int64_t)waves * kProjChunk) {
    const int64_t kend = kbeg + kProjChunk < ke ? kbeg + kProjChunk : ke;
    project_chunk<VEC>(a, lda, m, w, ldw, w_kr, a_scale, row, lane, kbeg, kend, sw[wave], acc);
  }
  // The per-wave tiles are dead once every wave has passed this barrier;
  // their first 4 KiB hold the waves' 16x16 sums.
  __syncthreads();
  float4v* red = reinterpret_cast<float4v*>(&sw[0][0]);
  red[wave * 64 + lane] = acc[0] + acc[1];
  __syncthreads();
  if (wave != 0) return;
  float4v c = red[lane];
  for (int w2 = 1; w2 < waves; ++w2) c += red[w2 * 64 + lane];
  float vals[4] = {c[0], c[1], c[2], c[3]};
  if (splits > 1 && !finish_splits<4>(vals, part, counters, mb, s, splits, lane)) return;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t mm = mb * 16 + (lane >> 4) * 4 + j;
    if (mm < m) out[mm * kRank + r] = f32_to_f16(vals[j]);
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

// Workgroup = (64-column block blockIdx.x, T split blockIdx.y of gridDim.y),
// blockDim.x / 64 waves.  Split s covers the 64-t chunks [s * cps, (s + 1) *
// cps); wave w takes chunks w, w + waves, ... of it.  The waves' sums are
// added in wave order through LDS, the splits' by finish_splits; the result
// is stored [16][n] or transposed [n][16].
constexpr int kColWaves = 4;

template <bool VEC>
__global__ __launch_bounds__(kColWaves * 64) void rank_grad_kernel(
    const half_t* __restrict__ p, int64_t ldp, const half_t* __restrict__ q, int64_t ldq,
    int64_t t, int64_t n, float q_scale, int64_t cps, int transpose, half_t* __restrict__ out,
    float* __restrict__ part, int* __restrict__ counters) {
  __shared__ __attribute__((aligned(16))) half_t sq[kColWaves][64 * 64];
  __shared__ __attribute__((aligned(16))) half_t sp[kColWaves][kRank * kGradLd];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int waves = blockDim.x >> 6;
  const int64_t nb = blockIdx.x;
  const int64_t s = blockIdx.y;
  const int64_t splits = gridDim.y;
  const int64_t n0 = nb * 64;
  const int64_t tb = s * cps * kGradChunk;
  const int64_t te = tb + cps * kGradChunk < t ? tb + cps * kGradChunk : t;
  float4v acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = float4v{0.f, 0.f, 0.f, 0.f};
  for (int64_t t0 = tb + (int64_t)wave * kGradChunk; t0 < te; t0 += (int64_t)waves * kGradChunk) {
    const int64_t tend = t0 + kGradChunk < te ? t0 + kGradChunk : te;
    grad_chunk<VEC>(p, ldp, q, ldq, n, q_scale, n0, lane, t0, tend, sq[wave], sp[wave], acc);
  }
  // The Q tiles are dead once every wave has passed this barrier; their first
  // 16 KiB hold the waves' 16x64 sums.
  __syncthreads();
  float4v* red = reinterpret_cast<float4v*>(&sq[0][0]);
#pragma unroll
  for (int c = 0; c < 4; ++c) red[(wave * 4 + c) * 64 + lane] = acc[c];
  __syncthreads();
  if (wave != 0) return;
  float vals[16];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float4v v = red[c * 64 + lane];
    for (int w2 = 1; w2 < waves; ++w2) v += red[(w2 * 4 + c) * 64 + lane];
#pragma unroll
    for (int j = 0; j < 4; ++j) vals[c * 4 + j] = v[j];
  }
  if (splits > 1 && !finish_splits<16>(vals, part, counters, nb, s, splits, lane)) return;
  // lane holds C[r' = 4*(lane/16) + j][n0 + 16c + lane%16] in vals[4c + j]
  const int r = lane & 15;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int64_t col = n0 + c * 16 + r;
    if (col >= n) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int rr = (lane >> 4) * 4 + j;
      out[transpose ? col * kRank + rr : rr * n + col] = f32_to_f16(vals[c * 4 + j]);
    }
  }
}

// Split plan: each wave of a split gets one chunk (cps = waves per
// workgroup chunks per split) unless that needs more than kMaxSplits splits.
struct RankPlan {
  int64_t splits, cps;
  int waves;
};

static RankPlan rank_plan(int64_t len, int64_t unit, int max_waves, bool can_split) {
  const int64_t chunks = cdiv(len > 0 ? len : 1, unit);
  RankPlan plan;
  plan.splits = can_split ? cdiv(chunks, max_waves) : 1;
  if (plan.splits > kMaxSplits) plan.splits = kMaxSplits;
  plan.cps = cdiv(chunks, plan.splits);
  plan.splits = cdiv(chunks, plan.cps);
  plan.waves = (int)(plan.cps < max_waves ? plan.cps : max_waves);
  return plan;
}

// Workspace layout: a fixed area of kCounters arrival counters (one int per
// output block; the same for every op and shape, so ops of different shapes
// can share one workspace without one's exchange data landing on another's
// counters), then the fp32 exchange area [blocks][splits][vals x 64].  Ops
// with more output blocks than kCounters do not split.
constexpr int64_t kCounters = 65536;
constexpr size_t kCounterBytes = kCounters * sizeof(int);

static size_t project_bytes(int64_t m) {
  const int64_t blocks = cdiv(m > 0 ? m : 1, 16);
  return kCounterBytes + (size_t)(blocks * kMaxSplits * 4 * 64) * sizeof(float);
}

static size_t grad_bytes(int64_t n) {
  const int64_t blocks = cdiv(n > 0 ? n : 1, 64);
  return kCounterBytes + (size_t)(blocks * kMaxSplits * 16 * 64) * sizeof(float);
}

static bool al16(const void* p, int64_t ld) {
  return reinterpret_cast<uintptr_t>(p) % 16 == 0 && ld % 8 == 0;
}

}  // namespace ss

using namespace ss;

extern "C" size_t ss_lora_workspace_size(int64_t rows, int64_t cols) {
  // Counters and exchange area of either op: project for a [rows x 16]
  // result, grad for a [16 x cols] result.
  const size_t a = project_bytes(rows), b = grad_bytes(cols);
  return a > b ? a : b;
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
  const bool can_split =
      workspace && workspace_bytes >= project_bytes(m) && mblocks <= kCounters;
  const RankPlan plan = rank_plan(k, kProjChunk, kRowWaves, can_split);
  int* counters = reinterpret_cast<int*>(workspace);
  float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
  // Vector loads need 16-byte aligned rows of both operands and K % 8 == 0.
  const bool vec = al16(a, lda) && al16(w, ldw) && k % 8 == 0;
  auto kern = vec ? rank_project_kernel<true> : rank_project_kernel<false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)mblocks, (unsigned)plan.splits), dim3(64 * plan.waves),
                     0, (hipStream_t)stream, reinterpret_cast<const half_t*>(a), lda, m, k,
                     reinterpret_cast<const half_t*>(w), ldw, w_kr, scale_a ? a_scale : 1.0f,
                     plan.cps, reinterpret_cast<half_t*>(out), part, counters);
  SS_CHECK_LAUNCH("rank_project_kernel");
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
  const bool can_split = workspace && workspace_bytes >= grad_bytes(n) && nblocks <= kCounters;
  const RankPlan plan = rank_plan(t, kGradChunk, kColWaves, can_split);
  int* counters = reinterpret_cast<int*>(workspace);
  float* part = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
  // Vector loads need 16-byte aligned rows of P and Q and N % 8 == 0.
  const bool vec = al16(q, ldq) && al16(p, ldp) && n % 8 == 0;
  auto kern = vec ? rank_grad_kernel<true> : rank_grad_kernel<false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)nblocks, (unsigned)plan.splits), dim3(64 * plan.waves),
                     0, (hipStream_t)stream, reinterpret_cast<const half_t*>(p), ldp,
                     reinterpret_cast<const half_t*>(q), ldq, t, n, scale_q ? q_scale : 1.0f,
                     plan.cps, transpose, reinterpret_cast<half_t*>(out), part, counters);
  SS_CHECK_LAUNCH("rank_grad_kernel");
  return SS_OK;
}
