// Block-level bodies of the rank-16 LoRA products (A10/A12), shared by the
// stand-alone kernels of lora_gemm.hip and the fused preparation launch of
// the QLoRA projection (rank products next to the NF4 decode).
//
// Reference: solution/lora.py:151-163 (Z = X.A^T under fp16 autocast) and
// solution/lora_pair.py:52-65 (dZ = dL.B, dB = dL^T.Z, dA = dZ^T.X).
//
// rank_project_block: C[M, 16] = A'[M, K] . W,  W(k, r) = w_kr ? w[k*ldw + r]
//   : w[r*ldw + k], A' = A or fp16(A * a_scale); one (16-row block, K split).
// rank_grad_block: C[16, N] = P[T, 16]^T . Q'[T, N], Q' = Q or fp16(Q * q_scale),
//   stored [16][N] or [N][16]; one (64-column block, T split).
// Both run on blocks of 64 * waves threads (waves past 4 only join the
// barriers) with `smem` of at least kRankProjSmem / kRankGradSmem bytes.
// DROP: A' (project) / Q' (grad) additionally pass through the LoRA dropout
// mask of g.drop (philox.h), for Z and dA of the dropout path.  A split's waves stream one chunk each
// (one memory round trip), add their sums through LDS, and the splits of an
// output block are added by the last workgroup to arrive (finish_splits).
#pragma once

#include "gemm.h"

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
template <bool VEC, bool DROP>
__device__ __forceinline__ void project_chunk(const half_t* __restrict__ a, int64_t lda,
                                              int64_t m, const half_t* __restrict__ w,
                                              int64_t ldw, int w_kr, float a_scale, int64_t row,
                                              int lane, int64_t kbeg, int64_t kend, half_t* tile,
                                              float4v (&acc)[2], const DropoutArgs& drop,
                                              int64_t cols) {
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
  if constexpr (DROP) {
    // Dropout of A (the LoRA input X): the keep bits of the lane's 8
    // consecutive elements (row, k .. k + 7); rows past m and columns past
    // kend hold zeros and are never stored, so their bits do not matter.
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const int64_t k = kbeg + st * 32 + kq;
      const uint32_t bits = row < m && k < kend ? keep8(drop, row * cols + k) : 0u;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        av[st][i] = f32_to_f16(dropped(drop, (float)av[st][i] * a_scale, (bits >> i) & 1u));
    }
  } else {
#pragma unroll
    for (int st = 0; st < 8; ++st)
#pragma unroll
      for (int i = 0; i < 8; ++i) av[st][i] = f32_to_f16((float)av[st][i] * a_scale);
  }
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
  // Ordering without cache maintenance: the compiler-only fences keep the
  // device-scope stores above the count and the device-scope loads below it
  // (the compiler may otherwise reorder relaxed accesses to different
  // addresses); the wait makes the stores complete in memory before the
  // count is issued, and the loads are issued only after the counted value
  // has returned (they depend on it through the branch).  A release/acquire
  // atomic would add whole-L2 writeback and invalidate instructions.
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  int seen = 0;
  if (lane == 0)
    seen = __hip_atomic_fetch_add(counters + blk, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  seen = __shfl(seen, 0, kWave);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
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

// One 64-t chunk [t0, tend) of a 64-column block at n0: acc[c] += P[chunk, :]^T .
// Q'[chunk, n0 + 16c .. +15], Q transposed through the wave's LDS tile.
template <bool VEC, bool DROP>
__device__ __forceinline__ void grad_chunk(const half_t* __restrict__ p, int64_t ldp,
                                           const half_t* __restrict__ q, int64_t ldq, int64_t n,
                                           float q_scale, int64_t n0, int lane, int64_t t0,
                                           int64_t tend, half_t* tile, half_t* ptile,
                                           float4v (&acc)[4], const DropoutArgs& drop) {
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
    // Dropout of Q (the LoRA input X for dA): keep bits of the lane's 8
    // consecutive elements; out-of-range ones are zeros that no sum uses.
    const int64_t t = t0 + tl;
    uint32_t bits = 0xffu;
    if constexpr (DROP) bits = t < tend && n0 + nl < n ? keep8(drop, t * n + n0 + nl) : 0u;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // fp16(q * 1.0) == q for every fp16 value, so "no scaling" is q_scale = 1.
      const float qv = (float)v[it][i] * q_scale;
      tile[qtile_index(nl + i, tl)] = f32_to_f16(DROP ? dropped(drop, qv, (bits >> i) & 1u) : qv);
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

constexpr int kRankMaxWaves = 4;
constexpr int kRankProjSmem = kRankMaxWaves * kRank * kProjLd * 2;
constexpr int kRankGradSmem = kRankMaxWaves * (64 * 64 + kRank * kGradLd) * 2;

// Split s of 16-row block mb: the 256-k chunks [s * cps, (s + 1) * cps);
// wave w takes chunks w, w + waves, ... of it.  out row stride 16.
template <bool VEC, bool DROP = false>
__device__ __forceinline__ void rank_project_block(const RankProjectArgs& g, int64_t mb,
                                                   int64_t s, unsigned char* smem) {
  half_t (*sw)[kRank * kProjLd] = reinterpret_cast<half_t (*)[kRank * kProjLd]>(smem);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // Waves past kRankMaxWaves (a block shared with a wider kernel) take no
  // chunk but join the barriers.
  const int waves = (int)(blockDim.x >> 6) < kRankMaxWaves ? (int)(blockDim.x >> 6) : kRankMaxWaves;
  const int r = lane & 15;
  const int64_t row = mb * 16 + r;
  const int64_t kb = s * g.cps * kProjChunk;
  const int64_t ke = kb + g.cps * kProjChunk < g.k ? kb + g.cps * kProjChunk : g.k;
  float4v acc[2] = {float4v{0.f, 0.f, 0.f, 0.f}, float4v{0.f, 0.f, 0.f, 0.f}};
  for (int64_t kbeg = kb + (int64_t)wave * kProjChunk; wave < waves && kbeg < ke;
       kbeg += (int64_t)waves * kProjChunk) {
    const int64_t kend = kbeg + kProjChunk < ke ? kbeg + kProjChunk : ke;
    project_chunk<VEC, DROP>(g.a, g.lda, g.m, g.w, g.ldw, g.w_kr, g.a_scale, row, lane, kbeg,
                             kend, sw[wave], acc, g.drop, g.k);
  }
  // The per-wave tiles are dead once every wave has passed this barrier;
  // their first 4 KiB hold the waves' 16x16 sums.
  __syncthreads();
  float4v* red = reinterpret_cast<float4v*>(smem);
  if (wave < waves) red[wave * 64 + lane] = acc[0] + acc[1];
  __syncthreads();
  if (wave != 0) return;
  float4v c = red[lane];
  for (int w2 = 1; w2 < waves; ++w2) c += red[w2 * 64 + lane];
  float vals[4] = {c[0], c[1], c[2], c[3]};
  if (g.splits > 1 && !finish_splits<4>(vals, g.part, g.counters, mb, s, g.splits, lane)) return;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t mm = mb * 16 + (lane >> 4) * 4 + j;
    if (mm < g.m) g.out[mm * kRank + r] = f32_to_f16(vals[j]);
  }
}

// Split s of 64-column block nb: the 64-t chunks [s * cps, (s + 1) * cps);
// wave w takes chunks w, w + waves, ... of it.
template <bool VEC, bool DROP = false>
__device__ __forceinline__ void rank_grad_block(const RankGradArgs& g, int64_t nb, int64_t s,
                                                unsigned char* smem) {
  half_t (*sq)[64 * 64] = reinterpret_cast<half_t (*)[64 * 64]>(smem);
  half_t (*sp)[kRank * kGradLd] = reinterpret_cast<half_t (*)[kRank * kGradLd]>(
      smem + kRankMaxWaves * 64 * 64 * 2);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  // Waves past kRankMaxWaves (a block shared with a wider kernel) take no
  // chunk but join the barriers.
  const int waves = (int)(blockDim.x >> 6) < kRankMaxWaves ? (int)(blockDim.x >> 6) : kRankMaxWaves;
  const int64_t n0 = nb * 64;
  const int64_t tb = s * g.cps * kGradChunk;
  const int64_t te = tb + g.cps * kGradChunk < g.t ? tb + g.cps * kGradChunk : g.t;
  float4v acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = float4v{0.f, 0.f, 0.f, 0.f};
  for (int64_t t0 = tb + (int64_t)wave * kGradChunk; wave < waves && t0 < te;
       t0 += (int64_t)waves * kGradChunk) {
    const int64_t tend = t0 + kGradChunk < te ? t0 + kGradChunk : te;
    grad_chunk<VEC, DROP>(g.p, g.ldp, g.q, g.ldq, g.n, g.q_scale, n0, lane, t0, tend,
                          sq[wave], sp[wave], acc, g.drop);
  }
  // The Q tiles are dead once every wave has passed this barrier; their first
  // 16 KiB hold the waves' 16x64 sums.
  __syncthreads();
  float4v* red = reinterpret_cast<float4v*>(smem);
  if (wave < waves) {
#pragma unroll
    for (int c = 0; c < 4; ++c) red[(wave * 4 + c) * 64 + lane] = acc[c];
  }
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
  if (g.splits > 1 && !finish_splits<16>(vals, g.part, g.counters, nb, s, g.splits, lane)) return;
  // lane holds C[r' = 4*(lane/16) + j][n0 + 16c + lane%16] in vals[4c + j]
  const int r = lane & 15;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int64_t col = n0 + c * 16 + r;
    if (col >= g.n) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int rr = (lane >> 4) * 4 + j;
      g.out[g.transpose ? col * kRank + rr : rr * g.n + col] = f32_to_f16(vals[c * 4 + j]);
    }
  }
}

// Tail block b (0 <= b < p.tail_blocks + p.tail2_blocks) of a GEMM launch:
// a block of p.tail, then of p.tail2.
__device__ __forceinline__ void run_tail_block(const GemmParams& p, int64_t b,
                                               unsigned char* smem) {
  const bool first = b < p.tail_blocks;
  const RankGradArgs& g = first ? p.tail : p.tail2;
  if (!first) b -= p.tail_blocks;
  const int64_t nblocks = cdiv(g.n, 64);
  rank_grad_block<true>(g, b % nblocks, b / nblocks, smem);
}

// Host plans and workspace layout of the rank-16 products.
//
// Rank workspace (zero-filled once by its owner): kCounterBytes of arrival
// counters -- project counters at [0, kCounters / 2), grad counters at
// [kCounters / 2, kCounters), so one project and one grad can run in the same
// launch -- then the project exchange area [mblocks][splits][4 x 64] fp32,
// then the grad exchange area [nblocks][splits][16 x 64] fp32.  Every op
// leaves its counters zero.  Ops with more output blocks than a counter
// region holds do not split.
constexpr int64_t kCounters = 65536;
constexpr size_t kCounterBytes = kCounters * sizeof(int);

struct RankPlan {
  int64_t splits, cps;
  int waves;
};

// Each wave of a split gets one chunk unless that needs more than kMaxSplits
// splits.
inline RankPlan rank_plan(int64_t len, int64_t unit, bool can_split) {
  const int64_t chunks = cdiv(len > 0 ? len : 1, unit);
  RankPlan plan;
  plan.splits = can_split ? cdiv(chunks, kRankMaxWaves) : 1;
  if (plan.splits > kMaxSplits) plan.splits = kMaxSplits;
  plan.cps = cdiv(chunks, plan.splits);
  plan.splits = cdiv(chunks, plan.cps);
  plan.waves = (int)(plan.cps < kRankMaxWaves ? plan.cps : kRankMaxWaves);
  return plan;
}

inline size_t rank_project_part_bytes(int64_t m) {
  return (size_t)(cdiv(m > 0 ? m : 1, 16) * kMaxSplits * 4 * 64) * sizeof(float);
}
inline size_t rank_grad_part_bytes(int64_t n) {
  return (size_t)(cdiv(n > 0 ? n : 1, 64) * kMaxSplits * 16 * 64) * sizeof(float);
}

// Jobs of one preparation launch (lora_gemm.hip qlora_prep_kernel): an
// optional project, an optional grad and an optional NF4 decode of W [rows,
// cols] (row-major into dec_out, or transposed).  proj_blocks / grad_blocks
// 0 for an absent job.
enum DecodeKind { kDecodeNone = 0, kDecodeRows = 1, kDecodeTransposed = 2 };
struct PrepJobs {
  RankProjectArgs proj;
  int64_t proj_blocks;
  RankGradArgs grad;
  int64_t grad_blocks;
  int dec_kind;
  Nf4View dec_w;
  half_t* dec_out;
  int64_t dec_rows, dec_cols, dec_blocks;
};
// vp / vg: the project / grad operands allow 16-byte vector loads.
int launch_prep(PrepJobs& pj, bool vp, bool vg, hipStream_t stream);

// Fill args for a project (grad) over the rank workspace `ws`; `rows` is the
// project row count of the same call (0 when there is none), which places
// the grad exchange area after the project's.  Returns the number of
// workgroups (output blocks x splits).
int64_t rank_project_setup(RankProjectArgs& g, const void* a, int64_t lda, int64_t m, int64_t k,
                           const void* w, int64_t ldw, int w_kr, float a_scale, void* out,
                           void* ws, size_t ws_bytes, int64_t rows, bool& vec);
// part_offset / counter_offset: extra bytes before the grad's exchange area
// and extra grad counters to skip, so that two grads of one launch (the
// backward's dB and dA tails) use disjoint areas.
int64_t rank_grad_setup(RankGradArgs& g, const void* p, int64_t ldp, const void* q, int64_t ldq,
                        int64_t t, int64_t n, float q_scale, int transpose, void* out, void* ws,
                        size_t ws_bytes, int64_t rows, bool& vec, size_t part_offset = 0,
                        int64_t counter_offset = 0);

}  // namespace ss

namespace ss {

// LoRA dropout (dropout.hip): the kernels' view of (seed, p), and the
// backward's tail launch -- dA = fp16(dZ^T . fp16(drop(X))) and the masked
// rank-16 term added to dX (which the dX GEMM computed without it).  The tail
// needs 16-byte aligned dZ, X, A and dX rows and k % 8 == 0
// (SS_ERR_UNSUPPORTED otherwise, before any launch).
DropoutArgs dropout_args(uint64_t seed, float p);
int launch_dropout_tail(const half_t* dz, const half_t* x, int64_t ldx, const half_t* lora_a,
                        int64_t t, int64_t k, half_t* dx, int64_t lddx, half_t* da,
                        const DropoutArgs& drop, void* rank_ws, size_t rank_ws_bytes,
                        hipStream_t stream);

}  // namespace ss
