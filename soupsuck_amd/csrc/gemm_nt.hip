// Dense NT GEMM main loop for gfx950: C[M,N] = alpha * A[M,K] . B[N,K]^T with
// both operands K-contiguous fp16 and fp32 accumulation on
// v_mfma_f32_32x32x16_f16.  This is the hot loop of the decode-first NF4
// projections (X . Wdec^T forward, dY . (Wdec^T)^T backward) and of the dense
// NT products; the epilogues (bias, LoRA add, rank-16 update, beta) are the
// ones of gemm.hip.
//
// Operand layouts, configurations and the epilogue: nt_core.h.
//
// Per stage a wave runs BK / 16 MFMA k-steps; fragments are double buffered
// so the reads of k-step kk+1 overlap the MFMAs of kk.  One s_barrier per
// stage sits before the last k-step: by then every wave has read all its
// fragments of stage kt (lgkmcnt(0)), so buffer kt % STAGES is refilled with
// stage kt + STAGES right after it, and stage kt+1 (waited for with vmcnt
// before the barrier) is read while the last MFMAs of stage kt run; the
// refill DMAs are interleaved between those MFMAs.
//
// The DMA is issued from inline asm.  The compiler does not know which LDS
// buffer an outstanding LDS DMA writes, and would wait for all of them
// (vmcnt(0)) before every LDS read, draining the pipeline; the waits are
// explicit instead.

#include "tuning.h"
#include <stdlib.h>

#include "nt_core.h"

namespace ss {
namespace {

// acc += A[m0.., kbeg .. kbeg+klen) . B[n0.., same k]^T for one output tile:
// the pipelined direct-to-LDS main loop.  All of the workgroup's LDS DMAs
// have completed when it returns; the caller puts a barrier between two calls
// (the last k-step's LDS reads of one call and the first DMAs of the next).
// Operand sources of one workgroup's tile (both main loops): per-lane DMA
// sources as 32-bit byte offsets from the per-stage operand base, and the
// per-stage advance of that base.  Rows past M / N (row-major operands) or
// chunks past M / N (K-major operands, L bits 0 / 1) are clamped to the last
// valid ones: they only feed accumulator rows / columns that are never stored.
template <class C, int L>
struct NtSources {
  static constexpr bool AT = (L & 1) != 0, BT = (L & 2) != 0;
  uint32_t a_off[C::kDmaA];
  uint32_t b_off[C::kDmaB];
  const half_t* a_base;
  const half_t* b_base;
  int64_t a_step, b_step;  // elements per stage

  __device__ __forceinline__ NtSources(const GemmParams& p, int64_t m0, int64_t n0, int64_t kbeg,
                                       int wave, int lane) {
    a_base = AT ? p.A + kbeg * p.lda : p.A + kbeg;
    b_base = BT ? p.B + kbeg * p.ldb : p.B + kbeg;
    a_step = AT ? (int64_t)C::BK * p.lda : C::BK;
    b_step = BT ? (int64_t)C::BK * p.ldb : C::BK;
#pragma unroll
    for (int j = 0; j < C::kDmaA; ++j) {
      int row, chunk;
      if constexpr (AT) {
        dma_source_t<C::BM>(wave * C::kDmaA + j, lane, row, chunk);
        const int64_t col = m0 + 8 * chunk <= p.M - 8 ? m0 + 8 * chunk : p.M - 8;
        a_off[j] = (uint32_t)((row * p.lda + col) * 2);
      } else {
        dma_source<C::BK>(wave * C::kDmaA + j, lane, row, chunk);
        const int64_t gr = m0 + row < p.M ? m0 + row : p.M - 1;
        a_off[j] = (uint32_t)((gr * p.lda + chunk * 8) * 2);
      }
    }
#pragma unroll
    for (int j = 0; j < C::kDmaB; ++j) {
      int row, chunk;
      if constexpr (BT) {
        dma_source_t<C::BN>(wave * C::kDmaB + j, lane, row, chunk);
        const int64_t col = n0 + 8 * chunk <= p.N - 8 ? n0 + 8 * chunk : p.N - 8;
        b_off[j] = (uint32_t)((row * p.ldb + col) * 2);
      } else {
        dma_source<C::BK>(wave * C::kDmaB + j, lane, row, chunk);
        const int64_t gr = n0 + row < p.N ? n0 + row : p.N - 1;
        b_off[j] = (uint32_t)((gr * p.ldb + chunk * 8) * 2);
      }
    }
  }
};

// Fragment offsets of one wave (both main loops): for a row-major operand the
// lane's offset per k-step plus the 32-row group stride; for a K-major one the
// offset of every (k-step, block) pair, read with read_frag_t.
template <class C, int L>
struct NtFrags {
  static constexpr bool AT = (L & 1) != 0, BT = (L & 2) != 0;
  static constexpr int kGroupBytes = 32 * C::BK * 2;
  int row_off[C::KK];
  int a_off[AT ? C::KK : 1][AT ? C::FM : 1];
  int b_off[BT ? C::KK : 1][BT ? C::FN : 1];
  int a_base, b_base;

  __device__ __forceinline__ NtFrags(int lane, int wm, int wn) {
#pragma unroll
    for (int kk = 0; kk < C::KK; ++kk) row_off[kk] = frag_offset<C::BK>(lane, kk);
    a_base = (wm * C::WM / 32) * kGroupBytes;
    b_base = C::kTileA + (wn * C::WN / 32) * kGroupBytes;
    if constexpr (AT) {
#pragma unroll
      for (int kk = 0; kk < C::KK; ++kk)
#pragma unroll
        for (int i = 0; i < C::FM; ++i)
          a_off[kk][i] = frag_offset_t<C::BM>(lane, kk, wm * C::WM + 32 * i);
    }
    if constexpr (BT) {
#pragma unroll
      for (int kk = 0; kk < C::KK; ++kk)
#pragma unroll
        for (int j = 0; j < C::FN; ++j)
          b_off[kk][j] = C::kTileA + frag_offset_t<C::BN>(lane, kk, wn * C::WN + 32 * j);
    }
  }
  __device__ __forceinline__ half8 a(const unsigned char* stage, int kk, int i) const {
    if constexpr (AT)
      return read_frag_t(stage + a_off[kk][i], C::BM * 2);
    else
      return *reinterpret_cast<const half8*>(stage + a_base + row_off[kk] + i * kGroupBytes);
  }
  __device__ __forceinline__ half8 b(const unsigned char* stage, int kk, int j) const {
    if constexpr (BT)
      return read_frag_t(stage + b_off[kk][j], C::BN * 2);
    else
      return *reinterpret_cast<const half8*>(stage + b_base + row_off[kk] + j * kGroupBytes);
  }
};

template <class C, int L = 0>
__device__ __forceinline__ void nt_mainloop(const GemmParams& p, int64_t m0, int64_t n0,
                                            int64_t kbeg, int64_t klen, unsigned char* smem,
                                            NtAcc<C>& acc) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int wm = wave / C::kWavesN;
  const int wn = wave % C::kWavesN;
  const uint32_t lds0 = lds_address(smem);
  const NtSources<C, L> src(p, m0, n0, kbeg, wave, lane);
  const uint32_t lds_a = __builtin_amdgcn_readfirstlane(lds0 + wave * C::kDmaA * 1024);
  const uint32_t lds_b = __builtin_amdgcn_readfirstlane(lds0 + C::kTileA + wave * C::kDmaB * 1024);
  const NtFrags<C, L> frags(lane, wm, wn);

  auto dma_one = [&](int64_t kt, int stage, int idx) {
    if (idx < C::kDmaA) {
      dma16(src.a_off[idx], src.a_base + kt * src.a_step,
            lds_a + stage * C::kStageBytes + idx * 1024);
    } else {
      const int j = idx - C::kDmaA;
      dma16(src.b_off[j], src.b_base + kt * src.b_step, lds_b + stage * C::kStageBytes + j * 1024);
    }
  };
  auto read_frags = [&](int64_t kt, int kk, half8 (&af)[C::FM], half8 (&bf)[C::FN]) {
    const unsigned char* base = smem + (kt % C::STAGES) * C::kStageBytes;
#pragma unroll
    for (int i = 0; i < C::FM; ++i) af[i] = frags.a(base, kk, i);
#pragma unroll
    for (int j = 0; j < C::FN; ++j) bf[j] = frags.b(base, kk, j);
  };
  // MFMA phases raise the wave's issue priority (s_setprio 1), so a SIMD's
  // other wave, in its load / LDS phase, does not delay them (measured +7 % at
  // 8192^3, neutral at the layer shapes).
  auto mfma_block = [&](const half8 (&af)[C::FM], const half8 (&bf)[C::FN]) {
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
      for (int j = 0; j < C::FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    __builtin_amdgcn_s_setprio(0);
  };

  constexpr int kS = C::STAGES;
  constexpr int kMfma = C::FM * C::FN;
  const int64_t ktiles = klen / C::BK;
  half8 fa[2][C::FM], fb[2][C::FN];
#pragma unroll
  for (int s = 0; s < kS; ++s)
    if (s < ktiles)
#pragma unroll
      for (int idx = 0; idx < C::kDma; ++idx) dma_one(s, s, idx);
  if (ktiles > 0) {
    wait_stages<C::kDma, kS - 1>((ktiles < kS ? ktiles : kS) - 1);
    asm volatile("s_barrier" ::: "memory");
    read_frags(0, 0, fa[0], fb[0]);
  }
  for (int64_t kt = 0; kt < ktiles; ++kt) {
#pragma unroll
    for (int kk = 0; kk + 1 < C::KK; ++kk) {
      read_frags(kt, kk + 1, fa[(kk + 1) & 1], fb[(kk + 1) & 1]);
      mfma_block(fa[kk & 1], fb[kk & 1]);
    }
    constexpr int kLast = (C::KK - 1) & 1;
    const bool more = kt + 1 < ktiles;
    const bool refill = kt + kS < ktiles;
    if (more) {
      // Stages requested so far: 0 .. min(kt + kS - 1, ktiles - 1); stage kt+1
      // must have landed.  lgkmcnt(0): this wave's reads of stage kt are done,
      // so buffer kt % kS may be refilled once every wave passed the barrier.
      const int64_t last = kt + kS - 1 < ktiles - 1 ? kt + kS - 1 : ktiles - 1;
      wait_stages<C::kDma, kS - 2>(last - (kt + 1));
      __builtin_amdgcn_s_waitcnt(0xC07F);
      asm volatile("s_barrier" ::: "memory");
    }
    const int refill_stage = (int)(kt % kS);
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int idx = 0; idx < kMfma; ++idx) {
      if (idx == kMfma / 2 && more) read_frags(kt + 1, 0, fa[0], fb[0]);
      acc[idx / C::FN][idx % C::FN] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
          fa[kLast][idx / C::FN], fb[kLast][idx % C::FN], acc[idx / C::FN][idx % C::FN], 0, 0,
          0);
      if (refill) {
#pragma unroll
        for (int d = idx * C::kDma / kMfma; d < (idx + 1) * C::kDma / kMfma; ++d)
          dma_one(kt + kS, refill_stage, d);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int d = kMfma < C::kDma ? kMfma * (C::kDma / kMfma) : C::kDma; d < C::kDma; ++d)
      if (refill) dma_one(kt + kS, refill_stage, d);
  }
}

// Ping-pong main loop of the 8-wave configurations (two waves per SIMD:
// wave w and w + 4).  Run in lockstep, the two waves of a SIMD issue their
// MFMAs, LDS reads and barrier waits at the same time, and the MFMA pipe
// idles while both wait.  Here every wave runs the same body per stage kt,
//   read the fragments of stage kt, issue its DMAs of stage kt - 1 + STAGES,
//   wait for its DMAs of stage kt + 1, barrier, the 16 MFMAs of stage kt,
//   barrier,
// but waves 4-7 pass one extra barrier before the first stage and waves 0-3
// one after the last.  The barrier instances then pair each MFMA phase of
// one group with a read phase of the other: on every SIMD one wave computes
// while the other loads.  Stage kt's buffer is read by waves 0-3 in phase 2kt
// and by waves 4-7 in phase 2kt + 1, and refilled (stage kt + STAGES) in read
// phases from 2kt + 2 on; each wave's wait for its DMAs of stage kt + 1
// precedes a barrier that ends before either group reads that stage.  The
// MFMAs of every accumulator run in the order of nt_mainloop, so the results
// are the same bit for bit.
template <class C, int L = 0>
__device__ __forceinline__ void nt_mainloop_pp(const GemmParams& p, int64_t m0, int64_t n0,
                                               int64_t kbeg, int64_t klen, unsigned char* smem,
                                               NtAcc<C>& acc) {
  static_assert(C::kWaves == 8 && C::KK == 2, "ping-pong: 8 waves, two k-steps per stage");
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // uniform: scalar branches
  const int wm = wave / C::kWavesN;
  const int wn = wave % C::kWavesN;
  const bool late = wave >= 4;  // SIMD partner of wave - 4
  const uint32_t lds0 = lds_address(smem);
  const NtSources<C, L> src(p, m0, n0, kbeg, wave, lane);
  const uint32_t lds_a = __builtin_amdgcn_readfirstlane(lds0 + wave * C::kDmaA * 1024);
  const uint32_t lds_b = __builtin_amdgcn_readfirstlane(lds0 + C::kTileA + wave * C::kDmaB * 1024);
  const NtFrags<C, L> frags(lane, wm, wn);

  constexpr int kS = C::STAGES;
  const int64_t ktiles = klen / C::BK;
  auto issue_stage = [&](int64_t kt) {
    if (kt >= ktiles) return;
    const int stage = (int)(kt % kS);
#pragma unroll
    for (int j = 0; j < C::kDmaA; ++j)
      dma16(src.a_off[j], src.a_base + kt * src.a_step, lds_a + stage * C::kStageBytes + j * 1024);
#pragma unroll
    for (int j = 0; j < C::kDmaB; ++j)
      dma16(src.b_off[j], src.b_base + kt * src.b_step, lds_b + stage * C::kStageBytes + j * 1024);
  };
  auto barrier = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

#pragma unroll
  for (int st = 0; st < kS; ++st) issue_stage(st);
  if (ktiles <= 0) return;
  wait_stages<C::kDma, kS - 1>((ktiles < kS ? ktiles : kS) - 1);
  barrier();  // stage 0 is in LDS
  if (late) barrier();
  for (int64_t kt = 0; kt < ktiles; ++kt) {
    half8 fa[2][C::FM], fb[2][C::FN];
    const unsigned char* base = smem + (kt % kS) * C::kStageBytes;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int i = 0; i < C::FM; ++i) fa[kk][i] = frags.a(base, kk, i);
#pragma unroll
      for (int j = 0; j < C::FN; ++j) fb[kk][j] = frags.b(base, kk, j);
    }
    if (kt >= 1) issue_stage(kt - 1 + kS);
    {
      // Stages this wave has issued: up to min(kt + kS - 1, ktiles - 1);
      // stage kt + 1 must have landed.
      const int64_t last = kt + kS - 1 < ktiles - 1 ? kt + kS - 1 : ktiles - 1;
      wait_stages<C::kDma, kS - 2>(last - (kt + 1));
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the fragments are in
    barrier();
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[kk][i], fb[kk][j], acc[i][j], 0,
                                                             0, 0);
    __builtin_amdgcn_s_setprio(0);
    barrier();
  }
  if (!late) barrier();
}

// LDS of a GEMM workgroup: the stage ring; for the dX epilogue (rank-16
// update) also room for a rank-16 grad tail block.
template <class C, int EPI>
constexpr int nt_smem_bytes() {
  constexpr int ring = C::STAGES * C::kStageBytes;
  return EPI == EPI_RANK && kRankGradSmem > ring ? kRankGradSmem : ring;
}

// Data-parallel / split-K kernel: workgroup = one output tile (blockIdx.x,
// XCD-remapped) or, split over K, one (tile, split) pair (split_tile;
// EPI_PARTIAL stores its fp32 accumulator to split plane `split`).  Workgroups past the tiles run the
// optional rank-16 grad tail (p.tail; rank-16 epilogue, unsplit launches)
// after the GEMM tiles, filling CUs the GEMM leaves idle.
template <class C, int CT, int EPI, int L = 0>
__global__ __launch_bounds__(C::kThreads, C::MINW) void gemm_nt_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[nt_smem_bytes<C, EPI>()];
  if (EPI == EPI_PLAIN && p.alpha_dev) p.alpha *= *p.alpha_dev;
  const int64_t tiles = gridDim.x - p.tail_blocks - p.tail2_blocks;
  if constexpr (EPI == EPI_RANK) {
    if ((int64_t)blockIdx.x >= tiles) {
      run_tail_block(p, blockIdx.x - tiles, smem);
      return;
    }
  }
  int64_t tile, split = 0;
  if constexpr (EPI == EPI_PARTIAL)
    split_tile(p.remap, tiles, tile, split);
  else
    tile = p.remap ? xcd_remap(blockIdx.x, tiles) : (int64_t)blockIdx.x;
  int64_t m0, n0;
  tile_origin<C>(p, tile, m0, n0);
  int64_t kbeg = 0, klen = p.K;
  if constexpr (EPI == EPI_PARTIAL) {
    kbeg = split * p.k_split;
    klen = p.K - kbeg < p.k_split ? p.K - kbeg : p.k_split;
  }
  NtAcc<C> acc;
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j) acc[i][j] = float16v{};
  if constexpr (C::kWaves == 8 && C::KK == 2) {
    if (p.pingpong)
      nt_mainloop_pp<C, L>(p, m0, n0, kbeg, klen, smem, acc);
    else
      nt_mainloop<C, L>(p, m0, n0, kbeg, klen, smem, acc);
  } else {
    nt_mainloop<C, L>(p, m0, n0, kbeg, klen, smem, acc);
  }
  static_assert(!GluStage<C>::kOk || GluStage<C>::kBytes <= nt_smem_bytes<C, EPI>(), "stage");
  nt_epilogue<C, CT, EPI>(p, m0, n0, acc, smem, split);
}

// Split-K reduction: out[row][col] = epilogue(sum over splits s = 0.. of
// part[s][row][col]), four columns per thread.  The epilogues are those of the
// GEMM kernel with the same rounding order; the rank-16 terms are summed in
// fp32 in rank order.
// TAIL: the first p.tail_blocks + p.tail2_blocks workgroups run the rank-16
// grads p.tail / p.tail2 (run_tail_block, vector loads) instead, overlapping
// the reduce: used for split-K dX products, whose dA and dB would otherwise
// need launches of their own.
template <int CT, int EPI, bool TAIL = false>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmParams p, int splits) {
  if (EPI == EPI_PLAIN && p.alpha_dev) p.alpha *= *p.alpha_dev;
  int64_t block = blockIdx.x;
  if constexpr (TAIL) {
    __shared__ __attribute__((aligned(16))) unsigned char smem[kRankGradSmem];
    if (block < p.tail_blocks + p.tail2_blocks) {
      run_tail_block(p, block, smem);
      return;
    }
    block -= p.tail_blocks + p.tail2_blocks;
  }
  const int64_t groups = cdiv(p.N, 4);
  const int64_t g = block * 256 + threadIdx.x;
  if (g >= p.M * groups) return;
  const int64_t row = g / groups;
  const int64_t c0 = (g % groups) * 4;
  const int64_t plane = p.M * p.N;
  // Every load of the thread -- the epilogue's operands (Z row, lora_B rows or
  // lora_A columns, bias, gate / up) and then up to eight partials -- is
  // issued before the first add, so the thread waits for memory once.
  // Rank-16 operands use 16-byte (Z, lora_B rows) and 8-byte (four lora_A
  // columns) loads where aligned.
  half8 z8[2];
  if (EPI == EPI_RANK || (EPI == EPI_LORA && !p.lora_plane)) {
    const half_t* zr = p.lz + row * 16;
    if (reinterpret_cast<uintptr_t>(p.lz) % 16 == 0) {
      z8[0] = *reinterpret_cast<const half8*>(zr);
      z8[1] = *reinterpret_cast<const half8*>(zr + 8);
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) z8[r / 8][r % 8] = zr[r];
    }
  }
  half4 a4[16];  // EPI_RANK: lora_A[r][c0 .. c0 + 3]
  if constexpr (EPI == EPI_RANK) {
    if (c0 + 4 <= p.N && p.ldlb % 4 == 0 && reinterpret_cast<uintptr_t>(p.lb) % 8 == 0) {
#pragma unroll
      for (int r = 0; r < 16; ++r) a4[r] = *reinterpret_cast<const half4*>(p.lb + r * p.ldlb + c0);
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) a4[r][e] = c0 + e < p.N ? p.lb[r * p.ldlb + c0 + e] : (half_t)0;
    }
  }
  half8 b8[4][2];  // EPI_LORA: lora_B rows of the four columns (no lora_plane)
  half_t lp[4];    // EPI_LORA: the rounded LoRA terms (lora_plane)
  if constexpr (EPI == EPI_LORA) {
    if (p.lora_plane) {
      const half_t* src = p.lora_plane + row * p.N + c0;
      if (p.N % 4 == 0) {
        const half4 v4 = *reinterpret_cast<const half4*>(src);
#pragma unroll
        for (int e = 0; e < 4; ++e) lp[e] = v4[e];
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) lp[e] = c0 + e < p.N ? src[e] : (half_t)0;
      }
    }
#pragma unroll
    for (int e = 0; e < 4 && !p.lora_plane; ++e) {
      const int64_t col = c0 + e < p.N ? c0 + e : p.N - 1;
      const half_t* br = p.lb + col * 16;
      if (reinterpret_cast<uintptr_t>(p.lb) % 16 == 0) {
        b8[e][0] = *reinterpret_cast<const half8*>(br);
        b8[e][1] = *reinterpret_cast<const half8*>(br + 8);
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) b8[e][r / 8][r % 8] = br[r];
      }
    }
  }
  float bias[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) bias[e] = p.bias && c0 + e < p.N ? (float)p.bias[c0 + e] : 0.0f;
  half_t gg[4], uu[4];  // EPI_GLU: gate / up of the four columns, loaded before any store
  if constexpr (EPI == EPI_GLU) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const bool in = c0 + e < p.N;
      gg[e] = in ? p.glu_gate[row * p.ldgate + c0 + e] : (half_t)0;
      uu[e] = in && p.glu == 2 ? p.glu_up[row * p.ldup + c0 + e] : (half_t)0;
    }
  }
  // Sum of the splits in split order.
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (p.N % 4 == 0) {
    constexpr int kAhead = 8;
    float4v t[kAhead];
#pragma unroll
    for (int s = 0; s < kAhead; ++s)
      if (s < splits) t[s] = *reinterpret_cast<const float4v*>(p.part + s * plane + row * p.N + c0);
#pragma unroll
    for (int s = 0; s < kAhead; ++s)
      if (s < splits)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += t[s][e];
    for (int s = kAhead; s < splits; ++s) {
      const float4v u = *reinterpret_cast<const float4v*>(p.part + s * plane + row * p.N + c0);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += u[e];
    }
  } else {
    for (int s = 0; s < splits; ++s)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (c0 + e < p.N) v[e] += p.part[s * plane + row * p.N + c0 + e];
  }
  float z[16];
  if constexpr (EPI == EPI_LORA || EPI == EPI_RANK) {
#pragma unroll
    for (int r = 0; r < 16; ++r) z[r] = (float)z8[r / 8][r % 8];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t col = c0 + e;
    if (col >= p.N) break;
    const int64_t idx = row * p.ldc + col;
    if constexpr (EPI == EPI_LORA) {
      const float y = (float)f32_to_f16(v[e] * p.alpha + bias[e]);
      float scaled;
      if (p.lora_plane) {
        scaled = (float)lp[e];
      } else {
        float l = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) l += z[r] * (float)b8[e][r / 8][r % 8];
        scaled = (float)f32_to_f16((float)f32_to_f16(l) * p.lscale);
      }
      reinterpret_cast<half_t*>(p.C)[idx] = f32_to_f16(y + scaled);
    } else if constexpr (EPI == EPI_RANK) {
      float l = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) l += z[r] * (float)a4[r][e];
      store_c<CT>(p.C, idx, v[e] + l, p.beta);
    } else {
      if constexpr (EPI == EPI_GLU)
        glu_apply(p, row, col, idx, v[e] * p.alpha + bias[e], gg[e], uu[e]);
      else
        store_c<CT>(p.C, idx, v[e] * p.alpha + bias[e], p.beta);
    }
  }
}

// Tile configurations: <BM, BN, waves M, waves N, BK, stages, min waves/SIMD>.
using NtSmall = NtCfg<64, 64, 2, 2, 32, 4, 2>;      // 4 waves of 32x32, 32 KiB LDS
using NtMid = NtCfg<128, 128, 2, 2, 32, 3, 2>;      // 4 waves of 64x64, 48 KiB LDS
using NtBig4 = NtCfg<256, 256, 2, 2, 32, 3, 1>;     // 4 waves of 128x128, 96 KiB LDS
using NtBig8 = NtCfg<256, 256, 2, 4, 64, 2, 2>;     // 8 waves of 128x64, 128 KiB LDS
using NtWide8 = NtCfg<256, 128, 4, 2, 64, 2, 2>;    // 8 waves of 64x64, 96 KiB LDS
using NtBig8s = NtCfg<256, 256, 2, 4, 32, 3, 2>;    // 8 waves of 128x64, 96 KiB LDS
using NtMid64 = NtCfg<128, 128, 2, 2, 64, 2, 2>;    // 4 waves of 64x64, 64 KiB LDS
using NtBig8s4 = NtCfg<256, 256, 2, 4, 32, 4, 2>;   // 8 waves of 128x64, 128 KiB LDS
using NtWide8s4 = NtCfg<256, 128, 4, 2, 32, 4, 1>;  // 8 waves of 64x64, 96 KiB LDS
using NtTall8s4 = NtCfg<128, 256, 2, 4, 32, 4, 1>;  // 8 waves of 64x64, 96 KiB LDS

template <class C, int CT, int EPI, int L = 0>
int launch_nt(const GemmParams& p, int64_t splits, hipStream_t stream) {
  const dim3 grid((unsigned)(cdiv(p.M, C::BM) * cdiv(p.N, C::BN) + p.tail_blocks +
                             p.tail2_blocks),
                  (unsigned)splits);
  hipLaunchKernelGGL((gemm_nt_kernel<C, CT, EPI, L>), grid, dim3(C::kThreads), 0, stream, p);
  SS_CHECK_LAUNCH("gemm_nt_kernel");
  if (EPI == EPI_GLU && p.glu_done) *p.glu_done = 1;
  return SS_OK;
}

// K-major operands (L != 0) take the configurations nt_plan picks (1, 2, 8, 9,
// 10); the others are reached only through a build-time override and keep
// row-major operands.
template <int CT, int EPI, int L>
int dispatch_nt_t(const GemmParams& p, int cfg, int64_t splits, hipStream_t stream) {
  switch (cfg) {
    case 10: return launch_nt<NtTall8s4, CT, EPI, L>(p, splits, stream);
    case 9: return launch_nt<NtWide8s4, CT, EPI, L>(p, splits, stream);
    case 8: return launch_nt<NtBig8s4, CT, EPI, L>(p, splits, stream);
    case 2: return launch_nt<NtMid, CT, EPI, L>(p, splits, stream);
    case 1: return launch_nt<NtSmall, CT, EPI, L>(p, splits, stream);
    default: return SS_ERR_UNSUPPORTED;
  }
}

template <int CT, int EPI>
int dispatch_nt(const GemmParams& p, int cfg, int64_t splits, hipStream_t stream) {
  const int layout = (p.a_t ? 1 : 0) | (p.b_t ? 2 : 0);
  if constexpr (EPI == EPI_PLAIN || EPI == EPI_PARTIAL) {
    if (layout == 1) return dispatch_nt_t<CT, EPI, 1>(p, cfg, splits, stream);
    if (layout == 2) return dispatch_nt_t<CT, EPI, 2>(p, cfg, splits, stream);
    if (layout == 3) return dispatch_nt_t<CT, EPI, 3>(p, cfg, splits, stream);
  } else {
    if (layout) return SS_ERR_UNSUPPORTED;
  }
  switch (cfg) {
    case 10: return launch_nt<NtTall8s4, CT, EPI>(p, splits, stream);
    case 9: return launch_nt<NtWide8s4, CT, EPI>(p, splits, stream);
    case 8: return launch_nt<NtBig8s4, CT, EPI>(p, splits, stream);
    case 7: return launch_nt<NtMid64, CT, EPI>(p, splits, stream);
    case 6: return launch_nt<NtBig8s, CT, EPI>(p, splits, stream);
    case 5: return launch_nt<NtWide8, CT, EPI>(p, splits, stream);
    case 4: return launch_nt<NtBig8, CT, EPI>(p, splits, stream);
    case 3: return launch_nt<NtBig4, CT, EPI>(p, splits, stream);
    case 2: return launch_nt<NtMid, CT, EPI>(p, splits, stream);
    default: return launch_nt<NtSmall, CT, EPI>(p, splits, stream);
  }
}

template <int CT, int EPI, bool TAIL = false>
int reduce_nt(const GemmParams& p, int64_t splits, hipStream_t stream) {
  const int64_t threads = p.M * cdiv(p.N, 4);
  const int64_t blocks = cdiv(threads, 256) + (TAIL ? p.tail_blocks + p.tail2_blocks : 0);
  hipLaunchKernelGGL((splitk_reduce_kernel<CT, EPI, TAIL>), dim3((unsigned)blocks), dim3(256), 0,
                     stream, p, (int)splits);
  SS_CHECK_LAUNCH("splitk_reduce_kernel");
  if (EPI == EPI_GLU && p.glu_done) *p.glu_done = 1;
  return SS_OK;
}

bool aligned16(const void* ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; }

}  // namespace

// Configuration and split-K plan for an M x N x K product.
//   128x256 (8 waves) when 96 or more 256x256 tiles would run but the
//   128x256 tiles still fit one wave on the CUs (K < 8192);
//   256x256 (8 waves, 4-stage ring) once it gives at least half the CUs a
//   tile;
//   a very long K (32768 or more) over at most 128 tiles of 256x256: those
//   tiles split over k into one wave of workgroups;
//   long K with few 128x128 tiles: split over k (each split at least 1024
//   k), 256x128 tiles with about one workgroup per CU where M fills 256-row
//   tiles, else 128x128 with about 512 workgroups;
//   96..127 tiles of 256x256 and a long K: 256x256 split in two;
//   128x128 while it gives half the CUs a tile; else 64x64.
// SS_TUNE_NT_TILE (1..10, the cases of dispatch_nt) and
// SS_TUNE_NT_SPLITS override the choice (build-time constants, tuning.h).
NtPlan nt_plan(int64_t m, int64_t n, int64_t k) {
  constexpr int forced = SS_TUNE_NT_TILE;
  constexpr int forced_splits = SS_TUNE_NT_SPLITS;
  NtPlan plan{1, 1, k};
  const int64_t t256 = cdiv(m, 256) * cdiv(n, 256);
  const int64_t t128 = cdiv(m, 128) * cdiv(n, 128);
  const int64_t t10 = cdiv(m, 128) * cdiv(n, 256);  // 128x256 tiles
  if (t256 >= 96 && t10 <= 256 && k < 8192) {
    // 96 or more tiles of 256x256, but one wave of 128x256 tiles (8 waves):
    // the half-height tiles fill the CUs better and pad M less (2048 x 3584
    // x 3584: 60.8 vs 67.3 us for 256x256, 70.6 us for 128x128; the
    // cross-entropy chunk 826 x 8192 x 1536: 31.5 vs 37.7 us).
    plan.cfg = 10;
  } else if (t256 >= 128) {
    plan.cfg = 8;
  } else if (k >= 32768 && t256 <= 128) {
    // A very long K over few output tiles (the cross-entropy dX over the whole
    // vocabulary, 523 x 1536 x 151936): 256x256 tiles split over K into one wave
    // of workgroups, one 8-wave workgroup per CU (14 splits: 403 us against 485
    // us for 128x128 split 8; 16 or 18 splits, a second partial wave: 490 us).
    plan.cfg = 8;
    int64_t s = 256 / t256;
    if (s > k / 2048) s = k / 2048;
    plan.splits = s < 1 ? 1 : s;
  } else if (k >= 2048 && t128 < 256) {
    plan.cfg = 2;
    int64_t s = 512 / t128;
    if (s > k / 1024) s = k / 1024;
    plan.splits = s < 1 ? 1 : (s > 8 ? 8 : s);
    // 256x128 tiles (8 waves) when M fills 256-row tiles as well as 128-row
    // ones and a split of about one workgroup per CU still gives 192 or more
    // workgroups (990 x 1536 x 8960: 44 us against 50 us for 128x128).
    const int64_t tw = cdiv(m, 256) * cdiv(n, 128);
    int64_t sw = 256 / tw;
    if (sw > k / 1024) sw = k / 1024;
    sw = sw < 1 ? 1 : (sw > 8 ? 8 : sw);
    if (cdiv(m, 256) * 2 == cdiv(m, 128) && tw * sw >= 192) {
      plan.cfg = 9;
      plan.splits = sw;
    }
  } else if (t256 >= 96) {
    // 96..127 tiles of 256x256 with a long K (k >= 8192 here): 256x256 split
    // in two (2048 x 3584 x 18944: 263 vs 295 us for 128x256, 354 us for
    // 128x128).
    plan.cfg = 8;
    plan.splits = 2;
  } else if (t128 >= 128) {
    plan.cfg = 2;
  } else if (t128 < 64 && k >= 1024) {
    // Few output tiles (e.g. a 256-wide k/v projection): 64x64 tiles split
    // over K until about 256 workgroups run, each split at least 384 deep.
    const int64_t t64 = cdiv(m, 64) * cdiv(n, 64);
    int64_t s = 256 / t64;
    if (s > k / 384) s = k / 384;
    plan.splits = s < 1 ? 1 : (s > 8 ? 8 : s);
  }
  if (forced >= 1 && forced <= 10) plan.cfg = forced;
  if (forced_splits >= 1) plan.splits = forced_splits;
  plan.k_split = cdiv(cdiv(k, plan.splits), 64) * 64;
  plan.splits = cdiv(k, plan.k_split);
  return plan;
}

int splitk_reduce(const GemmParams& p, int splits, int ct, int epi, hipStream_t stream) {
  if (ct == SS_F32) {
    if (epi != EPI_PLAIN) return SS_ERR_UNSUPPORTED;
    return reduce_nt<SS_F32, EPI_PLAIN>(p, splits, stream);
  }
  if (epi == EPI_LORA) return reduce_nt<SS_F16, EPI_LORA>(p, splits, stream);
  if (epi == EPI_RANK) return reduce_nt<SS_F16, EPI_RANK>(p, splits, stream);
  if (p.glu) return reduce_nt<SS_F16, EPI_GLU>(p, splits, stream);
  return reduce_nt<SS_F16, EPI_PLAIN>(p, splits, stream);
}

// Split-K scratch: the fp32 partial planes, then (256-byte aligned) the fp16
// LoRA plane of a split LoRA forward.
static size_t nt_plane_offset(int64_t m, int64_t n, int64_t splits) {
  return ((size_t)(splits * m * n) * sizeof(float) + 255) / 256 * 256;
}
static size_t nt_split_bytes(int64_t m, int64_t n, int64_t splits) {
  return nt_plane_offset(m, n, splits) + (size_t)(m * n) * sizeof(half_t);
}

size_t nt_partial_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0 || k % 64 != 0) return 0;
  const NtPlan plan = nt_plan(m, n, k);
  return plan.splits > 1 ? nt_split_bytes(m, n, plan.splits) : 0;
}

// SS_TUNE_NT_PINGPONG = 0 keeps the 8-wave configurations on the lockstep
// main loop (tuning.h).
static bool pingpong_enabled() { return SS_TUNE_NT_PINGPONG != 0; }

// SS_TUNE_NT_STAGED = 0 keeps fp16 epilogues on direct 2-byte stores.
bool staged_epilogue_enabled() { return SS_TUNE_NT_STAGED != 0; }

int gemm_nt(const GemmParams& p0, int ct, int epi, hipStream_t stream, void* partials,
            size_t partial_bytes) {
  GemmParams p = p0;
  p.pingpong = pingpong_enabled();
  p.c_vec = staged_epilogue_enabled() && ct == SS_F16 && !p.beta && p.N % 8 == 0 &&
            p.ldc % 8 == 0 && aligned16(p.C);
  if (p.M <= 0 || p.N <= 0 || p.K <= 0 || p.K % 64 != 0) return SS_ERR_UNSUPPORTED;  // K % 64
  if (!aligned16(p.A) || !aligned16(p.B) || p.lda % 8 != 0 || p.ldb % 8 != 0)
    return SS_ERR_UNSUPPORTED;
  // K-major operands: whole 16-byte chunks along M / N, plain or split-K
  // epilogues only.
  if ((p.a_t && p.M % 8 != 0) || (p.b_t && p.N % 8 != 0)) return SS_ERR_UNSUPPORTED;
  if ((p.a_t || p.b_t) && (epi != EPI_PLAIN || p.glu)) return SS_ERR_UNSUPPORTED;
  // The DMA addresses operands with 32-bit byte offsets from their base (per
  // stage for K-major operands, whose base moves BK rows a stage).
  const int64_t kMaxOff = (int64_t)1 << 32;
  const int64_t a_span = p.a_t ? 64 * p.lda + p.M : (p.M - 1) * p.lda + p.K;
  const int64_t b_span = p.b_t ? 64 * p.ldb + p.N : (p.N - 1) * p.ldb + p.K;
  if (a_span * 2 >= kMaxOff || b_span * 2 >= kMaxOff) return SS_ERR_UNSUPPORTED;
  if (epi != EPI_PLAIN && (!aligned16(p.lz) || (epi == EPI_LORA && !aligned16(p.lb))))
    return SS_ERR_UNSUPPORTED;
  if (ct != SS_F16 && epi != EPI_PLAIN) return SS_ERR_UNSUPPORTED;
  NtPlan plan = nt_plan(p.M, p.N, p.K);
  const size_t need = nt_split_bytes(p.M, p.N, plan.splits);
  if (plan.splits > 1 && (!partials || partial_bytes < need ||
                          reinterpret_cast<uintptr_t>(partials) % 16 != 0)) {
    plan.splits = 1;
    plan.k_split = p.K;
  }
  // The rank-16 grad tail rides on unsplit dX products (rank-16 epilogue)
  // after the GEMM tiles: measured, it fills idle CUs there (down / q / o / k
  // / v backward 6-11 us faster).  On the split-K launches of the long-K dX it
  // slowed the GEMM more than a launch of its own costs; there it leads the
  // reduce launch instead.
  if (epi != EPI_RANK) p.tail_blocks = p.tail2_blocks = 0;
  if (p.tail_blocks + p.tail2_blocks > 0 && p.tail_ran) *p.tail_ran = 1;
  if (plan.splits > 1) {
    p.part = reinterpret_cast<float*>(partials);
    p.k_split = plan.k_split;
    // The rank-16 update is folded into split 0's partial (the reduce then
    // only sums: its lora_A column loads dominated its load count); the
    // forward's rounded LoRA term goes from split 0 to a plane of its own
    // (its lora_B row loads doubled the reduce's load count: 990 x 1536 x
    // 8960 reduce 11.7 us against 6.9 us without the LoRA term).
    p.fold_rank = epi == EPI_RANK;
    p.lora_plane = epi == EPI_LORA
                       ? reinterpret_cast<half_t*>(static_cast<char*>(partials) +
                                                   nt_plane_offset(p.M, p.N, plan.splits))
                       : nullptr;
    const int64_t tail = p.tail_blocks, tail2 = p.tail2_blocks;
    p.tail_blocks = p.tail2_blocks = 0;
    const int rc = dispatch_nt<SS_F32, EPI_PARTIAL>(p, plan.cfg, plan.splits, stream);
    if (rc) return rc;
    p.tail_blocks = tail;
    p.tail2_blocks = tail2;
    if (ct == SS_F32) return reduce_nt<SS_F32, EPI_PLAIN>(p, plan.splits, stream);
    if (epi == EPI_LORA) return reduce_nt<SS_F16, EPI_LORA>(p, plan.splits, stream);
    if (epi == EPI_RANK) {
      GemmParams q = p;
      q.alpha = 1.0f;
      q.bias = nullptr;
      if (q.tail_blocks + q.tail2_blocks > 0)
        return reduce_nt<SS_F16, EPI_PLAIN, true>(q, plan.splits, stream);
      return reduce_nt<SS_F16, EPI_PLAIN>(q, plan.splits, stream);
    }
    if (p.glu) return reduce_nt<SS_F16, EPI_GLU>(p, plan.splits, stream);
    return reduce_nt<SS_F16, EPI_PLAIN>(p, plan.splits, stream);
  }
  if (ct == SS_F16) {
    if (epi == EPI_LORA) return dispatch_nt<SS_F16, EPI_LORA>(p, plan.cfg, 1, stream);
    if (epi == EPI_RANK) return dispatch_nt<SS_F16, EPI_RANK>(p, plan.cfg, 1, stream);
    if (p.glu) return dispatch_nt<SS_F16, EPI_GLU>(p, plan.cfg, 1, stream);
    return dispatch_nt<SS_F16, EPI_PLAIN>(p, plan.cfg, 1, stream);
  }
  return dispatch_nt<SS_F32, EPI_PLAIN>(p, plan.cfg, 1, stream);
}

}  // namespace ss
