// Dense NT GEMM main loop for gfx950: C[M,N] = alpha * A[M,K] . B[N,K]^T with
// both operands K-contiguous fp16 and fp32 accumulation on
// v_mfma_f32_32x32x16_f16.  This is the hot loop of the decode-first NF4
// projections (X . Wdec^T forward, dY . (Wdec^T)^T backward) and of the dense
// NT products; the epilogues (bias, LoRA add, rank-16 update, beta) are the
// ones of gemm.hip.
//
// Pipeline: STAGES LDS buffers of BK = 32 k.  Operand tiles move from global
// memory straight into LDS with global_load_lds_dwordx4 (no register
// staging): one wave-wide DMA writes 64 lanes x 16 B = 1 KiB of contiguous LDS
// (lane i at +16 i), i.e. 16 rows x 64 B of one operand tile.  Stage
// kt + STAGES - 1 is requested while stage kt is consumed, so STAGES - 1
// stages of loads are in flight behind the MFMAs.
//
// LDS layout: row r of a stage tile is 64 B (4 chunks of 8 halves); logical
// chunk c lives at physical chunk c ^ ((r >> 1) & 3).  The lane that fills
// physical chunk q of row r therefore fetches logical chunk q ^ ((r >> 1) & 3)
// from global memory.  A fragment read (32 consecutive rows, one logical
// chunk) then touches 8 distinct 16-byte bank groups per 8 lanes: no LDS bank
// conflicts.
//
// The DMA is issued from inline asm.  The compiler does not know which LDS
// buffer an outstanding LDS DMA writes, and would wait for all of them
// (vmcnt(0)) before every LDS read, draining the pipeline.  Waits are explicit
// instead: before stage kt is read, vmcnt lets only the DMAs of later stages
// stay outstanding; lgkmcnt(0) + s_barrier then make every wave's part of
// the stage visible and guarantee that no wave still reads the buffer that
// is refilled next.

#include <stdlib.h>

#include "gemm.h"

namespace ss {
namespace {

constexpr int kBK = 32;
typedef float float16v __attribute__((ext_vector_type(16)));

template <int BM_, int BN_, int WAVES_M, int WAVES_N, int STAGES_, int MINW_>
struct NtCfg {
  static constexpr int BM = BM_, BN = BN_, STAGES = STAGES_, MINW = MINW_;
  static constexpr int kWaves = WAVES_M * WAVES_N;
  static constexpr int kThreads = kWave * kWaves;
  static constexpr int kWavesN = WAVES_N;
  static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  static constexpr int FM = WM / 32, FN = WN / 32;  // 32x32 accumulator blocks per wave
  static constexpr int kDmaA = BM / 16 / kWaves;    // DMA instructions per wave per stage
  static constexpr int kDmaB = BN / 16 / kWaves;
  static constexpr int kDma = kDmaA + kDmaB;
  static constexpr int kTileA = BM * kBK * 2;       // bytes of one stage's A tile
  static constexpr int kStageBytes = (BM + BN) * kBK * 2;
  static_assert(BM % (16 * kWaves) == 0 && BN % (16 * kWaves) == 0, "DMA split over waves");
  static_assert(WM % 32 == 0 && WN % 32 == 0, "32x32 MFMA blocks");
  static_assert(STAGES >= 2 && STAGES <= 4, "pipeline depth");
};

// One wave-wide 16-byte-per-lane DMA: lane i's 16 bytes at `src` land at LDS
// byte address lds + 16 i.  `lds` must be wave-uniform.  s_nop covers the
// M0-write -> LDS-DMA hazard.
__device__ __forceinline__ void dma16(const half_t* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(lds)
               : "memory", "m0");
}

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt unconstrained).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// Wait until at most `ahead` stages of DMAs (kDma each) are outstanding.
template <int KDMA, int MAXAHEAD>
__device__ __forceinline__ void wait_stages(int64_t ahead) {
  if constexpr (MAXAHEAD >= 2) {
    if (ahead >= 2) {
      wait_vm<2 * KDMA>();
      return;
    }
  }
  if constexpr (MAXAHEAD >= 1) {
    if (ahead >= 1) {
      wait_vm<KDMA>();
      return;
    }
  }
  wait_vm<0>();
}

__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

template <class C, int CT, int EPI>
__global__ __launch_bounds__(C::kThreads, C::MINW) void gemm_nt_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[C::STAGES * C::kStageBytes];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int wm = wave / C::kWavesN;
  const int wn = wave % C::kWavesN;
  // M-fastest tile order: consecutive tiles share the B (weight) panel; with
  // the XCD remap they run back to back on one XCD and reuse it from L2.
  const int64_t mtiles = cdiv(p.M, C::BM);
  const int64_t tile = p.remap ? xcd_remap(blockIdx.x, gridDim.x) : (int64_t)blockIdx.x;
  const int64_t m0 = (tile % mtiles) * C::BM;
  const int64_t n0 = (tile / mtiles) * C::BN;
  const uint32_t lds0 = lds_address(smem);

  // Per-lane DMA sources: row (16 per DMA) and the logical chunk that belongs
  // in physical chunk (lane & 3).  Rows past M / N are clamped to the last
  // row: they only feed accumulator rows that are never stored.
  const half_t* a_src[C::kDmaA];
  const half_t* b_src[C::kDmaB];
#pragma unroll
  for (int j = 0; j < C::kDmaA; ++j) {
    const int row = (wave * C::kDmaA + j) * 16 + (lane >> 2);
    const int chunk = (lane & 3) ^ ((row >> 1) & 3);
    const int64_t gr = m0 + row < p.M ? m0 + row : p.M - 1;
    a_src[j] = p.A + gr * p.lda + chunk * 8;
  }
#pragma unroll
  for (int j = 0; j < C::kDmaB; ++j) {
    const int row = (wave * C::kDmaB + j) * 16 + (lane >> 2);
    const int chunk = (lane & 3) ^ ((row >> 1) & 3);
    const int64_t gr = n0 + row < p.N ? n0 + row : p.N - 1;
    b_src[j] = p.B + gr * p.ldb + chunk * 8;
  }
  auto issue = [&](int64_t kt, int stage) {
    const uint32_t base = lds0 + stage * C::kStageBytes;
#pragma unroll
    for (int j = 0; j < C::kDmaA; ++j)
      dma16(a_src[j] + kt * kBK,
            __builtin_amdgcn_readfirstlane(base + (wave * C::kDmaA + j) * 1024));
#pragma unroll
    for (int j = 0; j < C::kDmaB; ++j)
      dma16(b_src[j] + kt * kBK,
            __builtin_amdgcn_readfirstlane(base + C::kTileA + (wave * C::kDmaB + j) * 1024));
  };

  // Fragment offsets: lane reads row (lane & 31) of a 32-row block, logical
  // chunk 2 * kk + (lane >> 5), stored at chunk ^ ((row >> 1) & 3).
  const int lr = lane & 31;
  const int lh = lane >> 5;
  const int swz = (lr >> 1) & 3;
  const int frag_off[2] = {lr * 64 + ((lh ^ swz) << 4), lr * 64 + (((2 + lh) ^ swz) << 4)};

  float16v acc[C::FM][C::FN];
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j) acc[i][j] = float16v{};

  const int64_t ktiles = p.K / kBK;
#pragma unroll
  for (int s = 0; s < C::STAGES - 1; ++s)
    if (s < ktiles) issue(s, s);

  for (int64_t kt = 0; kt < ktiles; ++kt) {
    const int64_t ahead = ktiles - 1 - kt;  // stages already requested after kt
    wait_stages<C::kDma, C::STAGES - 2>(ahead);
    lds_barrier();
    if (kt + C::STAGES - 1 < ktiles) issue(kt + C::STAGES - 1, (int)((kt + C::STAGES - 1) % C::STAGES));
    const unsigned char* sa = smem + (kt % C::STAGES) * C::kStageBytes + (wm * C::WM) * 64;
    const unsigned char* sb = smem + (kt % C::STAGES) * C::kStageBytes + C::kTileA + (wn * C::WN) * 64;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      half8 af[C::FM];
      half8 bf[C::FN];
#pragma unroll
      for (int i = 0; i < C::FM; ++i)
        af[i] = *reinterpret_cast<const half8*>(sa + i * 32 * 64 + frag_off[kk]);
#pragma unroll
      for (int j = 0; j < C::FN; ++j)
        bf[j] = *reinterpret_cast<const half8*>(sb + j * 32 * 64 + frag_off[kk]);
#pragma unroll
      for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  }

  // Epilogue: lane holds D[8 (r / 4) + 4 (lane / 32) + r % 4][lane % 32] of
  // each 32x32 block in register r.
#pragma unroll
  for (int i = 0; i < C::FM; ++i) {
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
      const int64_t row_base = m0 + wm * C::WM + i * 32;
      const int64_t col = n0 + wn * C::WN + j * 32 + lr;
      float16v extra = float16v{};
      if constexpr (EPI != EPI_PLAIN) {
        // Rank-16 term of this block on one v_mfma_f32_32x32x16_f16:
        // A = Z rows (row lane%32, ranks 8 (lane/32)..+7), B = (rank, column).
        const int64_t zr = row_base + lr;
        const half8 zero = half8{};
        const half8 za = zr < p.M ? *reinterpret_cast<const half8*>(p.lz + zr * 16 + 8 * lh) : zero;
        half8 zb = zero;
        if (col < p.N) {
          if constexpr (EPI == EPI_LORA) {
            zb = *reinterpret_cast<const half8*>(p.lb + col * 16 + 8 * lh);
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) zb[e] = p.lb[(8 * lh + e) * p.ldlb + col];
          }
        }
        extra = __builtin_amdgcn_mfma_f32_32x32x16_f16(za, zb, extra, 0, 0, 0);
      }
      if (col >= p.N) continue;
      const float b = p.bias ? (float)p.bias[col] : 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = row_base + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (row >= p.M) continue;
        const int64_t idx = row * p.ldc + col;
        if constexpr (EPI == EPI_LORA) {
          const float y = (float)f32_to_f16(acc[i][j][r] * p.alpha + b);
          const float lora = (float)f32_to_f16(extra[r]);
          const float scaled = (float)f32_to_f16(lora * p.lscale);
          reinterpret_cast<half_t*>(p.C)[idx] = f32_to_f16(y + scaled);
        } else if constexpr (EPI == EPI_RANK) {
          store_c<CT>(p.C, idx, acc[i][j][r] + extra[r], p.beta);
        } else {
          store_c<CT>(p.C, idx, acc[i][j][r] * p.alpha + b, p.beta);
        }
      }
    }
  }
}

using NtBig = NtCfg<256, 256, 2, 2, 4, 1>;    // 128x128 per wave, 128 KiB LDS, 1 WG / CU
using NtMid = NtCfg<128, 128, 2, 2, 4, 2>;    // 64x64 per wave, 64 KiB LDS, 2 WG / CU
using NtSmall = NtCfg<64, 64, 2, 2, 4, 2>;    // 32x32 per wave, 32 KiB LDS

template <class C, int CT, int EPI>
int launch_nt(const GemmParams& p, hipStream_t stream) {
  const dim3 grid((unsigned)(cdiv(p.M, C::BM) * cdiv(p.N, C::BN)));
  hipLaunchKernelGGL((gemm_nt_kernel<C, CT, EPI>), grid, dim3(C::kThreads), 0, stream, p);
  SS_CHECK_LAUNCH("gemm_nt_kernel");
  return SS_OK;
}

// Tile choice: 256x256 once it fills every CU (least LDS and L2 traffic per
// flop), else 128x128 while it gives at least half the CUs a tile, else 64x64.
// SS_NT_TILE (1 = 64x64, 2 = 128x128, 3 = 256x256) overrides it; a tuning
// knob read once per process.
int nt_tile(int64_t m, int64_t n) {
  static const int forced = [] {
    const char* e = getenv("SS_NT_TILE");
    return e ? atoi(e) : 0;
  }();
  if (forced >= 1 && forced <= 3) return forced;
  if (cdiv(m, 256) * cdiv(n, 256) >= 256) return 3;
  if (cdiv(m, 128) * cdiv(n, 128) >= 128) return 2;
  return 1;
}

template <int CT, int EPI>
int dispatch_nt(const GemmParams& p, hipStream_t stream) {
  switch (nt_tile(p.M, p.N)) {
    case 3: return launch_nt<NtBig, CT, EPI>(p, stream);
    case 2: return launch_nt<NtMid, CT, EPI>(p, stream);
    default: return launch_nt<NtSmall, CT, EPI>(p, stream);
  }
}

bool aligned16(const void* ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; }

}  // namespace

int gemm_nt(const GemmParams& p, int ct, int epi, hipStream_t stream) {
  if (p.M <= 0 || p.N <= 0 || p.K <= 0 || p.K % kBK != 0) return SS_ERR_UNSUPPORTED;
  if (!aligned16(p.A) || !aligned16(p.B) || p.lda % 8 != 0 || p.ldb % 8 != 0)
    return SS_ERR_UNSUPPORTED;
  if (epi != EPI_PLAIN && (!aligned16(p.lz) || (epi == EPI_LORA && !aligned16(p.lb))))
    return SS_ERR_UNSUPPORTED;
  if (ct == SS_F16) {
    if (epi == EPI_LORA) return dispatch_nt<SS_F16, EPI_LORA>(p, stream);
    if (epi == EPI_RANK) return dispatch_nt<SS_F16, EPI_RANK>(p, stream);
    return dispatch_nt<SS_F16, EPI_PLAIN>(p, stream);
  }
  if (epi != EPI_PLAIN) return SS_ERR_UNSUPPORTED;
  return dispatch_nt<SS_F32, EPI_PLAIN>(p, stream);
}

}  // namespace ss
