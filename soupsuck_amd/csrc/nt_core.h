// Pieces of the dense NT GEMM shared by its kernels (gemm_nt.hip) and the
// fused NF4 kernels (gemm_nf4.hip): tile configurations, operand tile
// layouts in LDS, stage waits, tile order and the epilogue.
//
// Pipeline: STAGES LDS buffers of BK k (32 or 64).  Operand tiles move from
// global memory straight into LDS with global_load_lds_dwordx4 (no register
// staging): one wave-wide DMA writes 64 lanes x 16 B = 1 KiB of contiguous
// LDS (lane i at +16 i).  How many bytes of a row one DMA fetches sets the
// DMA throughput (measured on MI355X, L2-resident data: 128 B per row ->
// 43 B/clk/CU into LDS, 64 B -> 25, 32 B -> 14), so:
//   BK = 64: a DMA covers 8 rows x 128 B.  Block b (rows 8b .. 8b+7) is 1 KiB;
//     chunk c of row 8b + r sits at slot (c ^ (b & 1)) * 8 + r.
//   BK = 32: a DMA covers 16 rows x 64 B.  Row r is 64 B; chunk c sits at
//     chunk c ^ swz32(r), swz32(r) = ((r >> 1) & 3) ^ ((r >> 3) & 1).
// A 128-bit LDS read is served 16 lanes at a time over 64 four-byte banks
// (256 B): with 64-byte rows, rows r and r + 4 share bank quads, so the 16
// rows of one pass must cover the four chunk positions once per residue
// r % 4.  swz32 does that and also keeps each 8-lane group conflict-free
// (the narrower 128-byte pass); the former c ^ ((r >> 1) & 3) repeated with
// period 8 and measured a uniform 2-way conflict (SQ_LDS_BANK_CONFLICT =
// half of SQ_LDS_IDX_ACTIVE).  Both layouts make an MFMA 32x32x16 fragment
// read (32 consecutive rows, one chunk per lane half) conflict-free.
#pragma once

#include "rank16.h"

namespace ss {
namespace {

typedef float float16v __attribute__((ext_vector_type(16)));

template <int BM_, int BN_, int WAVES_M, int WAVES_N, int BK_, int STAGES_, int MINW_>
struct NtCfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, STAGES = STAGES_, MINW = MINW_;
  static constexpr int kWaves = WAVES_M * WAVES_N;
  static constexpr int kThreads = kWave * kWaves;
  static constexpr int kWavesN = WAVES_N;
  static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  static constexpr int FM = WM / 32, FN = WN / 32;   // 32x32 accumulator blocks per wave
  static constexpr int KK = BK / 16;                 // MFMA k-steps per stage
  static constexpr int kRowsPerDma = 1024 / (BK * 2);
  static constexpr int kDmaA = BM / kRowsPerDma / kWaves;  // DMAs per wave per stage
  static constexpr int kDmaB = BN / kRowsPerDma / kWaves;
  static constexpr int kDma = kDmaA + kDmaB;
  static constexpr int kTileA = BM * BK * 2;         // bytes of one stage's A tile
  static constexpr int kStageBytes = (BM + BN) * BK * 2;
  static_assert(BK == 32 || BK == 64, "stage depth");
  static_assert(BM % (kRowsPerDma * kWaves) == 0 && BN % (kRowsPerDma * kWaves) == 0,
                "DMA split over waves");
  static_assert(WM % 32 == 0 && WN % 32 == 0, "32x32 MFMA blocks");
  static_assert(STAGES >= 2 && STAGES <= 5, "pipeline depth");
  static_assert(STAGES * kStageBytes <= 160 * 1024, "LDS");
};

// Wait until at most `ahead` stages of DMAs (KDMA each) are outstanding.
template <int KDMA, int MAXAHEAD>
__device__ __forceinline__ void wait_stages(int64_t ahead) {
  static_assert(MAXAHEAD <= 4, "wait depth");
  if constexpr (MAXAHEAD >= 4) {
    if (ahead >= 4) {
      wait_vm<4 * KDMA>();
      return;
    }
  }
  if constexpr (MAXAHEAD >= 3) {
    if (ahead >= 3) {
      wait_vm<3 * KDMA>();
      return;
    }
  }
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

// Chunk swizzle of the BK = 32 layout (see the layout notes above).
__device__ __forceinline__ int swz32(int r) { return ((r >> 1) & 3) ^ ((r >> 3) & 1); }

// DMA g of an operand tile: the row and logical 16-byte chunk that lane
// fetches (its LDS slot is g * 1024 + 16 * lane).
template <int BK>
__device__ __forceinline__ void dma_source(int g, int lane, int& row, int& chunk) {
  if constexpr (BK == 64) {
    row = g * 8 + (lane & 7);
    chunk = (lane >> 3) ^ (g & 1);
  } else {
    row = g * 16 + (lane >> 2);
    chunk = (lane & 3) ^ swz32(row);
  }
}

// Byte offset (within a stage's operand tile, relative to the start of a
// 32-row group) of the lane's fragment for k-step kk: row lane % 32,
// logical chunk 2 kk + lane / 32.
template <int BK>
__device__ __forceinline__ int frag_offset(int lane, int kk) {
  const int r = lane & 31;
  const int c = 2 * kk + (lane >> 5);
  if constexpr (BK == 64) {
    const int b = r >> 3;
    return b * 1024 + ((((c ^ (b & 1)) * 8) + (r & 7)) << 4);
  } else {
    return r * 64 + ((c ^ swz32(r)) << 4);
  }
}

// K-major operands (GemmParams::a_t / b_t: element (r, k) of the M x K or
// N x K operand at X[k * ld + r], as a transposed view stores it).  Their stage
// tile sits in LDS as BK rows (k) of W halves (W = BM or BN), row-major, with
// 16-byte chunk L of row k at chunk L ^ tsw(k).  A DMA moves 64 / (W / 8) whole
// rows; each lane fetches the global chunk that belongs at its LDS slot.
//
// Fragments come from two gfx950 ds_read_b64_tr_b16.  Measured lane layout: in
// every 16-lane group, the 16 lanes' 8-byte reads form a 16 x 4 matrix M (row =
// reading lane); lane i of the group receives M[4 j + i / 4][i % 4] for j = 0..3.
// With lane l of group g = l / 16 pointing at row 16 kk + 8 (l / 32) + 4 h +
// (l % 16) / 4 and column c + 16 (g % 2) + 4 (l % 4), read h = 0, 1 delivers k =
// 16 kk + 8 (l / 32) + 4 h + 0..3 of column c + l % 32: the MFMA 32x32x16 operand
// layout (8 consecutive k of one row / column per lane).  A group reads 4 rows x
// 32 B; tsw spreads the 4 rows over 4 distinct 32-byte bank groups (W = 64, 128,
// 256), so the reads are conflict-free.
__device__ __forceinline__ int tsw(int k) { return (k & 3) << 1; }

template <int W>
__device__ __forceinline__ void dma_source_t(int g, int lane, int& row, int& chunk) {
  constexpr int kChunks = W / 8;       // 16-byte chunks per row (>= 8)
  constexpr int kRows = 64 / kChunks;  // rows per 1 KiB DMA
  static_assert(kChunks >= 8 && 64 % kChunks == 0, "K-major tile width");
  row = g * kRows + lane / kChunks;
  chunk = (lane % kChunks) ^ tsw(row);
}

// Byte offset, in a K-major tile of width W, of the lane's first transposed read
// for k-step kk and the 32-wide block at column cb; the second read is 4 rows
// (4 W * 2 bytes) further.
template <int W>
__device__ __forceinline__ int frag_offset_t(int lane, int kk, int cb) {
  const int k = 16 * kk + 8 * (lane >> 5) + ((lane & 15) >> 2);
  const int col = cb + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  return k * (W * 2) + (((col >> 3) ^ tsw(k)) << 4) + ((col & 7) << 1);
}

typedef short nt_short4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) nt_short4 nt_lds_short4;

__device__ __forceinline__ half8 read_frag_t(const unsigned char* p, int w_bytes) {
  const nt_short4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((nt_lds_short4*)p);
  const nt_short4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((nt_lds_short4*)(p + 4 * w_bytes));
  typedef short short8 __attribute__((ext_vector_type(8)));
  const short8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(half8, v);
}

template <class C>
using NtAcc = float16v[C::FM][C::FN];

// Tile id -> (m0, n0).  Consecutive tile ids walk groups of kGroupM M-tiles
// (M fastest) before moving to the next N-tile, so the tiles resident on one
// XCD at a time (after the XCD remap of workgroup ids) form a kGroupM x (n)
// block that reuses both its A panels and its B panels from that XCD's L2.
template <class C>
__device__ __forceinline__ void tile_origin(const GemmParams& p, int64_t tile, int64_t& m0,
                                            int64_t& n0) {
  const int64_t mtiles = cdiv(p.M, C::BM);
  const int64_t ntiles = cdiv(p.N, C::BN);
  constexpr int64_t kGroupM = 8;
  const int64_t per_group = kGroupM * ntiles;
  const int64_t first_m = (tile / per_group) * kGroupM;
  const int64_t group_m = mtiles - first_m < kGroupM ? mtiles - first_m : kGroupM;
  const int64_t in_group = tile % per_group;
  m0 = (first_m + in_group % group_m) * C::BM;
  n0 = (in_group / group_m) * C::BN;
}

// EPI_GLU epilogue: the gate (and up) values of each 32x32 block are loaded
// before the block's first store.
template <class C>
__device__ __forceinline__ void nt_glu_epilogue(const GemmParams& p, int64_t m0, int64_t n0,
                                                const NtAcc<C>& acc) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int wm = wave / C::kWavesN;
  const int wn = wave % C::kWavesN;
  const int lr = lane & 31;
  const int lh = lane >> 5;
#pragma unroll
  for (int i = 0; i < C::FM; ++i) {
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
      const int64_t row_base = m0 + wm * C::WM + i * 32;
      const int64_t col = n0 + wn * C::WN + j * 32 + lr;
      if (col >= p.N) continue;
      half_t g[16], u[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = row_base + 8 * (r >> 2) + 4 * lh + (r & 3);
        const bool in = row < p.M;
        g[r] = in ? p.glu_gate[row * p.ldgate + col] : (half_t)0;
        u[r] = in && p.glu == 2 ? p.glu_up[row * p.ldup + col] : (half_t)0;
      }
      const float b = p.bias ? (float)p.bias[col] : 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = row_base + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (row >= p.M) continue;
        glu_apply(p, row, col, row * p.ldc + col, acc[i][j][r] * p.alpha + b, g[r], u[r]);
      }
    }
  }
}

// EPI_GLU epilogue through LDS, with 16-byte gate / up / output accesses.
// For each wave row group q in turn, the waves of that group write their
// values h = fp16(alpha acc + bias) into an LDS tile [WM][BN + 8]; then every
// thread of the workgroup takes 8-column chunks of it (kGluBatch at a time:
// gate / up / staged chunks first, then the activation and the stores).
// Needs N, the leading dimensions and the base pointers 16-byte granular
// (p.glu_vec) and the whole workgroup (it synchronises); the stage ring is
// drained and free once the main loop has returned.
template <class C>
struct GluStage {
  static constexpr int kPitch = C::BN + 8;  // halves per staged row (bank spread)
  static constexpr int kChunksRow = C::BN / 8;
  static constexpr int kPer = C::WM * kChunksRow / C::kThreads;
  static constexpr int kBatch = kPer < 4 ? kPer : 4;
  static constexpr int kBytes = C::WM * kPitch * 2;
  static constexpr bool kOk = C::WM * kChunksRow % C::kThreads == 0 && kPer >= 1 && kPer <= 8 &&
                              kPer % kBatch == 0;
};

template <class C>
__device__ __forceinline__ void nt_glu_epilogue_lds(const GemmParams& p, int64_t m0, int64_t n0,
                                                    const NtAcc<C>& acc, unsigned char* smem) {
  using G = GluStage<C>;
  half_t* stage = reinterpret_cast<half_t*>(smem);
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int wm = wave / C::kWavesN;
  const int wn = wave % C::kWavesN;
  const int lr = lane & 31;
  const int lh = lane >> 5;
  wait_vm<0>();
  __syncthreads();
#pragma unroll 1
  for (int q = 0; q < C::BM / C::WM; ++q) {
    if (wm == q) {
#pragma unroll
      for (int i = 0; i < C::FM; ++i) {
#pragma unroll
        for (int j = 0; j < C::FN; ++j) {
          const int col_l = wn * C::WN + j * 32 + lr;
          const int64_t col = n0 + col_l;
          const float b = p.bias && col < p.N ? (float)p.bias[col] : 0.0f;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row_l = i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
            stage[row_l * G::kPitch + col_l] = f32_to_f16(acc[i][j][r] * p.alpha + b);
          }
        }
      }
    }
    __syncthreads();
#pragma unroll 1
    for (int k0 = 0; k0 < G::kPer; k0 += G::kBatch) {
      half8 h[G::kBatch], g[G::kBatch], u[G::kBatch];
      int64_t row[G::kBatch], col[G::kBatch];
      bool in[G::kBatch];
#pragma unroll
      for (int k = 0; k < G::kBatch; ++k) {
        const int c = tid + (k0 + k) * C::kThreads;
        const int row_l = c / G::kChunksRow;
        const int c8 = (c % G::kChunksRow) * 8;
        row[k] = m0 + q * C::WM + row_l;
        col[k] = n0 + c8;
        in[k] = row[k] < p.M && col[k] < p.N;
        h[k] = *reinterpret_cast<const half8*>(stage + row_l * G::kPitch + c8);
        g[k] = in[k] ? *reinterpret_cast<const half8*>(p.glu_gate + row[k] * p.ldgate + col[k])
                     : half8{};
        u[k] = in[k] && p.glu == 2
                   ? *reinterpret_cast<const half8*>(p.glu_up + row[k] * p.ldup + col[k])
                   : half8{};
      }
#pragma unroll
      for (int k = 0; k < G::kBatch; ++k) {
        if (!in[k]) continue;
        half8 o0, o1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const SwigluTerms t = swiglu_terms((float)g[k][e]);
          const float v = (float)h[k][e];
          if (p.glu == 1) {
            o1[e] = f32_to_f16(t.act * v);
          } else {
            o0[e] = f32_to_f16((v * (float)u[k][e]) * swiglu_slope(t));
            o1[e] = f32_to_f16(v * t.act);
          }
        }
        half_t* c_out = reinterpret_cast<half_t*>(p.C) + row[k] * p.ldc + col[k];
        if (p.glu == 2)
          *reinterpret_cast<half8*>(c_out) = o0;
        else if (p.glu_store_c)
          *reinterpret_cast<half8*>(c_out) = h[k];
        *reinterpret_cast<half8*>(p.glu_out + row[k] * p.ldglu + col[k]) = o1;
      }
    }
    __syncthreads();
  }
}

// Epilogue of one output tile.  Lane holds D[8 (r / 4) + 4 (lane / 32) + r %
// 4][lane % 32] of each 32x32 block in register r.
// Rank-16 term of a 32x32 block on one v_mfma_f32_32x32x16_f16 (EPI_LORA,
// EPI_RANK, or folded into a split-K partial): A = Z rows (row lane % 32,
// ranks 8 (lane / 32) .. + 7), B = (rank, column) -- a lora_B row ([N, 16],
// one 16-byte load; vec_b) or a lora_A column ([16, ldlb], eight 2-byte
// loads).  A wave loads the operands of all its FM x FN blocks (and their
// bias) before it finishes any block, so it waits for them once instead of
// once per block.
template <class C>
struct RankOps {
  half8 za[C::FM];
  half8 zb[C::FN];
  __device__ __forceinline__ void load(const GemmParams& p, int64_t m0, int64_t n0, int wm, int wn,
                                       int lr, int lh, bool vec_b) {
    const half8 zero = half8{};
#pragma unroll
    for (int i = 0; i < C::FM; ++i) {
      const int64_t zr = m0 + wm * C::WM + i * 32 + lr;
      za[i] = zr < p.M ? *reinterpret_cast<const half8*>(p.lz + zr * 16 + 8 * lh) : zero;
    }
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
      const int64_t col = n0 + wn * C::WN + j * 32 + lr;
      zb[j] = zero;
      if (col < p.N) {
        if (vec_b) {
          zb[j] = *reinterpret_cast<const half8*>(p.lb + col * 16 + 8 * lh);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) zb[j][e] = p.lb[(8 * lh + e) * p.ldlb + col];
        }
      }
    }
  }
  __device__ __forceinline__ float16v block(int i, int j) const {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(za[i], zb[j], float16v{}, 0, 0, 0);
  }
};

template <class C>
__device__ __forceinline__ void load_bias(const GemmParams& p, int64_t n0, int wn, int lr,
                                          float (&bias)[C::FN]) {
#pragma unroll
  for (int j = 0; j < C::FN; ++j) {
    const int64_t col = n0 + wn * C::WN + j * 32 + lr;
    bias[j] = p.bias && col < p.N ? (float)p.bias[col] : 0.0f;
  }
}

// fp16 epilogue (plain / LoRA / rank-16, beta = 0) with the tile staged
// through LDS: per wave row group, the waves write their rounded outputs
// (the values and rounding order of nt_epilogue's direct stores) into
// [WM][BN + 8], then the workgroup stores them as 16-byte row chunks -- one
// store instruction per 1 KiB instead of per 128 B.  Needs N, ldc and C
// 16-byte granular (p.c_vec) and the whole workgroup.  The stores are
// non-temporal (the kernel does not read its output): for a 990 x 8960
// output (17.7 MB, written when every tile finishes at once) the 256x256
// product takes ~1.5 us less; a SwiGLU reading that output next takes ~1.4
// us more (it no longer finds it in the last-level cache), and the whole
// decoder layer measured 0.4-1 % faster with them.
template <class C, int EPI>
__device__ __forceinline__ void nt_epilogue_staged(const GemmParams& p, int64_t m0, int64_t n0,
                                                   const NtAcc<C>& acc, unsigned char* smem) {
  using G = GluStage<C>;
  half_t* stage = reinterpret_cast<half_t*>(smem);
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int wm = wave / C::kWavesN;
  const int wn = wave % C::kWavesN;
  const int lr = lane & 31;
  const int lh = lane >> 5;
  constexpr bool kRank = EPI == EPI_LORA || EPI == EPI_RANK;
  RankOps<C> ops;
  if constexpr (kRank) ops.load(p, m0, n0, wm, wn, lr, lh, EPI == EPI_LORA);
  float bias[C::FN];
  load_bias<C>(p, n0, wn, lr, bias);
  wait_vm<0>();
  __syncthreads();
#pragma unroll 1
  for (int q = 0; q < C::BM / C::WM; ++q) {
    if (wm == q) {
#pragma unroll
      for (int i = 0; i < C::FM; ++i) {
#pragma unroll
        for (int j = 0; j < C::FN; ++j) {
          const int col_l = wn * C::WN + j * 32 + lr;
          float16v extra = float16v{};
          if constexpr (kRank) extra = ops.block(i, j);
          const float b = bias[j];
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row_l = i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
            half_t h;
            if constexpr (EPI == EPI_LORA) {
              const float y = (float)f32_to_f16(acc[i][j][r] * p.alpha + b);
              const float lora = (float)f32_to_f16(extra[r]);
              const float scaled = (float)f32_to_f16(lora * p.lscale);
              h = f32_to_f16(y + scaled);
            } else if constexpr (EPI == EPI_RANK) {
              h = f32_to_f16(acc[i][j][r] + extra[r]);
            } else {
              h = f32_to_f16(acc[i][j][r] * p.alpha + b);
            }
            stage[row_l * G::kPitch + col_l] = h;
          }
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < G::kPer; ++k) {
      const int c = tid + k * C::kThreads;
      const int row_l = c / G::kChunksRow;
      const int c8 = (c % G::kChunksRow) * 8;
      const int64_t row = m0 + q * C::WM + row_l;
      const int64_t col = n0 + c8;
      if (row < p.M && col < p.N)
        __builtin_nontemporal_store(
            *reinterpret_cast<const half8*>(stage + row_l * G::kPitch + c8),
            reinterpret_cast<half8*>(reinterpret_cast<half_t*>(p.C) + row * p.ldc + col));
    }
    __syncthreads();
  }
}

// `smem`: the kernel's LDS, at least GluStage<C>::kBytes (staged epilogues).
template <class C, int CT, int EPI>
__device__ __forceinline__ void nt_epilogue(const GemmParams& p, int64_t m0, int64_t n0,
                                            const NtAcc<C>& acc, unsigned char* smem = nullptr,
                                            int64_t split = 0) {
  if constexpr (EPI == EPI_GLU) {
    if constexpr (GluStage<C>::kOk) {
      if (p.glu_vec) {
        nt_glu_epilogue_lds<C>(p, m0, n0, acc, smem);
        return;
      }
    }
    nt_glu_epilogue<C>(p, m0, n0, acc);
    return;
  }
  if constexpr (CT == SS_F16 && EPI != EPI_PARTIAL && GluStage<C>::kOk) {
    if (p.c_vec && smem) {
      nt_epilogue_staged<C, EPI>(p, m0, n0, acc, smem);
      return;
    }
  }
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int wm = wave / C::kWavesN;
  const int wn = wave % C::kWavesN;
  const int lr = lane & 31;  // column within a 32x32 block
  const int lh = lane >> 5;
  // Split 0 of a rank-16 (dX) product adds dZ . A to its partial, so the
  // reduce is a plain sum (fold_rank); split 0 of a LoRA forward stores the
  // rounded LoRA term to lora_plane.  Same MFMA as the unsplit epilogue.
  const bool lora_plane = EPI == EPI_PARTIAL && p.lora_plane && split == 0;
  const bool rank = EPI == EPI_LORA || EPI == EPI_RANK ||
                    (EPI == EPI_PARTIAL && p.fold_rank && split == 0) || lora_plane;
  RankOps<C> ops;
  if (rank) ops.load(p, m0, n0, wm, wn, lr, lh, EPI == EPI_LORA || lora_plane);
  float bias[C::FN];
  if constexpr (EPI != EPI_PARTIAL) load_bias<C>(p, n0, wn, lr, bias);
#pragma unroll
  for (int i = 0; i < C::FM; ++i) {
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
      const int64_t row_base = m0 + wm * C::WM + i * 32;
      const int64_t col = n0 + wn * C::WN + j * 32 + lr;
      if constexpr (EPI == EPI_PARTIAL) {
        float16v extra = float16v{};
        if (rank) extra = ops.block(i, j);
        if (col >= p.N) continue;
        float* part = p.part + split * p.M * p.N;
        if (lora_plane) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int64_t row = row_base + 8 * (r >> 2) + 4 * lh + (r & 3);
            if (row >= p.M) continue;
            part[row * p.N + col] = acc[i][j][r];
            p.lora_plane[row * p.N + col] =
                f32_to_f16((float)f32_to_f16(extra[r]) * p.lscale);
          }
          continue;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = row_base + 8 * (r >> 2) + 4 * lh + (r & 3);
          if (row < p.M) part[row * p.N + col] = acc[i][j][r] + extra[r];
        }
        continue;
      }
      float16v extra = float16v{};
      if constexpr (EPI == EPI_LORA || EPI == EPI_RANK) extra = ops.block(i, j);
      if (col >= p.N) continue;
      const float b = bias[j];
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

}  // namespace
}  // namespace ss
