// MFMA GEMM engine for the NF4 projections and the dense fp16 products.
//
// C[M,N] = alpha * A[M,K] . B[K,N] (+ bias) (+ beta * C), fp16 operands on
// v_mfma_f32_16x16x32_f16 with fp32 accumulation.
//
// Operand sources (one loader per kind, chosen at compile time):
//   OP_ROW      fp16, element (r,k) at ptr[r*ld + k]   (K contiguous)
//   OP_COL      fp16, element (r,k) at ptr[k*ld + r]   (R contiguous; the
//               tile is transposed on its way into LDS)
//   OP_NF4_ROW  NF4 weight W[rows, cols] with r = W row, k = W col: the
//               forward Y = X . W^T (reference solution/kernels/nf4_gemm.py:
//               35-71, TRANSPOSE=False)
//   OP_NF4_COL  NF4 weight with r = W col, k = W row: the backward
//               dX = dY . W (nf4_gemm.py TRANSPOSE=True)
// NF4 tiles are decoded in registers with exactly the standalone decoder's
// arithmetic (fp32 scale, fp32 product, one RNE rounding; no contraction),
// so the MFMA consumes the bit-exact dequantized weight.
//
// Tiling: a 256-thread workgroup (4 wave64) owns a BM x BN output tile; the
// K loop walks BK=64 slices (exactly one NF4 block per weight row) through
// two LDS stages.  Global loads for slice k+1 are issued before the MFMAs of
// slice k and written to the other LDS stage afterwards: one barrier per
// slice.  LDS rows are padded by 8 halves (16 B) so the 16 lanes that read one
// MFMA fragment column (16 rows, same k) hit distinct bank groups.

#include <stdlib.h>

#include <mutex>

#include "gemm.h"
#include "soupsuck_amd.h"
#include "rank16.h"
#include "tuning.h"

namespace ss {

constexpr int kThreads = 256;
constexpr int kPad = 8;

union Vec16 {
  uint4 u;
  half8 h;
  uint32_t w[4];
};

// ------------------------------------------------------------ loaders ----
// Each loader moves one R x BK tile of its operand (R = BM for A, BN for B)
// from global memory into registers (load) and from registers into an LDS
// tile laid out as [R][BK + kPad] with k contiguous (store).

template <int R, int BK, int OP>
struct Loader;

// Loads are branch-free on the vector path: an out-of-range chunk reads a
// clamped, valid address and is zeroed when it is written to LDS (a per-chunk
// valid bit).  A divergent vector/scalar if-else writing the same registers
// would force a wait on every outstanding load (write-after-write across the
// exec-masked paths) and serialise the tile fetch.  The scalar path is taken
// only under the uniform `vec` flag (unaligned or K % 8 != 0 operands).

template <int R, int BK>
struct Loader<R, BK, OP_ROW> {
  static constexpr int kChunks = R * BK / 8 / kThreads;
  static_assert(kChunks >= 1 && R * BK / 8 % kThreads == 0, "tile/thread mismatch");
  u32x4 v[kChunks];
  uint32_t ok;
  template <bool VEC>
  __device__ __forceinline__ void load(const half_t* __restrict__ ptr, int64_t ld, int64_t r0,
                       int64_t rmax, int64_t k0, int64_t kmax, const Nf4View&) {
    ok = 0;
    if constexpr (VEC) {
#pragma unroll
      for (int i = 0; i < kChunks; ++i) {
        const int c = threadIdx.x + kThreads * i;
        const int64_t gr = r0 + c / (BK / 8);
        const int64_t gk = k0 + (c % (BK / 8)) * 8;
        const bool in = gr < rmax && gk < kmax;
        ok |= (uint32_t)in << i;
        const int64_t rr = in ? gr : 0;
        const int64_t kk = in ? gk : 0;
        v[i] = *reinterpret_cast<const u32x4*>(ptr + rr * ld + kk);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kChunks; ++i) {
        const int c = threadIdx.x + kThreads * i;
        const int64_t gr = r0 + c / (BK / 8);
        const int64_t gk = k0 + (c % (BK / 8)) * 8;
        half8 t;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          t[j] = (gr < rmax && gk + j < kmax) ? ptr[gr * ld + gk + j] : (half_t)0.0f;
        v[i] = __builtin_bit_cast(u32x4, t);
      }
      ok = ~0u;
    }
  }
  __device__ __forceinline__ void store(half_t* __restrict__ lds, const float*, const float*, float) {
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int c = threadIdx.x + kThreads * i;
      const int row = c / (BK / 8);
      const int kc = c % (BK / 8);
      const u32x4 val = ((ok >> i) & 1u) ? v[i] : u32x4{0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4*>(lds + row * (BK + kPad) + kc * 8) = val;
    }
  }
};

template <int R, int BK>
struct Loader<R, BK, OP_COL> {
  static constexpr int kChunks = R * BK / 8 / kThreads;
  static_assert(kChunks >= 1 && R * BK / 8 % kThreads == 0, "tile/thread mismatch");
  u32x4 v[kChunks];
  uint32_t ok;
  // Lanes walk k fastest so that the transposed 2-byte LDS writes of one
  // instruction land on consecutive addresses (no bank conflicts).
  template <bool VEC>
  __device__ __forceinline__ void load(const half_t* __restrict__ ptr, int64_t ld, int64_t r0,
                       int64_t rmax, int64_t k0, int64_t kmax, const Nf4View&) {
    ok = 0;
    if constexpr (VEC) {
#pragma unroll
      for (int i = 0; i < kChunks; ++i) {
        const int c = threadIdx.x + kThreads * i;
        const int64_t gk = k0 + c % BK;
        const int64_t gr = r0 + (c / BK) * 8;
        const bool in = gk < kmax && gr < rmax;
        ok |= (uint32_t)in << i;
        const int64_t kk = in ? gk : 0;
        const int64_t rr = in ? gr : 0;
        v[i] = *reinterpret_cast<const u32x4*>(ptr + kk * ld + rr);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kChunks; ++i) {
        const int c = threadIdx.x + kThreads * i;
        const int64_t gk = k0 + c % BK;
        const int64_t gr = r0 + (c / BK) * 8;
        half8 t;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          t[j] = (gk < kmax && gr + j < rmax) ? ptr[gk * ld + gr + j] : (half_t)0.0f;
        v[i] = __builtin_bit_cast(u32x4, t);
      }
      ok = ~0u;
    }
  }
  __device__ __forceinline__ void store(half_t* __restrict__ lds, const float*, const float*, float) {
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
      const int c = threadIdx.x + kThreads * i;
      const int k = c % BK;
      const int rc = c / BK;
      const u32x4 val = ((ok >> i) & 1u) ? v[i] : u32x4{0u, 0u, 0u, 0u};
      const half8 h = __builtin_bit_cast(half8, val);
#pragma unroll
      for (int j = 0; j < 8; ++j) lds[(rc * 8 + j) * (BK + kPad) + k] = h[j];
    }
  }
};

// Decode ELEMS consecutive NF4 codes (ELEMS/2 packed bytes in `words`,
// element order = byte order, high nibble first) with one fp32 scale.
template <int ELEMS>
__device__ __forceinline__ void decode_run(const uint32_t* words, float scale,
                                           const float* __restrict__ lut, half_t* out) {
#pragma unroll
  for (int wi = 0; wi < ELEMS / 8; ++wi) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t byte = (words[wi] >> (8 * b)) & 0xffu;
      out[8 * wi + 2 * b] = f32_to_f16(lut[byte >> 4] * scale);
      out[8 * wi + 2 * b + 1] = f32_to_f16(lut[byte & 15u] * scale);
    }
  }
}

struct Nf4Stage {
  bool valid;
  uint32_t q;
  float a2;
};

// Forward weight tile: r = weight row, k = weight column.  Each thread owns
// ELEMS consecutive k of one row; BK = 64 means one NF4 block per row.
template <int R, int BK>
struct Loader<R, BK, OP_NF4_ROW> {
  static constexpr int ELEMS = R * BK / kThreads;
  static_assert(ELEMS == 16 || ELEMS == 32, "NF4 row loader expects 16 or 32 codes per thread");
  static_assert(64 % ELEMS == 0 && BK % ELEMS == 0, "a thread's run must stay in one block");
  static constexpr int kParts = BK / ELEMS;
  uint32_t words[ELEMS / 8];
  Nf4Stage st;
  template <bool VEC>
  __device__ __forceinline__ void load(const half_t*, int64_t, int64_t r0, int64_t rmax, int64_t k0,
                       int64_t kmax, const Nf4View& w) {
    const int row = threadIdx.x / kParts;
    const int part = threadIdx.x % kParts;
    const int64_t gr = r0 + row;
    const int64_t gk = k0 + part * ELEMS;
    st.valid = gr < rmax && gk < kmax;
    // Clamped, always-valid address; invalid runs are zeroed in store().
    const int64_t e = st.valid ? gr * w.cols + gk : 0;
    const uint8_t* src = w.packed + (e >> 1);
    if constexpr (ELEMS == 32) {
      const u32x4 t = *reinterpret_cast<const u32x4*>(src);
      words[0] = t[0]; words[1] = t[1]; words[2] = t[2]; words[3] = t[3];
    } else {
      uint2 t = *reinterpret_cast<const uint2*>(src);
      words[0] = t.x; words[1] = t.y;
    }
    const int64_t block = e >> 6;
    st.q = w.qabs[block];
    st.a2 = w.absmax2[block >> 8];
  }
  __device__ __forceinline__ void store(half_t* __restrict__ lds, const float* __restrict__ code2,
                        const float* __restrict__ lut, float offset) {
    const int row = threadIdx.x / kParts;
    const int part = threadIdx.x % kParts;
    Vec16 out[ELEMS / 8];
    if (st.valid) {
      const float product = code2[st.q] * st.a2;
      const float scale = product + offset;
      decode_run<ELEMS>(words, scale, lut, reinterpret_cast<half_t*>(out));
    } else {
#pragma unroll
      for (int i = 0; i < ELEMS / 8; ++i) out[i].u = make_uint4(0, 0, 0, 0);
    }
    half_t* dst = lds + row * (BK + kPad) + part * ELEMS;
#pragma unroll
    for (int i = 0; i < ELEMS / 8; ++i) *reinterpret_cast<uint4*>(dst + 8 * i) = out[i].u;
  }
};

// Backward weight tile: r = weight column, k = weight row.  Each thread owns
// ELEMS consecutive weight columns of one weight row (one NF4 block run) and
// writes them transposed, so LDS again holds [r][k] with k contiguous.
template <int R, int BK>
struct Loader<R, BK, OP_NF4_COL> {
  static constexpr int ELEMS = R * BK / kThreads;
  static_assert(ELEMS == 16 || ELEMS == 32, "NF4 column loader expects 16 or 32 codes per thread");
  static_assert(kThreads % BK == 0 && R / ELEMS == kThreads / BK, "tile/thread mismatch");
  uint32_t words[ELEMS / 8];
  Nf4Stage st;
  template <bool VEC>
  __device__ __forceinline__ void load(const half_t*, int64_t, int64_t r0, int64_t rmax, int64_t k0,
                       int64_t kmax, const Nf4View& w) {
    const int krow = threadIdx.x % BK;
    const int cg = threadIdx.x / BK;
    const int64_t gk = k0 + krow;
    const int64_t gr = r0 + cg * ELEMS;
    st.valid = gk < kmax && gr < rmax;
    const int64_t e = st.valid ? gk * w.cols + gr : 0;
    const uint8_t* src = w.packed + (e >> 1);
    if constexpr (ELEMS == 32) {
      const u32x4 t = *reinterpret_cast<const u32x4*>(src);
      words[0] = t[0]; words[1] = t[1]; words[2] = t[2]; words[3] = t[3];
    } else {
      uint2 t = *reinterpret_cast<const uint2*>(src);
      words[0] = t.x; words[1] = t.y;
    }
    const int64_t block = e >> 6;
    st.q = w.qabs[block];
    st.a2 = w.absmax2[block >> 8];
  }
  __device__ __forceinline__ void store(half_t* __restrict__ lds, const float* __restrict__ code2,
                        const float* __restrict__ lut, float offset) {
    const int krow = threadIdx.x % BK;
    const int cg = threadIdx.x / BK;
    half_t vals[ELEMS];
    if (st.valid) {
      const float product = code2[st.q] * st.a2;
      const float scale = product + offset;
      decode_run<ELEMS>(words, scale, lut, vals);
    } else {
#pragma unroll
      for (int j = 0; j < ELEMS; ++j) vals[j] = (half_t)0.0f;
    }
#pragma unroll
    for (int j = 0; j < ELEMS; ++j) lds[(cg * ELEMS + j) * (BK + kPad) + krow] = vals[j];
  }
};

// ------------------------------------------------------------- kernel ----

template <int BM, int BN, int BK, int WM, int WN>
struct Tile {
  static constexpr int kBM = BM, kBN = BN, kBK = BK, kWM = WM, kWN = WN;
  static constexpr int kWavesN = BN / WN;
  static constexpr int kWavesM = BM / WM;
  static_assert(kWavesN * kWavesM == kThreads / kWave, "4 waves per workgroup");
  static_assert(WM % 16 == 0 && WN % 16 == 0 && BK % 32 == 0, "MFMA 16x16x32 tiling");
  static constexpr int kLdk = BK + kPad;
};

template <class T, int OPA, int OPB, int CT, int EPI, bool VEC>
__global__ __launch_bounds__(kThreads) void gemm_kernel(GemmParams p) {
  if (p.alpha_dev) p.alpha *= *p.alpha_dev;
  constexpr int BM = T::kBM, BN = T::kBN, BK = T::kBK, WM = T::kWM, WN = T::kWN;
  constexpr int LDK = T::kLdk;
  constexpr bool kNf4 = OPA >= OP_NF4_ROW || OPB >= OP_NF4_ROW;
  __shared__ __attribute__((aligned(16))) half_t sA[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) half_t sB[2][BN * LDK];
  __shared__ float s_code2[kNf4 ? 256 : 1];
  __shared__ float s_lut[16];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int wm = wave / T::kWavesN;
  const int wn = wave % T::kWavesN;
  // Workgroups are dispatched round-robin over the 8 XCDs (each with its own
  // L2).  Renumber so that every XCD owns a contiguous range of tiles, and walk
  // tiles M-fastest: the M-tiles that share one weight (B) tile run back to
  // back on the same XCD and re-read it from that XCD's L2.
  const int64_t mtiles = cdiv(p.M, BM);
  const int64_t tile = p.remap ? xcd_remap(blockIdx.x, gridDim.x) : (int64_t)blockIdx.x;
  const int64_t m0 = (tile % mtiles) * BM;
  const int64_t n0 = (tile / mtiles) * BN;

  float offset = 0.0f;
  if constexpr (kNf4) {
    s_code2[tid] = p.w.code2[tid];
    if (tid < 16) s_lut[tid] = kNF4[tid];
    offset = p.w.offset[0];
  }

  Loader<BM, BK, OPA> la;
  Loader<BN, BK, OPB> lb;
  const int64_t ktiles = cdiv(p.K, BK);

  if (ktiles > 0) {
    la.template load<VEC>(p.A, p.lda, m0, p.M, 0, p.K, p.w);
    lb.template load<VEC>(p.B, p.ldb, n0, p.N, 0, p.K, p.w);
  }
  __syncthreads();  // code tables visible before the first decode
  if (ktiles > 0) {
    la.store(sA[0], s_code2, s_lut, offset);
    lb.store(sB[0], s_code2, s_lut, offset);
  }
  __syncthreads();

  float4v acc[WM / 16][WN / 16];
#pragma unroll
  for (int i = 0; i < WM / 16; ++i)
#pragma unroll
    for (int j = 0; j < WN / 16; ++j) acc[i][j] = float4v{0.f, 0.f, 0.f, 0.f};

  const int frag_row = lane & 15;
  const int frag_k = (lane >> 4) * 8;

  for (int64_t kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < ktiles;
    if (more) {
      const int64_t k0 = (kt + 1) * BK;
      la.template load<VEC>(p.A, p.lda, m0, p.M, k0, p.K, p.w);
      lb.template load<VEC>(p.B, p.ldb, n0, p.N, k0, p.K, p.w);
    }
    const half_t* a_tile = sA[cur] + (wm * WM + frag_row) * LDK + frag_k;
    const half_t* b_tile = sB[cur] + (wn * WN + frag_row) * LDK + frag_k;
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      half8 af[WM / 16];
      half8 bf[WN / 16];
#pragma unroll
      for (int i = 0; i < WM / 16; ++i)
        af[i] = *reinterpret_cast<const half8*>(a_tile + i * 16 * LDK + ks * 32);
#pragma unroll
      for (int j = 0; j < WN / 16; ++j)
        bf[j] = *reinterpret_cast<const half8*>(b_tile + j * 16 * LDK + ks * 32);
#pragma unroll
      for (int i = 0; i < WM / 16; ++i)
#pragma unroll
        for (int j = 0; j < WN / 16; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      la.store(sA[cur ^ 1], s_code2, s_lut, offset);
      lb.store(sB[cur ^ 1], s_code2, s_lut, offset);
    }
    __syncthreads();
  }

  // Epilogue: lane holds D[4*(lane/16) + r][lane%16] of each 16x16 tile.
  const int crow = (lane >> 4) * 4;
  const int ccol = lane & 15;
#pragma unroll
  for (int i = 0; i < WM / 16; ++i) {
#pragma unroll
    for (int j = 0; j < WN / 16; ++j) {
      const int64_t row_base = m0 + wm * WM + i * 16;
      const int64_t col_base = n0 + wn * WN + j * 16;
      float4v extra = float4v{0.f, 0.f, 0.f, 0.f};
      if constexpr (EPI != EPI_PLAIN) {
        // Rank-16 product for this 16x16 tile on one v_mfma_f32_16x16x16_f16:
        // A = Z rows (lane: row lane%16, r = 4*(lane/16)..+3), B = (r, column).
        const int rq = (lane >> 4) * 4;
        const int64_t zr = row_base + (lane & 15);
        const int64_t bc = col_base + (lane & 15);
        half4 za, zb;
        if (zr < p.M) {
          za = *reinterpret_cast<const half4*>(p.lz + zr * 16 + rq);
        } else {
          za = half4{(half_t)0.0f, (half_t)0.0f, (half_t)0.0f, (half_t)0.0f};
        }
        if (bc < p.N) {
          if constexpr (EPI == EPI_LORA) {
            zb = *reinterpret_cast<const half4*>(p.lb + bc * 16 + rq);
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) zb[q] = p.lb[(rq + q) * p.ldlb + bc];
          }
        } else {
          zb = half4{(half_t)0.0f, (half_t)0.0f, (half_t)0.0f, (half_t)0.0f};
        }
        extra = __builtin_amdgcn_mfma_f32_16x16x16f16(za, zb, extra, 0, 0, 0);
      }
      const int64_t col = col_base + ccol;
      if (col >= p.N) continue;
      const float b = p.bias ? (float)p.bias[col] : 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = row_base + crow + r;
        if (row < p.M) {
          const int64_t idx = row * p.ldc + col;
          if constexpr (EPI == EPI_LORA) {
            const float y = (float)f32_to_f16(acc[i][j][r] * p.alpha + b);
            const float lora = (float)f32_to_f16(extra[r]);
            const float scaled = (float)f32_to_f16(lora * p.lscale);
            reinterpret_cast<half_t*>(p.C)[idx] = f32_to_f16(y + scaled);
          } else if constexpr (EPI == EPI_RANK) {
            store_c<CT>(p.C, idx, acc[i][j][r] + extra[r], p.beta);
          } else {
            const float v = acc[i][j][r] * p.alpha + b;
            store_c<CT>(p.C, idx, v, p.beta);
          }
        }
      }
    }
  }
}

// ------------------------------------------------------------- launch ----

using TileBig = Tile<128, 128, 64, 64, 64>;
using TileSmall = Tile<64, 64, 64, 32, 32>;
using TileWide = Tile<256, 128, 64, 128, 64>;
using TileTall = Tile<128, 256, 64, 64, 128>;

static int remap_setting() { return SS_TUNE_GEMM_REMAP; }

template <class T, int OPA, int OPB, int CT, int EPI>
static int launch(const GemmParams& p0, hipStream_t stream, const char* name) {
  GemmParams p = p0;
  p.remap = remap_setting();
  dim3 grid((unsigned)(cdiv(p.N, T::kBN) * cdiv(p.M, T::kBM)));
  // Vector (branch-free, 16-byte) operand loads when both operands allow them;
  // the scalar variant is a separate instantiation so the hot loop stays small.
  constexpr bool kAnyNf4 = OPA >= OP_NF4_ROW || OPB >= OP_NF4_ROW;
  const bool vec = (OPA >= OP_NF4_ROW || p.a_vec) && (OPB >= OP_NF4_ROW || p.b_vec);
  if (kAnyNf4 || vec) {
    hipLaunchKernelGGL((gemm_kernel<T, OPA, OPB, CT, EPI, true>), grid, dim3(kThreads), 0, stream,
                       p);
  } else {
    hipLaunchKernelGGL((gemm_kernel<T, OPA, OPB, CT, EPI, false>), grid, dim3(kThreads), 0, stream,
                       p);
  }
  SS_CHECK_LAUNCH(name);
  return SS_OK;
}

// Tile choice: 128x128 when it still gives every CU a workgroup, else 64x64.
// The 256x128 / 128x256 tiles (one wave per SIMD) measured slower than
// 128x128 at every Qwen shape, so only SS_TUNE_GEMM_TILE (1..4 = 64x64,
// 128x128, 256x128, 128x256; a build-time constant) selects them.
enum TileId { TILE_AUTO = 0, TILE_SMALL = 1, TILE_BIG = 2, TILE_WIDE = 3, TILE_TALL = 4 };

static int tile_override() { return SS_TUNE_GEMM_TILE; }

static int pick_tile(int64_t m, int64_t n) {
  const int forced = tile_override();
  if (forced >= TILE_SMALL && forced <= TILE_TALL) return forced;
  if (cdiv(m, 128) * cdiv(n, 128) >= 256) return TILE_BIG;
  return TILE_SMALL;
}

// SS_TUNE_GEMM_NT = 0 keeps dense NT products on the register-staged kernel.
static bool nt_enabled() { return SS_TUNE_GEMM_NT != 0; }

template <int OPA, int OPB, int CT, int EPI = EPI_PLAIN>
static int dispatch(const GemmParams& p, hipStream_t stream, const char* name,
                    void* partials = nullptr, size_t partial_bytes = 0) {
  if constexpr (OPA >= OP_NF4_ROW || OPB >= OP_NF4_ROW) {
    // The in-register NF4 decoders handle 128- and 64-row weight tiles.
    if (cdiv(p.M, 128) * cdiv(p.N, 128) >= 256 || tile_override() == TILE_BIG)
      return launch<TileBig, OPA, OPB, CT, EPI>(p, stream, name);
    return launch<TileSmall, OPA, OPB, CT, EPI>(p, stream, name);
  } else {
    // The pipelined direct-to-LDS kernel when its alignment / K % 64
    // requirements hold: K-contiguous operands as they are, K-major (OP_COL)
    // ones read through transposed LDS reads (plain epilogues).
    if (nt_enabled()) {
      GemmParams q = p;
      q.remap = remap_setting();
      q.a_t = OPA == OP_COL;
      q.b_t = OPB == OP_COL;
      const int rc = gemm_nt(q, CT, EPI, stream, partials, partial_bytes);
      if (rc != SS_ERR_UNSUPPORTED) return rc;
    }
    switch (pick_tile(p.M, p.N)) {
      case TILE_WIDE: return launch<TileWide, OPA, OPB, CT, EPI>(p, stream, name);
      case TILE_TALL: return launch<TileTall, OPA, OPB, CT, EPI>(p, stream, name);
      case TILE_BIG: return launch<TileBig, OPA, OPB, CT, EPI>(p, stream, name);
      default: return launch<TileSmall, OPA, OPB, CT, EPI>(p, stream, name);
    }
  }
}

static bool aligned16(const void* ptr, int64_t ld) {
  return reinterpret_cast<uintptr_t>(ptr) % 16 == 0 && ld % 8 == 0;
}

}  // namespace ss

using namespace ss;

// Decode-first workspace: the fp16 weight (forward [N,K], backward its
// transpose), rounded up to 256 bytes, followed by the fp32 split-K partials
// of the dense product when it is split.
static size_t decoded_bytes(int64_t n, int64_t k) {
  return ((size_t)n * (size_t)k * sizeof(uint16_t) + 255) / 256 * 256;
}

// From T rows on, decoding W once into fp16 (one 2.5 B/weight HBM pass) and
// running the dense MFMA GEMM beats decoding every W tile again for each of
// the ceil(T/BM) row tiles: in-loop decode costs about 1/(2*BM) VALU decodes
// per flop, more than the VALU can issue next to full-rate MFMA.
// SS_TUNE_NF4_DECODE_FIRST_T sets the crossover.
static int64_t decode_first_threshold() { return SS_TUNE_NF4_DECODE_FIRST_T; }

// Scratch the forward alone needs (the forward part of
// ss_nf4_gemm_workspace_size).
static size_t fwd_workspace_bytes(int64_t t, int64_t n, int64_t k) {
  if (n <= 0 || k <= 0 || t <= 0) return 0;
  if (t <= ss::kSkinnyMaxT) {
    size_t fwd = ss::skinny_partial_bytes(t, n, k);
    const size_t fwd_stream = ss::stream_partial_bytes(t, n, k);
    if (fwd_stream > fwd) fwd = fwd_stream;
    const size_t fwd_fused = ss::nf4_fused_partial_bytes(t, n, k);
    return fwd_fused > fwd ? fwd_fused : fwd;
  }
  if (t < decode_first_threshold()) return ss::nf4_fused_partial_bytes(t, n, k);
  return decoded_bytes(n, k) + ss::nt_partial_bytes(t, n, k);
}

extern "C" size_t ss_nf4_gemm_workspace_size(int64_t t, int64_t n, int64_t k) {
  const int64_t threshold = decode_first_threshold();
  if (n <= 0 || k <= 0 || t <= 0) return 0;
  if (t <= ss::kSkinnyMaxT) {
    // Forward: skinny-kernel partials.  Backward: decode W^T once and run the
    // split-K dense product (the in-loop decoder streams the weight with too
    // little parallelism at small T).
    size_t fwd = ss::skinny_partial_bytes(t, n, k);
    const size_t fwd_stream = ss::stream_partial_bytes(t, n, k);
    if (fwd_stream > fwd) fwd = fwd_stream;
    const size_t fwd_fused = ss::nf4_fused_partial_bytes(t, n, k);
    if (fwd_fused > fwd) fwd = fwd_fused;
    size_t dx = decoded_bytes(n, k) + ss::nt_partial_bytes(t, k, n);
    const size_t dx_stream = ss::stream_dx_partial_bytes(t, n, k);
    if (dx_stream > dx) dx = dx_stream;
    const size_t dx_fused = ss::nf4_dx_fused_partial_bytes(t, k, n);
    if (dx_fused > dx) dx = dx_fused;
    return fwd > dx ? fwd : dx;
  }
  // Below the threshold the forward may run the fused kernel (its split-K
  // partials); the backward still decodes W^T first: the in-loop column
  // decoder is the fallback without scratch only (measured on MI355X at
  // T = 200, 18944 x 3584: 316 us in-loop against 89 us decode-first).
  size_t dx = decoded_bytes(n, k) + ss::nt_partial_bytes(t, k, n);  // dX [t, k]
  const size_t dx_fused = ss::nf4_dx_fused_partial_bytes(t, k, n);
  if (dx_fused > dx) dx = dx_fused;
  if (t < threshold) {
    const size_t fwd_fused = ss::nf4_fused_partial_bytes(t, n, k);
    return fwd_fused > dx ? fwd_fused : dx;
  }
  const size_t fwd = decoded_bytes(n, k) + ss::nt_partial_bytes(t, n, k);  // Y [t, n]
  return fwd > dx ? fwd : dx;
}

static int check_nf4(const char* fn, const uint8_t* packed, const uint8_t* qabs,
                     const float* absmax2, const float* code2, const float* offset, int64_t n,
                     int64_t k) {
  SS_CHECK_ARG(packed && qabs && absmax2 && code2 && offset, "%s: null NF4 state pointer", fn);
  SS_CHECK_ARG(n > 0 && k > 0, "%s: weight shape [%lld,%lld] must be positive", fn,
               (long long)n, (long long)k);
  if (k % 64 != 0) {
    ss::set_error("%s: fused NF4 GEMM needs K %% 64 == 0 (got K=%lld)", fn, (long long)k);
    return SS_ERR_UNSUPPORTED;
  }
  if (reinterpret_cast<uintptr_t>(packed) % 16 != 0) {
    ss::set_error("%s: packed NF4 storage must be 16-byte aligned", fn);
    return SS_ERR_UNSUPPORTED;
  }
  return SS_OK;
}

namespace ss {

// Build-time switches of the small-T and fused paths (tuning.h).
static bool stream_enabled() { return SS_TUNE_NF4_STREAM != 0; }
static bool nf4_fused_enabled() { return SS_TUNE_NF4_FUSED != 0; }
static bool nf4_fused_forced() { return SS_TUNE_NF4_FUSED == 2; }
static bool nf4_dx_fused_enabled() { return SS_TUNE_NF4_DX_FUSED != 0; }

// Decode-first path with the decode fused into the preparation launch of the
// QLoRA step (rank-16 jobs + decode in one launch): T above the skinny range,
// aligned decode destination.
static bool fuse_decode(const GemmParams& p, int64_t n, int64_t k, void* workspace,
                        size_t workspace_bytes) {
  return p.M > kSkinnyMaxT && workspace && workspace_bytes >= (size_t)n * (size_t)k * 2 &&
         reinterpret_cast<uintptr_t>(workspace) % 16 == 0 && k % 64 == 0;
}

// prep (may be null): rank-16 jobs that must complete before the GEMM; they
// run in one launch ahead of it, together with the decode when the
// decode-first path is taken.
template <int EPI>
static int run_fwd(GemmParams& p, void* workspace, size_t workspace_bytes, hipStream_t s,
                   PrepJobs* prep = nullptr, bool vp = false, bool vg = false) {
  const int64_t n = p.N, k = p.K;
  const bool fused = prep && fuse_decode(p, n, k, workspace, workspace_bytes);
  if (prep && !fused) {
    const int r = launch_prep(*prep, vp, vg, s);
    if (r) return r;
  }
  if (p.M <= kStreamMaxT && workspace && stream_enabled()) {
    const int rc = nf4_stream_fwd(p, EPI, workspace, workspace_bytes, s);
    if (rc != SS_ERR_UNSUPPORTED) return rc;
  }
  if (p.M <= kSkinnyMaxT && workspace && !nf4_fused_forced()) {
    const int rc = nf4_skinny_fwd(p, EPI, workspace, workspace_bytes, s);
    if (rc != SS_ERR_UNSUPPORTED) return rc;
  }
  // With a preparation launch (the QLoRA step) the decode-first path decodes
  // inside that launch, without one of its own: there the fused kernel is
  // taken for one or two 128-row tiles only (measured: at T = 990 the q
  // projection forward takes 34.3 us fused, 31.0 us decode-first).
  const bool fused_pays = prep ? p.M > kSkinnyMaxT && p.M <= 256
                               : p.M > kSkinnyMaxT && gemm_nf4_fwd_preferred(p);
  if (nf4_fused_enabled() && gemm_nf4_fwd_ok(p, EPI) && (nf4_fused_forced() || fused_pays)) {
    // The weight is decoded inside the GEMM; the workspace holds split-K
    // partials only.  A deferred preparation launch carries no decode.
    if (fused) {
      const int r = launch_prep(*prep, vp, vg, s);
      if (r) return r;
    }
    return gemm_nf4_fwd(p, EPI, s, workspace, workspace_bytes);
  }
  if (workspace && workspace_bytes >= (size_t)n * (size_t)k * 2) {
    const Nf4View& w = p.w;
    int r;
    if (fused) {
      prep->dec_kind = kDecodeRows;
      prep->dec_w = w;
      prep->dec_out = reinterpret_cast<half_t*>(workspace);
      prep->dec_rows = n;
      prep->dec_cols = k;
      r = launch_prep(*prep, vp, vg, s);
    } else {
      r = ss_nf4_dequant_nested(w.packed, w.qabs, w.absmax2, w.code2, w.offset,
                                reinterpret_cast<uint16_t*>(workspace), n * k, s);
    }
    if (r) return r;
    p.B = reinterpret_cast<const half_t*>(workspace);
    p.ldb = k;
    p.b_vec = 1;
    const size_t dec = decoded_bytes(n, k);
    void* part = workspace_bytes > dec ? static_cast<char*>(workspace) + dec : nullptr;
    return dispatch<OP_ROW, OP_ROW, SS_F16, EPI>(p, s, "gemm_kernel<f16 nt>", part,
                                                 part ? workspace_bytes - dec : 0);
  }
  return dispatch<OP_ROW, OP_NF4_ROW, SS_F16, EPI>(p, s, "gemm_kernel<nf4 fwd>");
}

template <int EPI>
static int run_dx(GemmParams& p, int64_t n, int64_t k, void* workspace, size_t workspace_bytes,
                  hipStream_t s, PrepJobs* prep = nullptr, bool vp = false, bool vg = false) {
  // Above the streaming range and up to two 128-row tiles, the fused dX
  // decodes each weight tile into LDS (no decoded weight in HBM); a preparation
  // launch then carries the rank-16 jobs only.
  const bool nf4dx = p.M > kStreamDxMaxT && nf4_dx_fused_enabled() && gemm_nf4_dx_ok(p, EPI) &&
                     gemm_nf4_dx_preferred(p);
  const bool fused = !nf4dx && prep && fuse_decode(p, n, k, workspace, workspace_bytes) &&
                     reinterpret_cast<uintptr_t>(p.w.packed) % 8 == 0;
  if (prep && !fused) {
    const int r = launch_prep(*prep, vp, vg, s);
    if (r) return r;
  }
  if (nf4dx) return gemm_nf4_dx(p, EPI, s, workspace, workspace_bytes);
  if (p.M <= kStreamDxMaxT && workspace && stream_enabled()) {
    const int rc = nf4_stream_dx(p, EPI, workspace, workspace_bytes, s);
    if (rc != SS_ERR_UNSUPPORTED) return rc;
  }
  if (workspace && workspace_bytes >= (size_t)n * (size_t)k * 2) {
    // Decode W^T [k, n] once; dX = dY . W is then the K-contiguous NT product.
    const Nf4View& w = p.w;
    int r;
    if (fused) {
      prep->dec_kind = kDecodeTransposed;
      prep->dec_w = w;
      prep->dec_out = reinterpret_cast<half_t*>(workspace);
      prep->dec_rows = n;
      prep->dec_cols = k;
      r = launch_prep(*prep, vp, vg, s);
    } else {
      r = ss_nf4_dequant_nested_t(w.packed, w.qabs, w.absmax2, w.code2, w.offset,
                                  reinterpret_cast<uint16_t*>(workspace), n, k, s);
    }
    if (r) return r;
    p.B = reinterpret_cast<const half_t*>(workspace);
    p.ldb = n;
    p.b_vec = n % 8 == 0;
    const size_t dec = decoded_bytes(n, k);
    void* part = workspace_bytes > dec ? static_cast<char*>(workspace) + dec : nullptr;
    return dispatch<OP_ROW, OP_ROW, SS_F16, EPI>(p, s, "gemm_kernel<f16 nt>", part,
                                                 part ? workspace_bytes - dec : 0);
  }
  return dispatch<OP_ROW, OP_NF4_COL, SS_F16, EPI>(p, s, "gemm_kernel<nf4 dx>");
}

static GemmParams fwd_params(const uint16_t* x, int64_t ldx, int64_t t, const uint8_t* packed,
                             const uint8_t* qabs, const float* absmax2, const float* code2,
                             const float* offset, int64_t n, int64_t k, const uint16_t* bias,
                             uint16_t* y, int64_t ldy) {
  GemmParams p{};
  p.M = t; p.N = n; p.K = k;
  p.A = reinterpret_cast<const half_t*>(x); p.lda = ldx; p.a_vec = aligned16(x, ldx);
  p.w = Nf4View{packed, qabs, absmax2, code2, offset, k};
  p.bias = reinterpret_cast<const half_t*>(bias);
  p.C = y; p.ldc = ldy; p.alpha = 1.0f; p.beta = 0;
  return p;
}

static GemmParams dx_params(const uint16_t* dy, int64_t lddy, int64_t t, const uint8_t* packed,
                            const uint8_t* qabs, const float* absmax2, const float* code2,
                            const float* offset, int64_t n, int64_t k, uint16_t* dx,
                            int64_t lddx, int accumulate) {
  GemmParams p{};
  p.M = t; p.N = k; p.K = n;
  p.A = reinterpret_cast<const half_t*>(dy); p.lda = lddy;
  p.a_vec = aligned16(dy, lddy) && n % 8 == 0;
  p.w = Nf4View{packed, qabs, absmax2, code2, offset, k};
  p.C = dx; p.ldc = lddx; p.alpha = 1.0f; p.beta = accumulate ? 1 : 0;
  return p;
}

}  // namespace ss

extern "C" int ss_nf4_gemm_fwd(const uint16_t* x, int64_t ldx, int64_t t, const uint8_t* packed,
                               const uint8_t* qabs, const float* absmax2, const float* code2,
                               const float* offset, int64_t n, int64_t k, const uint16_t* bias,
                               uint16_t* y, int64_t ldy, void* workspace, size_t workspace_bytes,
                               void* stream) {
  const char* fn = "ss_nf4_gemm_fwd";
  SS_CHECK_ARG(t >= 0, "%s: t=%lld must be >= 0", fn, (long long)t);
  int rc = check_nf4(fn, packed, qabs, absmax2, code2, offset, n, k);
  if (rc) return rc;
  if (t == 0) return SS_OK;
  SS_CHECK_ARG(x && y, "%s: null activation/output pointer", fn);
  SS_CHECK_ARG(ldx >= k && ldy >= n, "%s: leading dimensions too small", fn);
  GemmParams p = fwd_params(x, ldx, t, packed, qabs, absmax2, code2, offset, n, k, bias, y, ldy);
  return run_fwd<EPI_PLAIN>(p, workspace, workspace_bytes, (hipStream_t)stream);
}

// ------------------------------------------------------ no-alloc forward ---
// ss_nf4_gemm_fwd_noalloc runs ss_nf4_gemm_fwd's dispatch with its scratch in
// a fixed device array instead of a caller workspace.  Every GPU the library
// runs on holds its own copy of the array (64 MiB) until the process ends;
// its address on the current device is looked up once per device with
// hipGetSymbolAddress.  The forward's scratch holds split-K / stage-group
// partial planes that each call writes in full before reading (and, at
// T >= 256 for weights small enough, the decoded weight), so nothing in it
// has to start at zero.  Calls that overlap in time on one GPU share the
// array and race.
namespace {

constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
__device__ __align__(256) static unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];

int scratch_on_current_device(const char* fn, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    ss::set_error("%s: hipGetDevice failed: %s", fn, hipGetErrorString(e));
    return SS_ERR_LAUNCH;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    ss::set_error("%s: device index %d outside 0..%d", fn, dev, kMaxDevices - 1);
    return SS_ERR_UNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      ss::set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", fn, dev,
                    hipGetErrorString(e));
      return SS_ERR_LAUNCH;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return SS_OK;
}

}  // namespace

extern "C" int ss_nf4_gemm_fwd_noalloc(const uint16_t* x, int64_t ldx, int64_t t,
                                       const uint8_t* packed, const uint8_t* qabs,
                                       const float* absmax2, const float* code2,
                                       const float* offset, int64_t n, int64_t k,
                                       const uint16_t* bias, uint16_t* y, int64_t ldy,
                                       void* stream) {
  const char* fn = "ss_nf4_gemm_fwd_noalloc";
  SS_CHECK_ARG(t >= 0, "%s: t=%lld must be >= 0", fn, (long long)t);
  int rc = check_nf4(fn, packed, qabs, absmax2, code2, offset, n, k);
  if (rc) return rc;
  if (t == 0) return SS_OK;
  SS_CHECK_ARG(x && y, "%s: null activation/output pointer", fn);
  SS_CHECK_ARG(ldx >= k && ldy >= n, "%s: leading dimensions too small", fn);
  // The streaming, skinny and fused kernels read X with 16-byte loads.  An X they cannot
  // take sends run_fwd to the decode-first path, as ss_nf4_gemm_fwd with its full
  // workspace does, so the scratch must then hold the decoded weight and the dense
  // product's partials; sizing it for the fast paths alone would fall through to the
  // in-loop decoder, a different kernel.
  const bool x_vec = reinterpret_cast<uintptr_t>(x) % 16 == 0 && ldx % 8 == 0;
  const size_t need = x_vec ? fwd_workspace_bytes(t, n, k)
                            : decoded_bytes(n, k) + ss::nt_partial_bytes(t, n, k);
  SS_CHECK_ARG(need <= kNoAllocScratchBytes,
               "%s: T=%lld N=%lld K=%lld needs %zu bytes of scratch, more than the fixed "
               "%zu-byte device scratch of this entry point; use ss_nf4_gemm_fwd with a "
               "workspace of ss_nf4_gemm_workspace_size() bytes",
               fn, (long long)t, (long long)n, (long long)k, need, kNoAllocScratchBytes);
  void* ws = nullptr;
  if (need) {
    rc = scratch_on_current_device(fn, &ws);
    if (rc) return rc;
  }
  GemmParams p = fwd_params(x, ldx, t, packed, qabs, absmax2, code2, offset, n, k, bias, y, ldy);
  return run_fwd<EPI_PLAIN>(p, ws, need, (hipStream_t)stream);
}

extern "C" int ss_qlora_fwd(const uint16_t* x, int64_t ldx, int64_t t, const uint8_t* packed,
                            const uint8_t* qabs, const float* absmax2, const float* code2,
                            const float* offset, int64_t n, int64_t k, const uint16_t* bias,
                            const uint16_t* z, const uint16_t* lora_b, float scale, uint16_t* y,
                            int64_t ldy, void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "ss_qlora_fwd";
  SS_CHECK_ARG(t >= 0, "%s: t=%lld must be >= 0", fn, (long long)t);
  int rc = check_nf4(fn, packed, qabs, absmax2, code2, offset, n, k);
  if (rc) return rc;
  if (t == 0) return SS_OK;
  SS_CHECK_ARG(x && y && z && lora_b, "%s: null pointer", fn);
  SS_CHECK_ARG(ldx >= k && ldy >= n, "%s: leading dimensions too small", fn);
  SS_CHECK_ARG(reinterpret_cast<uintptr_t>(z) % 8 == 0 &&
                   reinterpret_cast<uintptr_t>(lora_b) % 8 == 0,
               "%s: Z and lora_B must be 8-byte aligned", fn);
  GemmParams p = fwd_params(x, ldx, t, packed, qabs, absmax2, code2, offset, n, k, bias, y, ldy);
  p.lz = reinterpret_cast<const half_t*>(z);
  p.lb = reinterpret_cast<const half_t*>(lora_b);
  p.ldlb = 16;
  p.lscale = scale;
  return run_fwd<EPI_LORA>(p, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int ss_nf4_gemm_dx(const uint16_t* dy, int64_t lddy, int64_t t, const uint8_t* packed,
                              const uint8_t* qabs, const float* absmax2, const float* code2,
                              const float* offset, int64_t n, int64_t k, uint16_t* dx,
                              int64_t lddx, int accumulate, void* workspace,
                              size_t workspace_bytes, void* stream) {
  const char* fn = "ss_nf4_gemm_dx";
  SS_CHECK_ARG(t >= 0, "%s: t=%lld must be >= 0", fn, (long long)t);
  int rc = check_nf4(fn, packed, qabs, absmax2, code2, offset, n, k);
  if (rc) return rc;
  if (t == 0) return SS_OK;
  SS_CHECK_ARG(dy && dx, "%s: null gradient pointer", fn);
  SS_CHECK_ARG(lddy >= n && lddx >= k, "%s: leading dimensions too small", fn);
  GemmParams p = dx_params(dy, lddy, t, packed, qabs, absmax2, code2, offset, n, k, dx, lddx,
                           accumulate);
  return run_dx<EPI_PLAIN>(p, n, k, workspace, workspace_bytes, (hipStream_t)stream);
}

// The MLP's SwiGLU riding on the GEMM that produces its last operand.  The
// dense NT and fused NF4 epilogues (and the split-K reduce) apply it as they
// store (glu_apply); a path whose kernel stores plainly (streaming / skinny
// small-T kernels, the generic loader) leaves its output where the
// activation kernel then reads and overwrites it in place.  Either way the
// result is bit-identical to the product followed by ss_swiglu_fwd/bwd.
extern "C" int ss_nf4_gemm_fwd_swiglu(const uint16_t* x, int64_t ldx, int64_t t,
                                      const uint8_t* packed, const uint8_t* qabs,
                                      const float* absmax2, const float* code2,
                                      const float* offset, int64_t n, int64_t k,
                                      const uint16_t* gate, int64_t ldgate, uint16_t* up,
                                      int64_t ldup, uint16_t* act, int64_t ldact, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  const char* fn = "ss_nf4_gemm_fwd_swiglu";
  SS_CHECK_ARG(t >= 0, "%s: t=%lld must be >= 0", fn, (long long)t);
  int rc = check_nf4(fn, packed, qabs, absmax2, code2, offset, n, k);
  if (rc) return rc;
  if (t == 0) return SS_OK;
  SS_CHECK_ARG(x && gate && act, "%s: null pointer", fn);
  SS_CHECK_ARG(ldx >= k && ldgate >= n && ldact >= n && (!up || ldup >= n),
               "%s: leading dimensions too small", fn);
  uint16_t* c = up ? up : act;
  const int64_t ldc = up ? ldup : ldact;
  GemmParams p = fwd_params(x, ldx, t, packed, qabs, absmax2, code2, offset, n, k, nullptr, c,
                            ldc);
  int done = 0;
  p.glu = 1;
  p.glu_store_c = up != nullptr;
  p.glu_gate = reinterpret_cast<const half_t*>(gate);
  p.ldgate = ldgate;
  p.glu_out = reinterpret_cast<half_t*>(act);
  p.ldglu = ldact;
  p.glu_vec = n % 8 == 0 && aligned16(c, ldc) && aligned16(gate, ldgate) &&
              aligned16(act, ldact);
  p.glu_done = &done;
  rc = run_fwd<EPI_PLAIN>(p, workspace, workspace_bytes, (hipStream_t)stream);
  if (rc || done) return rc;
  return ss_swiglu_fwd(gate, SS_F16, ldgate, 1, c, SS_F16, ldc, 1, act, SS_F16, ldact, 1, t, n,
                       stream);
}

extern "C" int ss_nf4_gemm_dx_swiglu(const uint16_t* dy, int64_t lddy, int64_t t,
                                     const uint8_t* packed, const uint8_t* qabs,
                                     const float* absmax2, const float* code2,
                                     const float* offset, int64_t n, int64_t k,
                                     const uint16_t* gate, int64_t ldgate, const uint16_t* up,
                                     int64_t ldup, uint16_t* dgate, int64_t lddgate,
                                     uint16_t* dup, int64_t lddup, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  const char* fn = "ss_nf4_gemm_dx_swiglu";
  SS_CHECK_ARG(t >= 0, "%s: t=%lld must be >= 0", fn, (long long)t);
  int rc = check_nf4(fn, packed, qabs, absmax2, code2, offset, n, k);
  if (rc) return rc;
  if (t == 0) return SS_OK;
  SS_CHECK_ARG(dy && gate && up && dgate && dup, "%s: null pointer", fn);
  SS_CHECK_ARG(lddy >= n && ldgate >= k && ldup >= k && lddgate >= k && lddup >= k,
               "%s: leading dimensions too small", fn);
  GemmParams p = dx_params(dy, lddy, t, packed, qabs, absmax2, code2, offset, n, k, dgate,
                           lddgate, 0);
  int done = 0;
  p.glu = 2;
  p.glu_gate = reinterpret_cast<const half_t*>(gate);
  p.ldgate = ldgate;
  p.glu_up = reinterpret_cast<const half_t*>(up);
  p.ldup = ldup;
  p.glu_out = reinterpret_cast<half_t*>(dup);
  p.ldglu = lddup;
  p.glu_vec = k % 8 == 0 && aligned16(dgate, lddgate) && aligned16(gate, ldgate) &&
              aligned16(up, ldup) && aligned16(dup, lddup);
  p.glu_done = &done;
  rc = run_dx<EPI_PLAIN>(p, n, k, workspace, workspace_bytes, (hipStream_t)stream);
  if (rc || done) return rc;
  return ss_swiglu_bwd(gate, SS_F16, ldgate, 1, up, SS_F16, ldup, 1, dgate, SS_F16, lddgate, 1,
                       dgate, SS_F16, lddgate, 1, dup, SS_F16, lddup, 1, t, k, stream);
}

extern "C" int ss_qlora_dx(const uint16_t* dy, int64_t lddy, int64_t t, const uint8_t* packed,
                           const uint8_t* qabs, const float* absmax2, const float* code2,
                           const float* offset, int64_t n, int64_t k, const uint16_t* dz,
                           const uint16_t* lora_a, uint16_t* dx, int64_t lddx, void* workspace,
                           size_t workspace_bytes, void* stream) {
  const char* fn = "ss_qlora_dx";
  SS_CHECK_ARG(t >= 0, "%s: t=%lld must be >= 0", fn, (long long)t);
  int rc = check_nf4(fn, packed, qabs, absmax2, code2, offset, n, k);
  if (rc) return rc;
  if (t == 0) return SS_OK;
  SS_CHECK_ARG(dy && dx && dz && lora_a, "%s: null pointer", fn);
  SS_CHECK_ARG(lddy >= n && lddx >= k, "%s: leading dimensions too small", fn);
  SS_CHECK_ARG(reinterpret_cast<uintptr_t>(dz) % 8 == 0, "%s: dZ must be 8-byte aligned", fn);
  GemmParams p = dx_params(dy, lddy, t, packed, qabs, absmax2, code2, offset, n, k, dx, lddx, 0);
  p.lz = reinterpret_cast<const half_t*>(dz);
  p.lb = reinterpret_cast<const half_t*>(lora_a);
  p.ldlb = k;
  return run_dx<EPI_RANK>(p, n, k, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" size_t ss_qlora_rank_workspace_size(int64_t t, int64_t n, int64_t k) {
  const size_t fwd = ss_lora_workspace_size(t, 0);
  // The backward's dB and dA exchange areas follow dZ's, one after the other.
  const size_t bwd = ss_lora_workspace_size(t, n) + ss::rank_grad_part_bytes(k);
  const size_t da = ss_lora_workspace_size(0, k);
  size_t m = fwd > bwd ? fwd : bwd;
  return m > da ? m : da;
}

namespace ss {

// Body of ss_qlora_forward[_dropout]: drop == nullptr for the dropout-free
// projection, else Z = fp16(fp16(drop(X)) . A^T) with the call's mask.
static int qlora_forward(const char* fn, const uint16_t* x, int64_t ldx, int64_t t,
                         const uint8_t* packed, const uint8_t* qabs, const float* absmax2,
                         const float* code2, const float* offset, int64_t n, int64_t k,
                         const uint16_t* bias, const uint16_t* lora_a, const uint16_t* lora_b,
                         float scale, uint16_t* z, uint16_t* y, int64_t ldy, void* workspace,
                         size_t workspace_bytes, void* rank_workspace,
                         size_t rank_workspace_bytes, const DropoutArgs* drop, void* stream) {
  SS_CHECK_ARG(t >= 0, "%s: t=%lld must be >= 0", fn, (long long)t);
  int rc = check_nf4(fn, packed, qabs, absmax2, code2, offset, n, k);
  if (rc) return rc;
  if (t == 0) return SS_OK;
  SS_CHECK_ARG(x && y && z && lora_a && lora_b, "%s: null pointer", fn);
  SS_CHECK_ARG(ldx >= k && ldy >= n, "%s: leading dimensions too small", fn);
  SS_CHECK_ARG(reinterpret_cast<uintptr_t>(z) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(lora_b) % 16 == 0,
               "%s: Z and lora_B must be 16-byte aligned", fn);
  GemmParams p = fwd_params(x, ldx, t, packed, qabs, absmax2, code2, offset, n, k, bias, y, ldy);
  p.lz = reinterpret_cast<const half_t*>(z);
  p.lb = reinterpret_cast<const half_t*>(lora_b);
  p.ldlb = 16;
  p.lscale = scale;
  PrepJobs pj{};
  bool vp = false, vg = false;
  // Z = fp16(X . A^T): the rank-16 job the LoRA epilogue reads.
  pj.proj_blocks = rank_project_setup(pj.proj, x, ldx, t, k, lora_a, k, 0, 1.0f, z,
                                      rank_workspace, rank_workspace_bytes, t, vp);
  if (drop) pj.proj.drop = *drop;
  pj.grad_blocks = 0;
  pj.dec_kind = kDecodeNone;
  return run_fwd<EPI_LORA>(p, workspace, workspace_bytes, (hipStream_t)stream, &pj, vp, vg);
}

// Body of ss_qlora_backward[_dropout].  With dropout the dX GEMM runs without
// the rank-16 term, and one tail launch then computes dA from the masked X
// and adds the masked fp16(dZ . A) to dX.
static int qlora_backward(const char* fn, const uint16_t* dy, int64_t lddy, int64_t t,
                          const uint8_t* packed, const uint8_t* qabs, const float* absmax2,
                          const float* code2, const float* offset, int64_t n, int64_t k,
                          const uint16_t* x, int64_t ldx, const uint16_t* z,
                          const uint16_t* lora_a, const uint16_t* lora_b, float scale,
                          uint16_t* dx, int64_t lddx, uint16_t* dz, uint16_t* da, uint16_t* db,
                          void* workspace, size_t workspace_bytes, void* rank_workspace,
                          size_t rank_workspace_bytes, const DropoutArgs* drop, void* stream) {
  SS_CHECK_ARG(t >= 0, "%s: t=%lld must be >= 0", fn, (long long)t);
  int rc = check_nf4(fn, packed, qabs, absmax2, code2, offset, n, k);
  if (rc) return rc;
  SS_CHECK_ARG(da && db && lora_a && lora_b, "%s: null pointer", fn);
  if (t == 0) {
    // No rows: the adapter gradients are zero and dX is empty.
    rc = ss_lora_grad(nullptr, 16, nullptr, n, 0, k, 0, 1.0f, 0, da, nullptr, 0, stream);
    if (rc) return rc;
    return ss_lora_grad(nullptr, 16, nullptr, n, 0, n, 0, 1.0f, 1, db, nullptr, 0, stream);
  }
  SS_CHECK_ARG(dy && dx && dz && x && z, "%s: null pointer", fn);
  SS_CHECK_ARG(lddy >= n && lddx >= k && ldx >= k, "%s: leading dimensions too small", fn);
  SS_CHECK_ARG(reinterpret_cast<uintptr_t>(dz) % 16 == 0, "%s: dZ must be 16-byte aligned", fn);
  if (drop) {
    auto al = [](const void* q, int64_t ld) {
      return reinterpret_cast<uintptr_t>(q) % 16 == 0 && ld % 8 == 0;
    };
    if (!(al(x, ldx) && al(dx, lddx) && al(lora_a, k) && k % 8 == 0)) {
      ss::set_error("%s: the dropout path needs 16-byte aligned X, dX and lora_A rows and "
                    "K %% 8 == 0", fn);
      return SS_ERR_UNSUPPORTED;
    }
  }
  hipStream_t s = (hipStream_t)stream;
  PrepJobs pj{};
  bool vp = false, vg = false;
  // dZ = fp16(fp16(g * s) . B) and dB = fp16(fp16(g * s)^T . Z): both read g
  // once, neither depends on the other; the dX epilogue reads dZ.
  pj.proj_blocks = rank_project_setup(pj.proj, dy, lddy, t, n, lora_b, 16, 1, scale, dz,
                                      rank_workspace, rank_workspace_bytes, t, vp);
  pj.grad_blocks = rank_grad_setup(pj.grad, z, 16, dy, lddy, t, n, scale, 1, db, rank_workspace,
                                   rank_workspace_bytes, t, vg);
  pj.dec_kind = kDecodeNone;
  if (drop) {
    GemmParams p = dx_params(dy, lddy, t, packed, qabs, absmax2, code2, offset, n, k, dx, lddx,
                             0);
    rc = run_dx<EPI_PLAIN>(p, n, k, workspace, workspace_bytes, s, &pj, vp, vg);
    if (rc) return rc;
    return launch_dropout_tail(reinterpret_cast<const half_t*>(dz),
                               reinterpret_cast<const half_t*>(x), ldx,
                               reinterpret_cast<const half_t*>(lora_a), t, k,
                               reinterpret_cast<half_t*>(dx), lddx, reinterpret_cast<half_t*>(da),
                               *drop, rank_workspace, rank_workspace_bytes, s);
  }
  GemmParams p = dx_params(dy, lddy, t, packed, qabs, absmax2, code2, offset, n, k, dx, lddx, 0);
  p.lz = reinterpret_cast<const half_t*>(dz);
  p.lb = reinterpret_cast<const half_t*>(lora_a);
  p.ldlb = k;
  // dA = fp16(dZ^T . X) needs dZ from the preparation launch, as the dX GEMM
  // does; dB has no consumer in this call.  dA rides on the dense dX launch
  // (or on its split-K reduce) when that path runs with vector loads, else it
  // is launched on its own afterwards.  dB joins it on an unsplit dX launch,
  // in disjoint exchange areas (dB after dZ's, dA after dB's) and counter
  // ranges, where both fill CUs the GEMM leaves idle instead of lengthening
  // the preparation launch (measured at T = 990: k / v backward 18.0 -> 14.8
  // us, q / o 32 -> 30); next to a split-K reduce it gained nothing (the
  // reduce grew by what the preparation launch lost), so there it stays in
  // the preparation launch.
  bool vda = false, vdb = false;
  int da_ran = 0;
  RankGradArgs dbg;
  const int64_t db_blocks = rank_grad_setup(dbg, z, 16, dy, lddy, t, n, scale, 1, db,
                                            rank_workspace, rank_workspace_bytes, t, vdb);
  const int64_t da_blocks = rank_grad_setup(p.tail, dz, 16, x, ldx, t, k, 1.0f, 0, da,
                                            rank_workspace, rank_workspace_bytes, t, vda,
                                            rank_grad_part_bytes(n), kCounters / 4);
  if (vda) {
    p.tail_blocks = da_blocks;
    p.tail_ran = &da_ran;
    if (vdb && nt_plan(t, k, n).splits == 1) {
      p.tail2 = dbg;
      p.tail2_blocks = db_blocks;
      pj.grad_blocks = 0;
    }
  }
  rc = run_dx<EPI_RANK>(p, n, k, workspace, workspace_bytes, s, &pj, vp, vg);
  if (rc || da_ran) return rc;
  if (p.tail2_blocks) {
    rc = ss_lora_grad(z, 16, dy, lddy, t, n, 1, scale, 1, db, rank_workspace,
                      rank_workspace_bytes, stream);
    if (rc) return rc;
  }
  return ss_lora_grad(dz, 16, x, ldx, t, k, 0, 1.0f, 0, da, rank_workspace, rank_workspace_bytes,
                      stream);
}

static int check_dropout(const char* fn, float p) {
  SS_CHECK_ARG(p > 0.0f && p < 1.0f, "%s: dropout p=%g must be in (0, 1)", fn, (double)p);
  return SS_OK;
}

}  // namespace ss

extern "C" int ss_qlora_forward(const uint16_t* x, int64_t ldx, int64_t t, const uint8_t* packed,
                                const uint8_t* qabs, const float* absmax2, const float* code2,
                                const float* offset, int64_t n, int64_t k, const uint16_t* bias,
                                const uint16_t* lora_a, const uint16_t* lora_b, float scale,
                                uint16_t* z, uint16_t* y, int64_t ldy, void* workspace,
                                size_t workspace_bytes, void* rank_workspace,
                                size_t rank_workspace_bytes, void* stream) {
  return qlora_forward("ss_qlora_forward", x, ldx, t, packed, qabs, absmax2, code2, offset, n, k,
                       bias, lora_a, lora_b, scale, z, y, ldy, workspace, workspace_bytes,
                       rank_workspace, rank_workspace_bytes, nullptr, stream);
}

extern "C" int ss_qlora_forward_dropout(const uint16_t* x, int64_t ldx, int64_t t,
                                        const uint8_t* packed, const uint8_t* qabs,
                                        const float* absmax2, const float* code2,
                                        const float* offset, int64_t n, int64_t k,
                                        const uint16_t* bias, const uint16_t* lora_a,
                                        const uint16_t* lora_b, float scale, uint64_t seed,
                                        float p, uint16_t* z, uint16_t* y, int64_t ldy,
                                        void* workspace, size_t workspace_bytes,
                                        void* rank_workspace, size_t rank_workspace_bytes,
                                        void* stream) {
  const char* fn = "ss_qlora_forward_dropout";
  const int rc = check_dropout(fn, p);
  if (rc) return rc;
  SS_CHECK_ARG(k % 8 == 0, "%s: K=%lld must be a multiple of 8", fn, (long long)k);
  const DropoutArgs drop = dropout_args(seed, p);
  return qlora_forward(fn, x, ldx, t, packed, qabs, absmax2, code2, offset, n, k, bias, lora_a,
                       lora_b, scale, z, y, ldy, workspace, workspace_bytes, rank_workspace,
                       rank_workspace_bytes, &drop, stream);
}

extern "C" int ss_qlora_backward(const uint16_t* dy, int64_t lddy, int64_t t,
                                 const uint8_t* packed, const uint8_t* qabs,
                                 const float* absmax2, const float* code2, const float* offset,
                                 int64_t n, int64_t k, const uint16_t* x, int64_t ldx,
                                 const uint16_t* z, const uint16_t* lora_a,
                                 const uint16_t* lora_b, float scale, uint16_t* dx, int64_t lddx,
                                 uint16_t* dz, uint16_t* da, uint16_t* db, void* workspace,
                                 size_t workspace_bytes, void* rank_workspace,
                                 size_t rank_workspace_bytes, void* stream) {
  return qlora_backward("ss_qlora_backward", dy, lddy, t, packed, qabs, absmax2, code2, offset, n,
                        k, x, ldx, z, lora_a, lora_b, scale, dx, lddx, dz, da, db, workspace,
                        workspace_bytes, rank_workspace, rank_workspace_bytes, nullptr, stream);
}

extern "C" int ss_qlora_backward_dropout(const uint16_t* dy, int64_t lddy, int64_t t,
                                         const uint8_t* packed, const uint8_t* qabs,
                                         const float* absmax2, const float* code2,
                                         const float* offset, int64_t n, int64_t k,
                                         const uint16_t* x, int64_t ldx, const uint16_t* z,
                                         const uint16_t* lora_a, const uint16_t* lora_b,
                                         float scale, uint64_t seed, float p, uint16_t* dx,
                                         int64_t lddx, uint16_t* dz, uint16_t* da, uint16_t* db,
                                         void* workspace, size_t workspace_bytes,
                                         void* rank_workspace, size_t rank_workspace_bytes,
                                         void* stream) {
  const char* fn = "ss_qlora_backward_dropout";
  const int rc = check_dropout(fn, p);
  if (rc) return rc;
  const DropoutArgs drop = dropout_args(seed, p);
  return qlora_backward(fn, dy, lddy, t, packed, qabs, absmax2, code2, offset, n, k, x, ldx, z,
                        lora_a, lora_b, scale, dx, lddx, dz, da, db, workspace, workspace_bytes,
                        rank_workspace, rank_workspace_bytes, &drop, stream);
}

static int gemm_f16_impl(const char* fn, int a_trans, int b_trans, int64_t m, int64_t n, int64_t k,
                         float alpha, const float* alpha_dev, const uint16_t* a, int64_t lda,
                         const uint16_t* b,
                         int64_t ldb, const uint16_t* bias, float beta, void* c, int c_dtype,
                         int64_t ldc, void* workspace, size_t workspace_bytes, void* stream) {
  SS_CHECK_ARG(m >= 0 && n >= 0 && k >= 0, "%s: negative size", fn);
  SS_CHECK_ARG(c_dtype == SS_F16 || c_dtype == SS_F32, "%s: c_dtype must be SS_F16/SS_F32", fn);
  SS_CHECK_ARG(beta == 0.0f || beta == 1.0f, "%s: beta must be 0 or 1", fn);
  if (m == 0 || n == 0) return SS_OK;
  SS_CHECK_ARG(c && (k == 0 || (a && b)), "%s: null pointer", fn);
  SS_CHECK_ARG(lda >= (a_trans ? m : k) && ldb >= (b_trans ? k : n) && ldc >= n,
               "%s: leading dimensions too small", fn);
  GemmParams p{};
  p.M = m; p.N = n; p.K = k;
  // Vector loads need 16-byte aligned rows and no 8-element chunk crossing the
  // end of the contiguous dimension (K for row-major operands, M/N otherwise).
  p.A = reinterpret_cast<const half_t*>(a); p.lda = lda;
  p.a_vec = aligned16(a, lda) && (a_trans ? m % 8 == 0 : k % 8 == 0);
  p.B = reinterpret_cast<const half_t*>(b); p.ldb = ldb;
  p.b_vec = aligned16(b, ldb) && (b_trans ? k % 8 == 0 : n % 8 == 0);
  p.bias = reinterpret_cast<const half_t*>(bias);
  p.C = c; p.ldc = ldc; p.alpha = alpha; p.alpha_dev = alpha_dev; p.beta = beta != 0.0f;
  hipStream_t s = (hipStream_t)stream;
  // b_trans = 1: B stored [N,K] -> OP_ROW; b_trans = 0: B stored [K,N] -> OP_COL.
  const int code = (a_trans ? 2 : 0) + (b_trans ? 0 : 1) + (c_dtype == SS_F32 ? 4 : 0);
  void* const w = workspace;
  const size_t wb = workspace_bytes;
  switch (code) {
    case 0: return dispatch<OP_ROW, OP_ROW, SS_F16>(p, s, "gemm_kernel<f16 nt>", w, wb);
    case 1: return dispatch<OP_ROW, OP_COL, SS_F16>(p, s, "gemm_kernel<f16 nn>", w, wb);
    case 2: return dispatch<OP_COL, OP_ROW, SS_F16>(p, s, "gemm_kernel<f16 tt>", w, wb);
    case 3: return dispatch<OP_COL, OP_COL, SS_F16>(p, s, "gemm_kernel<f16 tn>", w, wb);
    case 4: return dispatch<OP_ROW, OP_ROW, SS_F32>(p, s, "gemm_kernel<f32 nt>", w, wb);
    case 5: return dispatch<OP_ROW, OP_COL, SS_F32>(p, s, "gemm_kernel<f32 nn>", w, wb);
    case 6: return dispatch<OP_COL, OP_ROW, SS_F32>(p, s, "gemm_kernel<f32 tt>", w, wb);
    default: return dispatch<OP_COL, OP_COL, SS_F32>(p, s, "gemm_kernel<f32 tn>", w, wb);
  }
}

extern "C" int ss_gemm_f16(int a_trans, int b_trans, int64_t m, int64_t n, int64_t k, float alpha,
                           const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                           const uint16_t* bias, float beta, void* c, int c_dtype, int64_t ldc,
                           void* stream) {
  return gemm_f16_impl("ss_gemm_f16", a_trans, b_trans, m, n, k, alpha, nullptr, a, lda, b, ldb,
                       bias, beta, c, c_dtype, ldc, nullptr, 0, stream);
}

extern "C" size_t ss_gemm_f16_workspace_size(int a_trans, int b_trans, int64_t m, int64_t n,
                                             int64_t k) {
  // Split-K partials of the dense NT kernel (every operand layout).
  (void)a_trans;
  (void)b_trans;
  return ss::nt_partial_bytes(m, n, k);
}

extern "C" int ss_gemm_f16_split(int a_trans, int b_trans, int64_t m, int64_t n, int64_t k,
                                 float alpha, const float* alpha_dev, const uint16_t* a,
                                 int64_t lda, const uint16_t* b, int64_t ldb,
                                 const uint16_t* bias, float beta, void* c, int c_dtype,
                                 int64_t ldc, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  return gemm_f16_impl("ss_gemm_f16_split", a_trans, b_trans, m, n, k, alpha, alpha_dev, a, lda,
                       b, ldb, bias, beta, c, c_dtype, ldc, workspace, workspace_bytes, stream);
}
