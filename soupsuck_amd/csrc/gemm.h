// Declarations shared by the GEMM kernels (gemm.hip: general operand
// sources; gemm_nt.hip: the dense K-contiguous x K-contiguous main loop).
#pragma once

#include "common.h"

namespace ss {

enum Operand { OP_ROW = 0, OP_COL = 1, OP_NF4_ROW = 2, OP_NF4_COL = 3 };

struct Nf4View {
  const uint8_t* packed;
  const uint8_t* qabs;
  const float* absmax2;
  const float* code2;
  const float* offset;
  int64_t cols;  // weight row length (elements); a multiple of 64
};

// Epilogue variants: plain (alpha * acc + bias, + beta * C); the LoRA
// forward out = fp16(fp16(acc + bias) + fp16(fp16(Z . B^T) * s)) with Z
// [M,16] and B = lora_B [N,16]; and a rank-16 update out = fp16(acc + dZ . A)
// with dZ [M,16] and A = lora_A [16, N] (row stride ldlb).
// EPI_PARTIAL (split-K, dense NT kernel only): the raw fp32 accumulator of
// split blockIdx.y is stored to part[split][M][N]; a reduce kernel sums the
// splits in order and applies the requested epilogue.
enum Epilogue { EPI_PLAIN = 0, EPI_LORA = 1, EPI_RANK = 2, EPI_PARTIAL = 3 };

struct GemmParams {
  int64_t M, N, K;
  const half_t* A;
  int64_t lda;
  int a_vec;  // 16-byte vector loads are aligned for A
  const half_t* B;
  int64_t ldb;
  int b_vec;
  Nf4View w;
  const half_t* bias;
  void* C;
  int64_t ldc;
  float alpha;
  int beta;
  const half_t* lz;   // Z or dZ, [M, 16] contiguous
  const half_t* lb;   // lora_B [N, 16] (EPI_LORA) or lora_A [16, ldlb] (EPI_RANK)
  int64_t ldlb;
  float lscale;
  int remap;   // XCD-aware tile numbering (default on)
  float* part;      // split-K partials [splits][M][N] fp32 (EPI_PARTIAL)
  int64_t k_split;  // k elements per split (a multiple of 64)
};

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own
// L2).  xcd_remap renumbers a 1-D grid so that every XCD owns a contiguous
// range of tile ids.
__device__ __forceinline__ int64_t xcd_remap(int64_t p, int64_t n) {
  constexpr int64_t kXcd = 8;
  const int64_t q = n / kXcd, r = n % kXcd;
  const int64_t x = p % kXcd, local = p / kXcd;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + local;
}

template <int CT>
__device__ __forceinline__ void store_c(void* C, int64_t idx, float v, int beta) {
  if constexpr (CT == SS_F16) {
    half_t* c = reinterpret_cast<half_t*>(C);
    if (beta) v += (float)c[idx];
    c[idx] = f32_to_f16(v);
  } else {
    float* c = reinterpret_cast<float*>(C);
    if (beta) v += c[idx];
    c[idx] = v;
  }
}

// Dense NT GEMM (A [M,K] and B [N,K] both K-contiguous fp16) on the
// direct-to-LDS pipelined kernel.  Returns SS_ERR_UNSUPPORTED (nothing
// launched) when the operands do not meet its requirements: 16-byte aligned
// rows and K % 64 == 0.  `partials` (may be null) is scratch for split-K:
// long-K products with few output tiles are split over k when it holds
// nt_partial_bytes(M, N, K) bytes.
int gemm_nt(const GemmParams& p, int ct, int epi, hipStream_t stream, void* partials = nullptr,
            size_t partial_bytes = 0);
// fp32 split-K scratch that gemm_nt uses for an M x N x K product (0: no split).
size_t nt_partial_bytes(int64_t m, int64_t n, int64_t k);

// Split-K reduction: C = epilogue(sum over `splits` planes of p.part
// [splits][M][N]) with the epilogue `epi` (EPI_PLAIN / EPI_LORA / EPI_RANK)
// and output dtype `ct` (LoRA / rank epilogues: fp16 only).
int splitk_reduce(const GemmParams& p, int splits, int ct, int epi, hipStream_t stream);

// Skinny NF4 forward (nf4_skinny.hip) for T <= kSkinnyMaxT rows and K % 128
// == 0: the weight streams from HBM once, decoded in registers; K is split
// and the fp32 partials are reduced by splitk_reduce.
constexpr int64_t kSkinnyMaxT = 128;
struct SkinnyPlan {
  int mt;                  // 16-row M tiles per workgroup (0: not applicable)
  int64_t splits, k_split;
};
SkinnyPlan skinny_plan(int64_t t, int64_t n, int64_t k);
size_t skinny_partial_bytes(int64_t t, int64_t n, int64_t k);
// Y = X . Wdec^T with p.M = T, p.N = N, p.K = K, p.A = X, p.w = the NF4
// weight and the epilogue fields of p; SS_ERR_UNSUPPORTED when not applicable.
int nf4_skinny_fwd(const GemmParams& p, int epi, void* partials, size_t partial_bytes,
                   hipStream_t stream);

}  // namespace ss
