// Declarations shared by the GEMM kernels (gemm.hip: general operand
// sources; gemm_nt.hip: the dense K-contiguous x K-contiguous main loop).
#pragma once

#include "common.h"
#include "swiglu.h"
#include "philox.h"

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
// EPI_PARTIAL (split-K): the raw fp32 accumulator of a workgroup's split
// (split_tile) is stored to part[split][M][N]; a reduce kernel sums the
// splits in order and applies the requested epilogue.
// EPI_GLU (dense NT, fused NF4, split-K reduce): the plain value passed
// through glu_apply; entry points request it with EPI_PLAIN and p.glu set, the
// launchers pick the EPI_GLU instantiation (the plain kernels carry no
// activation code, which would cost the 256x256 tiles registers).
enum Epilogue { EPI_PLAIN = 0, EPI_LORA = 1, EPI_RANK = 2, EPI_PARTIAL = 3, EPI_GLU = 4 };

// Arguments of one rank-16 product; splits / cps from the host plan,
// part / counters inside a zero-filled rank workspace (rank16.h, lora_gemm.hip).
struct RankProjectArgs {
  const half_t* a;
  int64_t lda, m, k;
  const half_t* w;
  int64_t ldw;
  int w_kr;
  float a_scale;
  int64_t cps, splits;
  half_t* out;
  float* part;
  int* counters;
  DropoutArgs drop;  // A' = dropout(A) (rows x k, row-major element index) when drop.on
};

struct RankGradArgs {
  const half_t* p;
  int64_t ldp;
  const half_t* q;
  int64_t ldq, t, n;
  float q_scale;
  int64_t cps, splits;
  int transpose;
  half_t* out;
  float* part;
  int* counters;
  DropoutArgs drop;  // Q' = dropout(Q) (t x n, row-major element index) when drop.on
};

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
  // Device fp32 scalar multiplying alpha when not null (read once per
  // workgroup; the plain dense GEMMs and their split-K reduce), so a caller
  // whose scale is computed on the device needs no host round trip.
  const float* alpha_dev;
  int beta;
  const half_t* lz;   // Z or dZ, [M, 16] contiguous
  const half_t* lb;   // lora_B [N, 16] (EPI_LORA) or lora_A [16, ldlb] (EPI_RANK)
  int64_t ldlb;
  float lscale;
  int remap;   // XCD-aware tile numbering (default on)
  float* part;      // split-K partials [splits][M][N] fp32 (EPI_PARTIAL)
  int64_t k_split;  // k elements per split (a multiple of 64)
  int fold_rank;    // EPI_PARTIAL: split 0 adds the rank-16 term lz . lb (EPI_RANK layout)
  // EPI_PARTIAL of an EPI_LORA product: split 0 also stores the rounded LoRA
  // term fp16(fp16(lz . lb^T) * lscale) here ([M][N]), which the reduce adds
  // instead of recomputing it from lora_B rows.
  half_t* lora_plane;
  int pingpong;     // 8-wave NT configurations: ping-pong main loop (set by gemm_nt)
  // Dense NT kernels: A (B) stored K-major, element (m, k) at A[k * lda + m]
  // ((n, k) at B[k * ldb + n]), as a transposed view stores it; plain and
  // split-K epilogues only.
  int a_t, b_t;
  // Optional rank-16 grads riding on the dense NT launch (unsplit) or on its
  // split-K reduce: tail_blocks + tail2_blocks extra workgroups each run one
  // block of `tail`, then of `tail2` (rank_grad_block, vector loads).  The
  // two write disjoint counter and exchange areas.  tail_ran (host side) is
  // set when a launch took the tails.
  RankGradArgs tail;
  int64_t tail_blocks;
  RankGradArgs tail2;
  int64_t tail2_blocks;
  int* tail_ran;
  // Gated (SwiGLU) store of an fp16, beta = 0 output (glu_apply): glu = 1
  // forward, the product is `up` -- act = silu(gate) up goes to glu_out and
  // up to C when glu_store_c; glu = 2 backward, the product is dact -- dgate
  // to C, dup to glu_out.  Applied by the EPI_GLU instantiations of the dense
  // NT and fused NF4 kernels and of the split-K reduce, whose host launchers
  // set *glu_done; other kernels store C unchanged and leave the activation
  // to the caller.
  int glu;
  int glu_store_c;
  int glu_vec;  // N, ldc / ldgate / ldup / ldglu and the pointers 16-byte granular
  // fp16 output through the LDS-staged epilogue (16-byte stores): set by the
  // NT / fused NF4 launchers when beta = 0 and N, ldc and C are 16-byte granular.
  int c_vec;
  const half_t* glu_gate;
  int64_t ldgate;
  const half_t* glu_up;
  int64_t ldup;
  half_t* glu_out;
  int64_t ldglu;
  int* glu_done;
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

// (tile, split) of a split-K workgroup of a (tiles, splits) grid.  The pairs
// are numbered split-major and, with remap, every XCD owns a contiguous range
// of them: the workgroups that share an L2 then read one K slice of A and B
// instead of every XCD reading the same rows of every slice (a row-major
// remap of blockIdx.x alone gives each XCD all M tiles of its N columns in
// every split, so A is fetched once per XCD).
__device__ __forceinline__ void split_tile(bool remap, int64_t tiles, int64_t& tile,
                                           int64_t& split) {
  const int64_t w = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
  const int64_t l = remap ? xcd_remap(w, tiles * gridDim.y) : w;
  split = l / tiles;
  tile = l - split * tiles;
}

// LDS DMA (gfx950 global_load_lds_*).  One wave-wide dwordx4 DMA: lane i's
// 16 bytes at base + voff land at LDS byte address lds + 16 i; the dword form
// puts lane i's 4 bytes at lds + 4 i.  `base` and `lds` are wave-uniform
// (SGPRs); voff is the lane's 32-bit byte offset.  s_nop covers the M0-write
// -> LDS-DMA hazard.  Completion is counted by vmcnt, in issue order with the
// wave's other vector-memory loads.
__device__ __forceinline__ void dma16(uint32_t voff, const void* base, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(base), "s"(lds)
               : "memory", "m0");
}
__device__ __forceinline__ void dma4(uint32_t voff, const void* base, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :
               : "v"(voff), "s"(base), "s"(lds)
               : "memory", "m0");
}

// s_waitcnt vmcnt(N) (expcnt and lgkmcnt unconstrained).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// Vector loads the compiler does not track: it inserts no wait for them.
// The caller waits explicitly (wait_vm) and then passes the value through
// tie() before its first use, so that no use is scheduled ahead of the wait.
__device__ __forceinline__ u32x4 vload16(const void* p) {
  u32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(p) : "memory");
  return v;
}
__device__ __forceinline__ uint32_t vload4(const void* p) {
  uint32_t v;
  asm volatile("global_load_dword %0, %1, off" : "=v"(v) : "v"(p) : "memory");
  return v;
}
__device__ __forceinline__ uint32_t vload_u16(const void* p) {
  uint32_t v;
  asm volatile("global_load_ushort %0, %1, off" : "=v"(v) : "v"(p) : "memory");
  return v;
}
template <class T>
__device__ __forceinline__ void tie(T& v) {
  asm volatile("" : "+v"(v));
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
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

// Gated store of output element (row, col) with value v = alpha acc + bias
// and the element's gate g (and, backward, up u) already loaded: v is
// rounded to fp16 first (the product as the unfused path stores it), then the
// activation of swiglu.hip is applied to that fp16 value.  Callers load the
// gate / up values of a whole fragment before its first store: a load placed
// after a store through another pointer of the struct cannot be moved above
// it, and one memory round trip per element serialises the epilogue.
__device__ __forceinline__ void glu_apply(const GemmParams& p, int64_t row, int64_t col,
                                          int64_t idx, float v, half_t g, half_t u) {
  const half_t h = f32_to_f16(v);
  const SwigluTerms t = swiglu_terms((float)g);
  if (p.glu == 1) {
    if (p.glu_store_c) reinterpret_cast<half_t*>(p.C)[idx] = h;
    p.glu_out[row * p.ldglu + col] = f32_to_f16(t.act * (float)h);
  } else {
    reinterpret_cast<half_t*>(p.C)[idx] = f32_to_f16(((float)h * (float)u) * swiglu_slope(t));
    p.glu_out[row * p.ldglu + col] = f32_to_f16((float)h * t.act);
  }
}

// One fp16 output element of the epilogues, with the rounding order of the
// GEMM kernels: plain alpha * v + bias (+ C if beta); LoRA fp16(fp16(v +
// bias) + fp16(fp16(Z[row] . B[col]) * s)); rank fp16(v + dZ[row] . A[:, col])
// (+ C if beta).  v is the fp32 accumulator of (row, col).
template <int EPI>
__device__ __forceinline__ void epilogue_f16(const GemmParams& p, int64_t row, int64_t col,
                                             float v) {
  const int64_t idx = row * p.ldc + col;
  if constexpr (EPI == EPI_LORA) {
    float l = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) l += (float)p.lz[row * 16 + r] * (float)p.lb[col * 16 + r];
    const float b = p.bias ? (float)p.bias[col] : 0.0f;
    const float y = (float)f32_to_f16(v * p.alpha + b);
    const float scaled = (float)f32_to_f16((float)f32_to_f16(l) * p.lscale);
    reinterpret_cast<half_t*>(p.C)[idx] = f32_to_f16(y + scaled);
  } else if constexpr (EPI == EPI_RANK) {
    float l = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) l += (float)p.lz[row * 16 + r] * (float)p.lb[r * p.ldlb + col];
    store_c<SS_F16>(p.C, idx, v + l, p.beta);
  } else {
    const float b = p.bias ? (float)p.bias[col] : 0.0f;
    store_c<SS_F16>(p.C, idx, v * p.alpha + b, p.beta);
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
// LDS-staged fp16 epilogue switch of the NT and fused NF4 launchers (default on).
bool staged_epilogue_enabled();
// Split-K scratch that gemm_nt uses for an M x N x K product (0: no split):
// the fp32 partial planes and an fp16 plane for a LoRA forward's rank term.
size_t nt_partial_bytes(int64_t m, int64_t n, int64_t k);
// Tile configuration (1..10 in gemm_nt.hip's list) and split-K plan of an
// M x N x K product on the NT kernels.
struct NtPlan {
  int cfg;
  int64_t splits, k_split;
};
NtPlan nt_plan(int64_t m, int64_t n, int64_t k);

// Fused NF4 forward (gemm_nf4.hip): Y = X . Wdec^T with p.M = T, p.N = N,
// p.K = K, p.A = X, p.w = the NF4 weight, the NT kernel's tile plan and
// epilogues (EPI_PLAIN / EPI_LORA); the weight is decoded into LDS tiles, never
// written to memory.  `partials` (may be null) holds the split-K planes
// (nt_partial_bytes).  SS_ERR_UNSUPPORTED (nothing launched) unless
// gemm_nf4_fwd_ok.
bool gemm_nf4_fwd_ok(const GemmParams& p, int epi);
// Whether the fused kernel is the faster path for this product (tile plan and
// M tiles; measured).
bool gemm_nf4_fwd_preferred(const GemmParams& p);
// The fused kernel's tile / split plan and its split-K scratch (0: no split).
NtPlan nf4_plan(int64_t m, int64_t n, int64_t k);
size_t nf4_fused_partial_bytes(int64_t m, int64_t n, int64_t k);
// Fused NF4 dX for T <= 256 (gemm_nf4.hip): the weight tiles decoded into LDS
// (K-major B tiles) inside the GEMM; plain (beta) and rank-16 epilogues.  Split-K partials in
// `partials` (nf4_dx_fused_partial_bytes); SS_ERR_UNSUPPORTED when
// gemm_nf4_dx_ok fails.
bool gemm_nf4_dx_ok(const GemmParams& p, int epi);
bool gemm_nf4_dx_preferred(const GemmParams& p);
size_t nf4_dx_fused_partial_bytes(int64_t m, int64_t n, int64_t k);
int gemm_nf4_dx(const GemmParams& p, int epi, hipStream_t stream, void* partials,
                size_t partial_bytes);
int gemm_nf4_fwd(const GemmParams& p, int epi, hipStream_t stream, void* partials,
                 size_t partial_bytes);

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

// Streaming NF4 forward (nf4_stream.hip) for T <= kStreamMaxT rows and K % 256
// == 0: the codes stream through per-wave LDS rings and are decoded with a
// bank-replicated code table, the block scales applied to the MFMA results;
// fp32 partial planes, reduced by splitk_reduce.  Same contract as
// nf4_skinny_fwd.
constexpr int64_t kStreamMaxT = 32;
size_t stream_partial_bytes(int64_t t, int64_t n, int64_t k);
int nf4_stream_fwd(const GemmParams& p, int epi, void* partials, size_t partial_bytes,
                   hipStream_t stream);

// Streaming NF4 backward (nf4_stream_dx.hip) for T <= kStreamDxMaxT rows, N %
// 16 == 0 and K % 256 == 0: dX = dY . Wdec with the codes read transposed from
// LDS and the block scales folded into dY; fp32 partial planes per row range,
// reduced (with the epilogue) by splitk_reduce.  p: M = T, N = K (dX columns),
// K = N (weight rows), A = dY.  SS_ERR_UNSUPPORTED when not applicable.
constexpr int64_t kStreamDxMaxT = 16;
size_t stream_dx_partial_bytes(int64_t t, int64_t n, int64_t k);
int nf4_stream_dx(const GemmParams& p, int epi, void* partials, size_t partial_bytes,
                  hipStream_t stream);

}  // namespace ss
