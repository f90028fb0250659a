// Rank-16 products of the LoRA branch on MFMA (A10/A12), and the fused
// preparation launch of the QLoRA projection.
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
// (1 KiB or 4 KiB per workgroup).  The block bodies are in rank16.h.
//
// Preparation launch (qlora_prep_kernel): the jobs of a projection step that
// do not depend on each other -- the rank-16 products that must precede its
// GEMM (forward Z; backward dZ and dB) and the NF4 decode of the
// decode-first path -- run as one launch, each workgroup taking one job
// block (all jobs use 256-thread blocks).  At T ~ 1000 every launch costs a
// few microseconds of latency whatever its size, so this removes two or
// three of the step's launches per projection.

#include "decode_blocks.h"
#include "rank16.h"

namespace ss {

template <bool VEC>
__global__ __launch_bounds__(kRankMaxWaves * 64) void rank_project_kernel(RankProjectArgs g) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[kRankProjSmem];
  rank_project_block<VEC>(g, blockIdx.x, blockIdx.y, smem);
}

template <bool VEC>
__global__ __launch_bounds__(kRankMaxWaves * 64) void rank_grad_kernel(RankGradArgs g) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[kRankGradSmem];
  rank_grad_block<VEC>(g, blockIdx.x, blockIdx.y, smem);
}

constexpr int cmax(int a, int b) { return a > b ? a : b; }
constexpr int kPrepSmem = cmax(cmax(kRankGradSmem, kRankProjSmem), cmax(cmax(kDecodeSmem, kDecodeT2Smem), kDecodeRowsSmem));

// The wide transposed decode tile (64 n x 128 k) applies to cols % 128 == 0
// and 16-byte aligned codes.
static bool wide_t(const Nf4View& w, int64_t cols) {
  return cols % 128 == 0 && reinterpret_cast<uintptr_t>(w.packed) % 16 == 0;
}

// Blocks [0, proj_blocks): project (mblocks x splits, block-major); then
// grad blocks; then decode blocks (row-major decode: grid-stride over
// dec_blocks, sixteen code dwords in flight per lane; transposed decode: one
// 64 x 128 tile each, 64 x 64 when the columns are not a multiple of 128).
// With vector grad loads (VG) at most 168 VGPRs, so that three workgroups
// share a CU (the LDS allows three).  The decode blocks inherit the rank blocks' footprint: with one
// code dword in flight per lane they ran at half the stand-alone decoder's
// rate (gate 8960 x 1536: prep 19.8 us against 10.9 us for the decode
// alone); with eight, the launch costs about what its longer job costs;
// sixteen make up for the three workgroups per CU the rank blocks allow
// (gate forward prep 12.4 -> 11.5 us, down forward 17.0 -> 15.2 us).
template <bool VP, bool VG, bool DROP>
__global__ __launch_bounds__(256, VG && !DROP ? 3 : 2) void qlora_prep_kernel(PrepJobs pj) {
  __shared__ __attribute__((aligned(16))) unsigned char smem[kPrepSmem];
  int64_t b = blockIdx.x;
  if (b < pj.proj_blocks) {
    const int64_t mblocks = cdiv(pj.proj.m, 16);
    rank_project_block<VP, DROP>(pj.proj, b % mblocks, b / mblocks, smem);
    return;
  }
  b -= pj.proj_blocks;
  if (b < pj.grad_blocks) {
    const int64_t nblocks = cdiv(pj.grad.n, 64);
    rank_grad_block<VG>(pj.grad, b % nblocks, b / nblocks, smem);
    return;
  }
  b -= pj.grad_blocks;
  const Nf4View& w = pj.dec_w;
  if (pj.dec_kind == kDecodeRows) {
    decode_rows_block<true, 16>(reinterpret_cast<const uint32_t*>(w.packed), w.qabs, nullptr,
                               w.absmax2, w.code2, w.offset,
                               reinterpret_cast<half8*>(pj.dec_out),
                               pj.dec_rows * pj.dec_cols / 8, b, pj.dec_blocks, smem);
  } else if (pj.dec_cols % 128 == 0 && reinterpret_cast<uintptr_t>(w.packed) % 16 == 0) {
    decode_t2_block(w.packed, w.qabs, w.absmax2, w.code2, w.offset, pj.dec_out, pj.dec_rows,
                    pj.dec_cols, b, smem);
  } else {
    decode_t_block(w.packed, w.qabs, w.absmax2, w.code2, w.offset, pj.dec_out, pj.dec_rows,
                   pj.dec_cols, b, smem);
  }
}

static bool al16(const void* p, int64_t ld) {
  return reinterpret_cast<uintptr_t>(p) % 16 == 0 && ld % 8 == 0;
}

int64_t rank_project_setup(RankProjectArgs& g, const void* a, int64_t lda, int64_t m, int64_t k,
                           const void* w, int64_t ldw, int w_kr, float a_scale, void* out,
                           void* ws, size_t ws_bytes, int64_t rows, bool& vec) {
  (void)rows;
  const int64_t mblocks = cdiv(m, 16);
  const bool can_split = ws && ws_bytes >= kCounterBytes + rank_project_part_bytes(m) &&
                         mblocks <= kCounters / 2;
  const RankPlan plan = rank_plan(k, kProjChunk, can_split);
  g.a = reinterpret_cast<const half_t*>(a);
  g.lda = lda; g.m = m; g.k = k;
  g.w = reinterpret_cast<const half_t*>(w);
  g.ldw = ldw; g.w_kr = w_kr; g.a_scale = a_scale;
  g.cps = plan.cps; g.splits = plan.splits;
  g.out = reinterpret_cast<half_t*>(out);
  g.counters = reinterpret_cast<int*>(ws);
  g.part = reinterpret_cast<float*>(static_cast<char*>(ws) + kCounterBytes);
  g.drop = DropoutArgs{0, 0, 1.0f, 0};
  // Vector loads need 16-byte aligned rows of both operands and K % 8 == 0.
  vec = al16(a, lda) && al16(w, ldw) && k % 8 == 0;
  return mblocks * plan.splits;
}

int64_t rank_grad_setup(RankGradArgs& g, const void* p, int64_t ldp, const void* q, int64_t ldq,
                        int64_t t, int64_t n, float q_scale, int transpose, void* out, void* ws,
                        size_t ws_bytes, int64_t rows, bool& vec, size_t part_offset,
                        int64_t counter_offset) {
  const int64_t nblocks = cdiv(n, 64);
  const size_t proj_part = (rows > 0 ? rank_project_part_bytes(rows) : 0) + part_offset;
  const bool can_split = ws && ws_bytes >= kCounterBytes + proj_part + rank_grad_part_bytes(n) &&
                         counter_offset + nblocks <= kCounters / 2;
  const RankPlan plan = rank_plan(t, kGradChunk, can_split);
  g.p = reinterpret_cast<const half_t*>(p);
  g.ldp = ldp;
  g.q = reinterpret_cast<const half_t*>(q);
  g.ldq = ldq; g.t = t; g.n = n; g.q_scale = q_scale;
  g.cps = plan.cps; g.splits = plan.splits;
  g.transpose = transpose;
  g.out = reinterpret_cast<half_t*>(out);
  g.counters = reinterpret_cast<int*>(ws) + kCounters / 2 + counter_offset;
  g.drop = DropoutArgs{0, 0, 1.0f, 0};
  g.part = reinterpret_cast<float*>(static_cast<char*>(ws) + kCounterBytes + proj_part);
  // Vector loads need 16-byte aligned rows of P and Q and N % 8 == 0.
  vec = al16(q, ldq) && al16(p, ldp) && n % 8 == 0;
  return nblocks * plan.splits;
}

int launch_prep(PrepJobs& pj, bool vp, bool vg, hipStream_t stream) {
  int64_t dec = 0;
  if (pj.dec_kind == kDecodeRows) {
    const int64_t groups = pj.dec_rows * pj.dec_cols / 8;
    const int64_t cap = 4096;
    pj.dec_blocks = cdiv(groups, 16 * 256) < cap ? cdiv(groups, 16 * 256) : cap;
    dec = pj.dec_blocks;
  } else if (pj.dec_kind == kDecodeTransposed) {
    pj.dec_blocks = cdiv(pj.dec_rows, 64) *
                    (wide_t(pj.dec_w, pj.dec_cols) ? pj.dec_cols / 128 : pj.dec_cols / 64);
    dec = pj.dec_blocks;
  }
  const int64_t blocks = pj.proj_blocks + pj.grad_blocks + dec;
  if (blocks == 0) return SS_OK;
  // Without grad blocks the grad variant is irrelevant; the vector one has
  // the smaller register footprint.
  if (pj.grad_blocks == 0) vg = true;
  // The forward's Z of the dropout path masks X (the only job that does).
  if (pj.proj.drop.on) {
    auto kern = vp ? qlora_prep_kernel<true, true, true> : qlora_prep_kernel<false, true, true>;
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, stream, pj);
    SS_CHECK_LAUNCH("qlora_prep_kernel");
    return SS_OK;
  }
  auto kern = vp ? (vg ? qlora_prep_kernel<true, true, false> : qlora_prep_kernel<true, false, false>)
                 : (vg ? qlora_prep_kernel<false, true, false>
                       : qlora_prep_kernel<false, false, false>);
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, stream, pj);
  SS_CHECK_LAUNCH("qlora_prep_kernel");
  return SS_OK;
}

}  // namespace ss

using namespace ss;

extern "C" size_t ss_lora_workspace_size(int64_t rows, int64_t cols) {
  // Counters, then the exchange areas of a project with a [rows x 16] result
  // and a grad with a [16 x cols] result.
  return kCounterBytes + rank_project_part_bytes(rows) + rank_grad_part_bytes(cols);
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
  RankProjectArgs g;
  bool vec;
  rank_project_setup(g, a, lda, m, k, w, ldw, w_kr, scale_a ? a_scale : 1.0f, out, workspace,
                     workspace_bytes, m, vec);
  const int waves = rank_plan(k, kProjChunk, g.splits > 1).waves;
  auto kern = vec ? rank_project_kernel<true> : rank_project_kernel<false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(m, 16), (unsigned)g.splits), dim3(64 * waves), 0,
                     (hipStream_t)stream, g);
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
  RankGradArgs g;
  bool vec;
  rank_grad_setup(g, p, ldp, q, ldq, t, n, scale_q ? q_scale : 1.0f, transpose, out, workspace,
                  workspace_bytes, 0, vec);
  const int waves = rank_plan(t, kGradChunk, g.splits > 1).waves;
  auto kern = vec ? rank_grad_kernel<true> : rank_grad_kernel<false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(n, 64), (unsigned)g.splits), dim3(64 * waves), 0,
                     (hipStream_t)stream, g);
  SS_CHECK_LAUNCH("rank_grad_kernel");
  return SS_OK;
}
