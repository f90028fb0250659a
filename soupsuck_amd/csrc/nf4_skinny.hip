// Skinny NF4 forward GEMM for small T: Y[T, N] = X[T, K] . Wdec^T (+ epilogue).
//
// Reference: the bnb fused small-M path behind matmul_4bit (solution/
// nf4_patch.py:108-120, solution/kernels/nf4_gemm.py:127-151).  For T <= 128
// the product is bound by reading the NF4 weight once from HBM (0.5 B codes +
// 1/64 B qabs per weight), not by MFMA: this kernel streams the codes
// straight into registers, decodes them there bit-exactly (the standalone
// decoder's arithmetic) into MFMA B fragments, and never stages the weight in
// LDS or writes it back.
//
// Mapping (v_mfma_f32_16x16x32_f16, fp32 accumulate): a wave owns NB blocks of
// 16 weight rows; per iteration it covers 128 k.  Lane l (r = l % 16,
// g = l / 16) loads the 16 bytes = 32 codes of row n0 + r, k 32 g .. 32 g + 31
// (one load, one NF4 64-block, one scale).  Those 32 k feed four MFMA
// k-steps: k-step j takes k 32 g + 8 j .. + 7 from every lane group g.  The
// MFMA sums over its 32 k in any order, so X is read with the same
// permutation: lane (r, g) supplies X[m + r][32 g + 8 j .. + 7].
// Every load an iteration consumes -- weight runs and X -- is issued PF
// iterations ahead into a register ring (statically indexed by unrolling),
// which keeps tens of KB of weight reads in flight per CU.  X is small and
// L2-resident: for up to two 16-row M tiles each lane loads its 64-byte X
// fragment runs directly (no LDS, no barrier: the waves of a workgroup run
// independently); for more M tiles X is shared through a double-buffered LDS
// tile whose 272-byte row pitch keeps the 16-row fragment reads
// bank-conflict-free.
//
// K is split over grid.y; every split writes fp32 partials [split][T][N] and
// the split-K reduce applies the epilogue (bias, LoRA add) with the GEMM's
// rounding order.

#include "gemm.h"

namespace ss {
namespace {

constexpr int kSkK = 128;          // k per iteration
constexpr int kSkPitch = kSkK + 8; // LDS row pitch of the X tile (halves)
constexpr int kSkNB = 2;           // 16-row weight blocks per wave
constexpr int kSkRowsPerWG = 4 * kSkNB * 16;

// Everything one iteration consumes, loaded kPF iterations ahead: the weight
// runs (codes, qabs byte, absmax2) and the X data -- direct path: the lane's
// 64-byte X fragment run per M tile; LDS path: the thread's X tile chunks.
// Because no load is consumed soon after it is issued, the in-order load
// counter never forces the ring's newer loads to complete early.
template <int MT, bool XLDS>
struct Slot {
  static constexpr int kX = XLDS ? MT : MT * 4;
  u32x4 codes[kSkNB];
  uint32_t q[kSkNB];
  float a2[kSkNB];
  u32x4 x[kX];
};

template <int MT, bool XLDS, int PF>
__global__ __launch_bounds__(256, 2) void nf4_skinny_fwd_kernel(
    const half_t* __restrict__ x, int64_t ldx, int64_t t, Nf4View w, int64_t n, int64_t k,
    int64_t k_split, float* __restrict__ part) {
  using SlotT = Slot<MT, XLDS>;
  __shared__ __attribute__((aligned(16))) half_t sx[XLDS ? 2 : 1][XLDS ? MT * 16 * kSkPitch : 8];
  __shared__ float s_code2[256];
  // Both NF4 values of a code byte in one LDS read: {NF4[e >> 4], NF4[e & 15]}.
  __shared__ __attribute__((aligned(8))) float2 s_pair[256];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  s_code2[tid] = w.code2[tid];
  s_pair[tid] = float2{kNF4[tid >> 4], kNF4[tid & 15]};
  const float offset = w.offset[0];

  const int64_t kbeg = (int64_t)blockIdx.y * k_split;
  const int64_t klen = k - kbeg < k_split ? k - kbeg : k_split;
  const int iters = (int)(klen / kSkK);
  const int64_t wrow0 = (int64_t)blockIdx.x * kSkRowsPerWG + wave * kSkNB * 16;

  // Sources.  Weight rows past N and X rows past T are clamped (their outputs
  // are never stored).
  int64_t code_elem[kSkNB];  // element index of the lane's run at iteration 0
#pragma unroll
  for (int nb = 0; nb < kSkNB; ++nb) {
    int64_t row = wrow0 + nb * 16 + r16;
    row = row < n ? row : n - 1;
    code_elem[nb] = row * k + kbeg + 32 * g;
  }
  const half_t* xsrc[SlotT::kX];
#pragma unroll
  for (int i = 0; i < SlotT::kX; ++i) {
    if constexpr (XLDS) {
      const int c = tid + 256 * i;  // X tile chunk: row c / 16, 16-byte chunk c % 16
      int64_t row = c >> 4;
      row = row < t ? row : t - 1;
      xsrc[i] = x + row * ldx + kbeg + (c & 15) * 8;
    } else {
      const int mt = i >> 2, j = i & 3;  // lane's run X[mt*16 + r][32 g + 8 j ..]
      int64_t row = mt * 16 + r16;
      row = row < t ? row : t - 1;
      xsrc[i] = x + row * ldx + kbeg + 32 * g + 8 * j;
    }
  }
  auto fetch = [&](int it, SlotT& sl) {
#pragma unroll
    for (int nb = 0; nb < kSkNB; ++nb) {
      const int64_t e = code_elem[nb] + (int64_t)it * kSkK;
      const int64_t block = e >> 6;
      sl.codes[nb] = *reinterpret_cast<const u32x4*>(w.packed + (e >> 1));
      sl.q[nb] = w.qabs[block];
      sl.a2[nb] = w.absmax2[block >> 8];
    }
#pragma unroll
    for (int i = 0; i < SlotT::kX; ++i)
      sl.x[i] = *reinterpret_cast<const u32x4*>(xsrc[i] + (int64_t)it * kSkK);
  };

  float4v acc[MT][kSkNB];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nb = 0; nb < kSkNB; ++nb) acc[mt][nb] = float4v{0.f, 0.f, 0.f, 0.f};

  SlotT ring[PF];
  const int last = iters > 0 ? iters - 1 : 0;
  // Slot fills stay in program order (sched_barrier): the ring's depth is
  // only real if slot s is never among the newest outstanding loads when
  // step s reads it.
#pragma unroll
  for (int s = 0; s < PF; ++s) {
    fetch(s < last ? s : last, ring[s]);
    __builtin_amdgcn_sched_barrier(0);
  }
  __syncthreads();  // code tables visible

  auto step = [&](int it, SlotT& sl, bool refill) {
    if constexpr (XLDS) {
      // Publish this iteration's X tile (double buffered: the barrier of the
      // previous iteration ordered every wave's reads of this buffer from two
      // iterations ago before this write).
      const int buf = it & 1;
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int c = tid + 256 * i;
        *reinterpret_cast<u32x4*>(&sx[buf][(c >> 4) * kSkPitch + (c & 15) * 8]) = sl.x[i];
      }
      // LDS-only barrier: __syncthreads() would also wait for every
      // outstanding global load, i.e. drain the prefetch ring.
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this thread's LDS writes done
      asm volatile("s_barrier" ::: "memory");
    }
    half8 bfrag[kSkNB][4];
#pragma unroll
    for (int nb = 0; nb < kSkNB; ++nb) {
      const float scale = s_code2[sl.q[nb]] * sl.a2[nb] + offset;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const uint32_t byte = (sl.codes[nb][j] >> (8 * b)) & 0xffu;
          const float2 pr = s_pair[byte];
          bfrag[nb][j][2 * b] = f32_to_f16(pr.x * scale);
          bfrag[nb][j][2 * b + 1] = f32_to_f16(pr.y * scale);
        }
      }
    }
    // k-step j outermost: the MT x NB MFMAs of one k-step update distinct
    // accumulators, so each MFMA's dependency on the previous update of its
    // accumulator is MT x NB instructions back (m-tile outermost left only
    // NB = 2 independent chains and stalled on every other MFMA).  The X
    // fragments of a k-step are read before its MFMAs.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      half8 af[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if constexpr (XLDS) {
          af[mt] = *reinterpret_cast<const half8*>(
              &sx[it & 1][(mt * 16 + r16) * kSkPitch + 32 * g + 8 * j]);
        } else {
          af[mt] = __builtin_bit_cast(half8, sl.x[mt * 4 + j]);
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nb = 0; nb < kSkNB; ++nb)
          acc[mt][nb] =
              __builtin_amdgcn_mfma_f32_16x16x32_f16(af[mt], bfrag[nb][j], acc[mt][nb], 0, 0, 0);
    }
    // Refill with iteration it + PF, clamped to a valid iteration so that the
    // loads are always issued (the load counts stay the same every
    // iteration).
    __builtin_amdgcn_sched_barrier(0);
    if (refill) fetch(it + PF < last ? it + PF : last, sl);
    __builtin_amdgcn_sched_barrier(0);
  };

  // Main loop: whole groups of PF iterations, straight-line; tail after it.
  const int full = iters / PF * PF;
  for (int it0 = 0; it0 < full; it0 += PF) {
#pragma unroll
    for (int s = 0; s < PF; ++s) step(it0 + s, ring[s], true);
  }
#pragma unroll
  for (int s = 0; s < PF; ++s)
    if (full + s < iters) step(full + s, ring[s], false);

  // Partials: lane holds D[4 g + r][r16] of each 16x16 (rows = X rows, cols =
  // weight rows).
  float* out = part + (int64_t)blockIdx.y * t * n;
#pragma unroll
  for (int nb = 0; nb < kSkNB; ++nb) {
    const int64_t col = wrow0 + nb * 16 + r16;
    if (col >= n) continue;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t row = mt * 16 + 4 * g + r;
        if (row < t) out[row * n + col] = acc[mt][nb][r];
      }
  }
}

}  // namespace

SkinnyPlan skinny_plan(int64_t t, int64_t n, int64_t k) {
  SkinnyPlan plan{0, 0, 0};
  if (t <= 0 || t > kSkinnyMaxT || n <= 0 || k <= 0 || k % kSkK != 0) return plan;
  plan.mt = t <= 16 ? 1 : t <= 32 ? 2 : t <= 64 ? 4 : 8;
  // About two workgroups per CU, each split at least two iterations long.
  const int64_t cols = cdiv(n, kSkRowsPerWG);
  int64_t s = 512 / cols;
  if (s > k / (2 * kSkK)) s = k / (2 * kSkK);
  if (s < 1) s = 1;
  plan.k_split = cdiv(cdiv(k, s), kSkK) * kSkK;
  plan.splits = cdiv(k, plan.k_split);
  return plan;
}

size_t skinny_partial_bytes(int64_t t, int64_t n, int64_t k) {
  const SkinnyPlan plan = skinny_plan(t, n, k);
  return plan.mt ? (size_t)(plan.splits * t * n) * sizeof(float) : 0;
}

int nf4_skinny_fwd(const GemmParams& p, int epi, void* partials, size_t partial_bytes,
                   hipStream_t stream) {
  const SkinnyPlan plan = skinny_plan(p.M, p.N, p.K);
  if (!plan.mt || !partials || partial_bytes < skinny_partial_bytes(p.M, p.N, p.K) ||
      reinterpret_cast<uintptr_t>(partials) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(p.A) % 16 != 0 || p.lda % 8 != 0 ||
      reinterpret_cast<uintptr_t>(p.w.packed) % 16 != 0)
    return SS_ERR_UNSUPPORTED;
  if (epi != EPI_PLAIN && (reinterpret_cast<uintptr_t>(p.lz) % 16 != 0))
    return SS_ERR_UNSUPPORTED;
  float* part = reinterpret_cast<float*>(partials);
  const dim3 grid((unsigned)cdiv(p.N, kSkRowsPerWG), (unsigned)plan.splits);
  switch (plan.mt) {
    case 1:
      hipLaunchKernelGGL((nf4_skinny_fwd_kernel<1, false, 4>), grid, dim3(256), 0, stream, p.A,
                         p.lda, p.M, p.w, p.N, p.K, plan.k_split, part);
      break;
    case 2:
      hipLaunchKernelGGL((nf4_skinny_fwd_kernel<2, false, 3>), grid, dim3(256), 0, stream, p.A,
                         p.lda, p.M, p.w, p.N, p.K, plan.k_split, part);
      break;
    case 4:
      hipLaunchKernelGGL((nf4_skinny_fwd_kernel<4, true, 4>), grid, dim3(256), 0, stream, p.A,
                         p.lda, p.M, p.w, p.N, p.K, plan.k_split, part);
      break;
    default:
      hipLaunchKernelGGL((nf4_skinny_fwd_kernel<8, true, 2>), grid, dim3(256), 0, stream, p.A,
                         p.lda, p.M, p.w, p.N, p.K, plan.k_split, part);
      break;
  }
  SS_CHECK_LAUNCH("nf4_skinny_fwd_kernel");
  GemmParams q = p;
  q.part = part;
  return splitk_reduce(q, (int)plan.splits, SS_F16, epi, stream);
}

}  // namespace ss
