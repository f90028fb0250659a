// Fused NF4 GEMM for gfx950: Y[T, N] = X[T, K] . Wdec^T with the NF4 weight
// decoded inside the GEMM, for T above the streaming / skinny kernels' range.
//
// Reference: bnb.matmul_4bit's forward (solution/nf4_patch.py:108-120) and
// the fused tile analogue nf4_tile_matmul_kernel (solution/kernels/
// nf4_gemm.py:35-71: decode a tile, cast to fp16, dot with fp32
// accumulation).  The decode-first path writes the decoded fp16 weight (2 B
// per weight) to memory and reads it back in the GEMM; here the weight moves
// as its codes (0.5 B + 1/64 B of qabs per weight) and the fp16 tile exists
// only in LDS.
//
// The A operand (X rows) and the MFMA / epilogue part are those of the dense
// NT kernel (nt_core.h, same tile configurations, stage depth BK = 32), so a
// launch computes exactly what the decode-first path computes with the same
// configuration: identical fp16 B values (the standalone decoder's
// arithmetic: fp16_rne(fp32(NF4[c]) * fp32(fp32(code2[q] * absmax2) +
// offset))), identical k order.
//
// Per stage kt (32 k) each thread owns DPT = BN * 16 / threads code bytes of
// one weight row (TPR = 16 / DPT threads per row): they come with the row's
// qabs byte and absmax2 entry as plain vector loads into a register ring
// issued D stages ahead (D >= STAGES, the A tile ring's depth), in the same
// per-iteration pattern as the A tile DMAs, so one vmcnt wait covers both.
// The thread decodes them (the 256-entry table of NF4 value pairs, one read
// per code byte, and the 256-entry code2 table in LDS) and writes 2 * DPT
// fp16 values into a double-buffered B tile with the dense kernel's BK = 32
// layout.
//
// Loop, iteration kt: read the fragments of stage kt; wait for stage kt + 1;
// decode stage kt + 1 into the other B tile, its arithmetic interleaved with
// the MFMAs of stage kt (the two waves of a SIMD leave the barrier together,
// so each wave must overlap its own decode with its MFMAs); one barrier (the
// B tile of kt + 1 is complete, every wave is done with A slot kt % STAGES
// and B tile kt % 2); refill the A slot with stage kt + STAGES and the
// register slot with the codes of stage kt + D.

#include "decode_blocks.h"
#include "nt_core.h"

namespace ss {
namespace {

__device__ __forceinline__ u32x2 vload8_off(uint32_t voff, const void* base) {
  u32x2 v;
  asm volatile("global_load_dwordx2 %0, %1, %2" : "=v"(v) : "v"(voff), "s"(base) : "memory");
  return v;
}
__device__ __forceinline__ uint32_t vload4_off(uint32_t voff, const void* base) {
  uint32_t v;
  asm volatile("global_load_dword %0, %1, %2" : "=v"(v) : "v"(voff), "s"(base) : "memory");
  return v;
}
__device__ __forceinline__ uint32_t vload1_off(uint32_t voff, const void* base) {
  uint32_t v;
  asm volatile("global_load_ubyte %0, %1, %2" : "=v"(v) : "v"(voff), "s"(base) : "memory");
  return v;
}

// Code bytes, qabs byte and absmax2 bits of one stage (codes.y unused when
// DPT == 4).
struct Nf4Slot {
  u32x2 codes;
  uint32_t q;
  uint32_t a2;
};

template <class C>
struct Nf4Layout {
  static_assert(C::BK == 32, "fused NF4 stages are 32 k deep");
  static constexpr int DPT = C::BN * 16 / C::kThreads;  // code bytes per thread per stage
  static constexpr int TPR = 16 / DPT;                  // threads per weight row
  static_assert(DPT == 4 || DPT == 8, "decode split");
  static constexpr int kTileA = C::BM * 64;
  static constexpr int kTileB = C::BN * 64;
  static constexpr int kOffB = C::STAGES * kTileA;
  static constexpr int kOffLut = kOffB + 2 * kTileB;
  static constexpr int kOffCode2 = kOffLut + kPairBytes;
  static constexpr int kSmem = kOffCode2 + 1024;
  static constexpr int kOps = C::kDmaA + 3;  // vector-memory ops per stage and wave
  static_assert(kSmem <= 160 * 1024, "LDS");
};

template <class C, int CD>
__device__ __forceinline__ void nf4_mainloop(const GemmParams& p, int64_t m0, int64_t n0,
                                             int64_t kbeg, int64_t klen, unsigned char* smem,
                                             NtAcc<C>& acc) {
  using L = Nf4Layout<C>;
  constexpr int kS = C::STAGES;
  constexpr int kD = CD;  // code ring depth (stages of codes in flight)
  static_assert(kD >= kS && kD % kS == 0, "code ring depth");
  constexpr int kGroupBytes = 32 * 64;  // one 32-row group of a BK = 32 tile
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int wm = wave / C::kWavesN;
  const int wn = wave % C::kWavesN;
  const Nf4View& w = p.w;
  float* const code2 = reinterpret_cast<float*>(smem + L::kOffCode2);

  // Tables first, with tracked loads, before any untracked load is issued.
  const float2* const pair = load_pairs(smem + L::kOffLut);
  for (int i = tid; i < 256; i += C::kThreads) code2[i] = w.code2[i];
  float offset = w.offset[0];
  tie(offset);
  __syncthreads();

  // A tile DMA sources (rows past M clamped; never stored).
  const uint32_t lds0 = lds_address(smem);
  const half_t* a_base = p.A + kbeg;
  uint32_t a_off[C::kDmaA];
#pragma unroll
  for (int j = 0; j < C::kDmaA; ++j) {
    int row, chunk;
    dma_source<32>(wave * C::kDmaA + j, lane, row, chunk);
    const int64_t gr = m0 + row < p.M ? m0 + row : p.M - 1;
    a_off[j] = (uint32_t)((gr * p.lda + chunk * 8) * 2);
  }
  const uint32_t lds_a = __builtin_amdgcn_readfirstlane(lds0 + wave * C::kDmaA * 1024);

  // This thread's weight row (clamped) and byte range within a stage.
  const int brow = tid / L::TPR;
  const int bpart = tid % L::TPR;
  const int64_t wrow = n0 + brow < p.N ? n0 + brow : p.N - 1;
  const int64_t kq = p.K >> 6;  // scale blocks per weight row
  const uint32_t code_off = (uint32_t)(wrow * (p.K >> 1) + (kbeg >> 1) + bpart * L::DPT);
  const int64_t block0 = wrow * kq + (kbeg >> 6);
  const uint32_t q_off = (uint32_t)block0;

  auto issue_a = [&](int64_t kt, int slot_a) {
#pragma unroll
    for (int j = 0; j < C::kDmaA; ++j)
      dma16(a_off[j], a_base + kt * 32, lds_a + slot_a * L::kTileA + j * 1024);
  };
  auto issue_c = [&](int64_t kt, Nf4Slot& sl) {
    const uint8_t* cbase = w.packed + kt * 16;
    if constexpr (L::DPT == 8) {
      sl.codes = vload8_off(code_off, cbase);
    } else {
      sl.codes[0] = vload4_off(code_off, cbase);
    }
    sl.q = vload1_off(q_off, w.qabs + (kt >> 1));
    sl.a2 = vload4_off((uint32_t)(((block0 + (kt >> 1)) >> 8) * 4), w.absmax2);
  };

  // Decode one stage's codes into B tile `buf`: fp16_rne(NF4[c] * scale),
  // element 2j of a byte in its high nibble.
  auto decode = [&](Nf4Slot& sl, int buf) {
    tie(sl.codes);
    tie(sl.q);
    tie(sl.a2);
    const float scale = code2[sl.q & 0xffu] * __builtin_bit_cast(float, sl.a2) + offset;
    unsigned char* bt = smem + L::kOffB + buf * L::kTileB + brow * 64;
#pragma unroll
    for (int h = 0; h < L::DPT / 4; ++h) {
      const uint32_t word = sl.codes[h];
      half8 v;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const float2 pr = pair[(word >> (8 * b)) & 0xffu];
        v[2 * b] = f32_to_f16(pr.x * scale);
        v[2 * b + 1] = f32_to_f16(pr.y * scale);
      }
      const int chunk = bpart * (L::DPT / 4) + h;
      *reinterpret_cast<half8*>(bt + ((chunk ^ swz32(brow)) << 4)) = v;
    }
  };

  int frag_off[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) frag_off[kk] = frag_offset<32>(lane, kk);
  auto read_frags = [&](int slot_a, int buf, int kk, half8 (&af)[C::FM], half8 (&bf)[C::FN]) {
    const unsigned char* sa =
        smem + slot_a * L::kTileA + (wm * C::WM / 32) * kGroupBytes + frag_off[kk];
    const unsigned char* sb =
        smem + L::kOffB + buf * L::kTileB + (wn * C::WN / 32) * kGroupBytes + frag_off[kk];
#pragma unroll
    for (int i = 0; i < C::FM; ++i) af[i] = *reinterpret_cast<const half8*>(sa + i * kGroupBytes);
#pragma unroll
    for (int j = 0; j < C::FN; ++j) bf[j] = *reinterpret_cast<const half8*>(sb + j * kGroupBytes);
  };

  // Every iteration issues the A tile of stage kt + kS and the codes of stage
  // kt + kD (past the end: the last stage again, into slots nobody reads), so
  // the wait counts are the same every time.  The codes run further ahead
  // than the A tiles: at small T they stream from HBM and their latency,
  // not the MFMA, sets the pace.  The prologue is kD virtual iterations
  // -kD .. -1 of the same pattern (the first kD - kS without A tiles).
  const int64_t ktiles = klen / 32;
  auto clampk = [&](int64_t kt) { return kt < ktiles ? kt : ktiles - 1; };
  Nf4Slot ring[kD];
#pragma unroll
  for (int v = -kD; v < 0; ++v) {
    if (v + kS >= 0) issue_a(clampk(v + kS), v + kS);
    issue_c(clampk(v + kD), ring[v + kD]);
  }
  // A tile 0 was followed by the codes of one virtual iteration and kS - 1
  // whole virtual iterations.
  wait_vm<3 + (kS - 1) * L::kOps>();
  decode(ring[0], 0);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");

  // Iteration kt; j = kt % kD is a compile-time constant (the register ring
  // is indexed statically).  The decode of stage kt + 1 (after the last
  // stage: of a repeated stage, into the B tile nobody reads) runs as
  // kSteps micro-steps -- code2 read, per code byte its pair-table read, the
  // scale, per byte two products and a packed conversion, the tile writes --
  // spread between the MFMAs of stage kt (sched_barrier keeps the order):
  // the two waves of a SIMD leave the barrier together, so a wave must
  // overlap its own decode with its MFMAs.
  constexpr int kBytes = L::DPT;
  constexpr int kChunks = L::DPT / 4;
  constexpr int kSteps = 2 * kBytes + 2 + kChunks;
  constexpr int kMfma = 2 * C::FM * C::FN;
  auto iteration = [&](int64_t kt, int j, Nf4Slot& next, Nf4Slot& own) {
    const int sa = j % kS;  // A slot of stage kt
    half8 fa[2][C::FM], fb[2][C::FN];
    read_frags(sa, (int)(kt & 1), 0, fa[0], fb[0]);
    read_frags(sa, (int)(kt & 1), 1, fa[1], fb[1]);
    // Stage kt + 1: its A tile was followed by one iteration's codes and kS - 2
    // whole iterations; its codes were issued before its A tile.
    wait_vm<3 + (kS - 2) * L::kOps>();
    tie(next.codes);
    tie(next.q);
    tie(next.a2);
    unsigned char* const bt = smem + L::kOffB + (int)((kt + 1) & 1) * L::kTileB + brow * 64;
    float c2 = 0.0f, scale = 0.0f;
    float tv[2 * kBytes];
    half8 outv[kChunks];
    auto micro = [&](int st) {
      if (st == 0) {
        c2 = code2[next.q & 0xffu];
      } else if (st <= kBytes) {
        const int b = st - 1;
        const float2 pr = pair[(next.codes[b >> 2] >> (8 * (b & 3))) & 0xffu];
        tv[2 * b] = pr.x;
        tv[2 * b + 1] = pr.y;
      } else if (st == kBytes + 1) {
        scale = c2 * __builtin_bit_cast(float, next.a2) + offset;
      } else if (st <= 2 * kBytes + 1) {
        const int b = st - kBytes - 2;
        outv[b >> 2][2 * (b & 3)] = f32_to_f16(tv[2 * b] * scale);
        outv[b >> 2][2 * (b & 3) + 1] = f32_to_f16(tv[2 * b + 1] * scale);
      } else {
        const int h = st - 2 * kBytes - 2;
        const int chunk = bpart * kChunks + h;
        *reinterpret_cast<half8*>(bt + ((chunk ^ swz32(brow)) << 4)) = outv[h];
      }
    };
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < kMfma; ++m) {
      const int kk = m / (C::FM * C::FN);
      const int i = (m / C::FN) % C::FM;
      const int jj = m % C::FN;
      acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[kk][i], fb[kk][jj], acc[i][jj], 0,
                                                          0, 0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int st = m * kSteps / kMfma; st < (m + 1) * kSteps / kMfma; ++st) micro(st);
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
    issue_a(clampk(kt + kS), sa);
    issue_c(clampk(kt + kD), own);
  };

  for (int64_t kt0 = 0; kt0 < ktiles; kt0 += kD) {
#pragma unroll
    for (int j = 0; j < kD; ++j) {
      if (kt0 + j >= ktiles) break;
      iteration(kt0 + j, j, ring[(j + 1) % kD], ring[j]);
    }
  }
  // No LDS DMA may land after the workgroup ends, and no register load after
  // its register is reused: the loads issued in the last iterations are never
  // decoded, so to the compiler their results are dead as soon as the asm
  // that "produced" them, and it would hand their registers to other values
  // (epilogue addresses) while the loads are still in flight.  The ties keep
  // every ring register allocated until the wait has retired its load.
  wait_vm<0>();
#pragma unroll
  for (int s = 0; s < kD; ++s) {
    tie(ring[s].codes);
    tie(ring[s].q);
    tie(ring[s].a2);
  }
}

// ---------------------------------------------------------------------------
// Fused dX (dX = dY . Wdec).  The weight's rows are the reduction of
// dX = dY . Wdec, so a stage's 32 weight rows, each contiguous over the dX
// columns, are the B operand stored K-major: they are decoded as they lie,
// row pieces as in the forward kernel, into a K-major B tile (32 rows of BN
// halves, 16-byte chunk L of row r at L ^ tsw(r)), and the MFMA fragments
// come out of it through transposed LDS reads (read_frag_t), as in the dense
// kernel's K-major operands.  Thread t owns weight row t / (BN / 16) of the
// stage and its 16 columns 16 (t % (BN / 16)) .. + 15: one 8-byte code piece,
// one block scale (the 16 columns lie in one 64-wide block), eight pair
// lookups and two contiguous 16-byte chunk writes; no code or scale table,
// no transposed code read.  Same fp16 B values (fp16_rne(NF4[c] * scale),
// scale = code2[q] * absmax2 + offset), same MFMA order: the result equals
// the decode-first path's with the same tile plan.
template <class C, int CD>
__device__ __forceinline__ void nf4k_mainloop(const GemmParams& p, int64_t m0, int64_t n0,
                                              int64_t kbeg, int64_t klen, unsigned char* smem,
                                              NtAcc<C>& acc) {
  using L = Nf4Layout<C>;  // A ring, two B tiles of BN x 64 bytes, pair and code2 tables
  constexpr int kS = C::STAGES;
  constexpr int kD = CD;  // code ring depth (stages of codes in flight)
  static_assert(kD >= kS && kD % kS == 0, "code ring depth");
  constexpr int kTpr = C::BN / 16;  // threads per weight row and stage, 8 code bytes each
  static_assert(C::kThreads == 32 * kTpr, "one 8-byte code piece per thread and stage");
  constexpr int kGroupBytes = 32 * 64;  // one 32-row group of the A tile
  constexpr int kRowBytes = C::BN * 2;  // one K-major B tile row
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int wm = wave / C::kWavesN;
  const int wn = wave % C::kWavesN;
  const Nf4View& w = p.w;
  float* const code2 = reinterpret_cast<float*>(smem + L::kOffCode2);

  // Tables first, with tracked loads, before any untracked load is issued.
  const float2* const pair = load_pairs(smem + L::kOffLut);
  for (int i = tid; i < 256; i += C::kThreads) code2[i] = w.code2[i];
  float offset = w.offset[0];
  tie(offset);
  __syncthreads();

  // A tile DMA sources (rows past M clamped; never stored).
  const uint32_t lds0 = lds_address(smem);
  const half_t* a_base = p.A + kbeg;
  uint32_t a_off[C::kDmaA];
#pragma unroll
  for (int j = 0; j < C::kDmaA; ++j) {
    int row, chunk;
    dma_source<32>(wave * C::kDmaA + j, lane, row, chunk);
    const int64_t gr = m0 + row < p.M ? m0 + row : p.M - 1;
    a_off[j] = (uint32_t)((gr * p.lda + chunk * 8) * 2);
  }
  const uint32_t lds_a = __builtin_amdgcn_readfirstlane(lds0 + wave * C::kDmaA * 1024);

  // This thread's weight row of a stage and its first column (columns past N
  // clamped to the last 16; never stored).  Each stage adds 32 weight rows.
  const int brow = tid / kTpr;
  const int bpart = tid % kTpr;
  const int64_t col = n0 + 16 * bpart <= p.N - 16 ? n0 + 16 * bpart : p.N - 16;
  const int64_t kb = p.N >> 1;  // code bytes per weight row
  const int64_t kq = p.N >> 6;  // scale blocks per weight row
  const uint32_t code_off = (uint32_t)((kbeg + brow) * kb + (col >> 1));
  const int64_t block0 = (kbeg + brow) * kq + (col >> 6);
  const uint32_t q_off = (uint32_t)block0;

  auto issue_a = [&](int64_t kt, int slot_a) {
#pragma unroll
    for (int j = 0; j < C::kDmaA; ++j)
      dma16(a_off[j], a_base + kt * 32, lds_a + slot_a * L::kTileA + j * 1024);
  };
  auto issue_c = [&](int64_t kt, Nf4Slot& sl) {
    sl.codes = vload8_off(code_off, w.packed + kt * 32 * kb);
    sl.q = vload1_off(q_off, w.qabs + kt * 32 * kq);
    sl.a2 = vload4_off((uint32_t)(((block0 + kt * 32 * kq) >> 8) * 4), w.absmax2);
  };

  // Micro-steps of one stage's decode into B tile `buf`: the code2 read, per
  // code byte its pair-table read, the scale, per byte two products and a
  // packed conversion, the two chunk writes.
  constexpr int kSteps = 2 * 8 + 2 + 2;
  float c2 = 0.0f, scale = 0.0f;
  float tv[16];
  half8 outv[2];
  auto micro = [&](int st, const Nf4Slot& sl, int buf) {
    if (st == 0) {
      c2 = code2[sl.q & 0xffu];
    } else if (st <= 8) {
      const int b = st - 1;
      const float2 pr = pair[(sl.codes[b >> 2] >> (8 * (b & 3))) & 0xffu];
      tv[2 * b] = pr.x;
      tv[2 * b + 1] = pr.y;
    } else if (st == 9) {
      scale = c2 * __builtin_bit_cast(float, sl.a2) + offset;
    } else if (st <= 17) {
      const int b = st - 10;
      outv[b >> 2][2 * (b & 3)] = f32_to_f16(tv[2 * b] * scale);
      outv[b >> 2][2 * (b & 3) + 1] = f32_to_f16(tv[2 * b + 1] * scale);
    } else {
      const int h = st - 18;
      unsigned char* const bt = smem + L::kOffB + buf * L::kTileB + brow * kRowBytes;
      *reinterpret_cast<half8*>(bt + (((2 * bpart + h) ^ tsw(brow)) << 4)) = outv[h];
    }
  };

  int a_frag[2];
  int b_frag[2][C::FN];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    a_frag[kk] = (wm * C::WM / 32) * kGroupBytes + frag_offset<32>(lane, kk);
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
      b_frag[kk][j] = L::kOffB + frag_offset_t<C::BN>(lane, kk, wn * C::WN + 32 * j);
  }
  auto read_frags = [&](int slot_a, int buf, int kk, half8 (&af)[C::FM], half8 (&bf)[C::FN]) {
    const unsigned char* sa = smem + slot_a * L::kTileA + a_frag[kk];
#pragma unroll
    for (int i = 0; i < C::FM; ++i) af[i] = *reinterpret_cast<const half8*>(sa + i * kGroupBytes);
#pragma unroll
    for (int j = 0; j < C::FN; ++j)
      bf[j] = read_frag_t(smem + buf * L::kTileB + b_frag[kk][j], kRowBytes);
  };

  // The forward kernel's pipeline: every iteration issues the A tile of stage
  // kt + kS and the codes of stage kt + kD (past the end: the last stage
  // again, into slots nobody reads); the prologue is kD virtual iterations.
  const int64_t ktiles = klen / 32;
  auto clampk = [&](int64_t kt) { return kt < ktiles ? kt : ktiles - 1; };
  Nf4Slot ring[kD];
#pragma unroll
  for (int v = -kD; v < 0; ++v) {
    if (v + kS >= 0) issue_a(clampk(v + kS), v + kS);
    issue_c(clampk(v + kD), ring[v + kD]);
  }
  wait_vm<3 + (kS - 1) * L::kOps>();
  tie(ring[0].codes);
  tie(ring[0].q);
  tie(ring[0].a2);
#pragma unroll
  for (int st = 0; st < kSteps; ++st) micro(st, ring[0], 0);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  asm volatile("s_barrier" ::: "memory");

  // Iteration kt: the decode of stage kt + 1 into B tile (kt + 1) % 2 runs as
  // micro-steps between the MFMAs of stage kt; one barrier; the next loads.
  constexpr int kMfma = 2 * C::FM * C::FN;
  auto iteration = [&](int64_t kt, int j, Nf4Slot& next, Nf4Slot& own) {
    const int sa = j % kS;
    half8 fa[2][C::FM], fb[2][C::FN];
    read_frags(sa, (int)(kt & 1), 0, fa[0], fb[0]);
    read_frags(sa, (int)(kt & 1), 1, fa[1], fb[1]);
    wait_vm<3 + (kS - 2) * L::kOps>();
    tie(next.codes);
    tie(next.q);
    tie(next.a2);
    const int buf = (int)((kt + 1) & 1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int m = 0; m < kMfma; ++m) {
      const int kk = m / (C::FM * C::FN);
      const int i = (m / C::FN) % C::FM;
      const int jj = m % C::FN;
      acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[kk][i], fb[kk][jj], acc[i][jj], 0,
                                                          0, 0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int st = m * kSteps / kMfma; st < (m + 1) * kSteps / kMfma; ++st) micro(st, next, buf);
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
    issue_a(clampk(kt + kS), sa);
    issue_c(clampk(kt + kD), own);
  };

  for (int64_t kt0 = 0; kt0 < ktiles; kt0 += kD) {
#pragma unroll
    for (int j = 0; j < kD; ++j) {
      if (kt0 + j >= ktiles) break;
      iteration(kt0 + j, j, ring[(j + 1) % kD], ring[j]);
    }
  }
  // As in the forward: the ring registers stay allocated until every load
  // issued into them has retired.
  wait_vm<0>();
#pragma unroll
  for (int s2 = 0; s2 < kD; ++s2) {
    tie(ring[s2].codes);
    tie(ring[s2].q);
    tie(ring[s2].a2);
  }
}

template <class C, int CD, int CT, int EPI>
__global__ __launch_bounds__(C::kThreads, C::MINW) void gemm_nf4t_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[Nf4Layout<C>::kSmem];
  const int64_t tiles = gridDim.x;
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
  nf4k_mainloop<C, CD>(p, m0, n0, kbeg, klen, smem, acc);
  static_assert(!GluStage<C>::kOk || GluStage<C>::kBytes <= Nf4Layout<C>::kSmem, "stage");
  nt_epilogue<C, CT, EPI>(p, m0, n0, acc, smem, split);
}

template <class C, int CD, int CT, int EPI>
__global__ __launch_bounds__(C::kThreads, C::MINW) void gemm_nf4_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(1024))) unsigned char smem[Nf4Layout<C>::kSmem];
  const int64_t tiles = gridDim.x;
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
  nf4_mainloop<C, CD>(p, m0, n0, kbeg, klen, smem, acc);
  static_assert(!GluStage<C>::kOk || GluStage<C>::kBytes <= Nf4Layout<C>::kSmem, "stage");
  nt_epilogue<C, CT, EPI>(p, m0, n0, acc, smem, split);
}

// Configurations (same tiles, waves and stage depth as the dense kernel's
// configurations 1, 2 and 8).
using Nf4Small = NtCfg<64, 64, 2, 2, 32, 4, 2>;
using Nf4Mid = NtCfg<128, 128, 2, 2, 32, 4, 2>;
using Nf4Big = NtCfg<256, 256, 2, 4, 32, 4, 2>;

template <class C, int CD, int CT, int EPI>
int launch_nf4(const GemmParams& p, int64_t splits, hipStream_t stream) {
  const dim3 grid((unsigned)(cdiv(p.M, C::BM) * cdiv(p.N, C::BN)), (unsigned)splits);
  hipLaunchKernelGGL((gemm_nf4_kernel<C, CD, CT, EPI>), grid, dim3(C::kThreads), 0, stream, p);
  SS_CHECK_LAUNCH("gemm_nf4_kernel");
  return SS_OK;
}

template <int CT, int EPI>
int dispatch_nf4(const GemmParams& p, int cfg, int64_t splits, hipStream_t stream) {
  switch (cfg) {
    case 8: return launch_nf4<Nf4Big, 8, CT, EPI>(p, splits, stream);
    case 2: return launch_nf4<Nf4Mid, 12, CT, EPI>(p, splits, stream);
    default: return launch_nf4<Nf4Small, 12, CT, EPI>(p, splits, stream);
  }
}

using Nf4tMid = Nf4Mid;  // 128x128, 4 waves: one 8-byte code piece per thread and stage
constexpr int kNf4tRing = 12;

template <int CT, int EPI>
int dispatch_nf4t(const GemmParams& p, int64_t splits, hipStream_t stream) {
  const dim3 grid((unsigned)(cdiv(p.M, Nf4tMid::BM) * cdiv(p.N, Nf4tMid::BN)), (unsigned)splits);
  hipLaunchKernelGGL((gemm_nf4t_kernel<Nf4tMid, kNf4tRing, CT, EPI>), grid,
                     dim3(Nf4tMid::kThreads), 0, stream, p);
  SS_CHECK_LAUNCH("gemm_nf4t_kernel");
  return SS_OK;
}

}  // namespace

// Tile plan of the fused kernel: the NT kernel's plan (configurations 1, 2
// and 8 only), except for one or two 128-row tiles, where streaming the
// weight sets the pace: 64x64 tiles up to 64 rows, 128x128 above, split over
// k until about 512 workgroups run, each split at least 512 deep.
NtPlan nf4_plan(int64_t m, int64_t n, int64_t k) {
  if (m > 256) {
    NtPlan plan = nt_plan(m, n, k);
    if (plan.cfg != 1 && plan.cfg != 2 && plan.cfg != 8) plan.cfg = 2;
    return plan;
  }
  NtPlan plan{m <= 64 ? 1 : 2, 1, k};
  const int64_t bm = plan.cfg == 1 ? 64 : 128;
  const int64_t tiles = cdiv(m, bm) * cdiv(n, bm);
  int64_t s = 512 / tiles;
  if (s > k / 512) s = k / 512;
  if (s < 1) s = 1;
  plan.k_split = cdiv(cdiv(k, s), 64) * 64;
  plan.splits = cdiv(k, plan.k_split);
  return plan;
}

bool gemm_nf4_fwd_ok(const GemmParams& p, int epi) {
  if (p.M <= 0 || p.N <= 0 || p.K <= 0 || p.K % 64 != 0) return false;
  if (reinterpret_cast<uintptr_t>(p.A) % 16 != 0 || p.lda % 8 != 0 ||
      reinterpret_cast<uintptr_t>(p.w.packed) % 8 != 0)
    return false;
  // 32-bit offsets: A rows (DMA), code bytes and qabs from their bases.
  const int64_t kMaxOff = (int64_t)1 << 32;
  if (((p.M - 1) * p.lda + p.K) * 2 >= kMaxOff || p.N * (p.K / 2) >= kMaxOff) return false;
  if (epi != EPI_PLAIN && epi != EPI_LORA) return false;
  if (epi == EPI_LORA && (reinterpret_cast<uintptr_t>(p.lz) % 16 != 0 ||
                          reinterpret_cast<uintptr_t>(p.lb) % 16 != 0))
    return false;
  return true;
}

// The fused kernel decodes each weight once per M tile, on the VALU of the
// GEMM's own waves; the decode-first path decodes it once (2 B written and
// read back per weight) and runs the dense GEMM.  Measured on MI355X (HIP
// graph, one call at a time, weights rotated through HBM for the 7B shapes):
//   T in (128, 256] (one or two 128-row tiles): fused ahead at every shape
//     (7B gate 18944 x 3584 at T = 256: 88 vs 103 us; 1.5B gate: 34 vs 44);
//   larger T: behind once the decode runs at the stand-alone decoder's rate
//     (990 x 1536 x 1536: 25.0 vs 24.2 us; 990 x 8960 x 1536: 62.8 vs 56.1;
//     2048 x 18944 x 3584: 392 vs 360).
// T <= 128 stays on the streaming / skinny kernels (7B gate at T = 33: 32 vs
// 48 us fused).
bool gemm_nf4_fwd_preferred(const GemmParams& p) {
  return p.M > kSkinnyMaxT && p.M <= 256;
}

size_t nf4_fused_partial_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0 || k % 64 != 0) return 0;
  const NtPlan plan = nf4_plan(m, n, k);
  return plan.splits > 1 ? (size_t)(plan.splits * m * n) * sizeof(float) : 0;
}

int gemm_nf4_fwd(const GemmParams& p0, int epi, hipStream_t stream, void* partials,
                 size_t partial_bytes) {
  if (!gemm_nf4_fwd_ok(p0, epi)) return SS_ERR_UNSUPPORTED;
  GemmParams p = p0;
  p.c_vec = staged_epilogue_enabled() && !p.beta && p.N % 8 == 0 && p.ldc % 8 == 0 &&
            reinterpret_cast<uintptr_t>(p.C) % 16 == 0;
  NtPlan plan = nf4_plan(p.M, p.N, p.K);
  const size_t need = (size_t)(plan.splits * p.M * p.N) * sizeof(float);
  if (plan.splits > 1 && (!partials || partial_bytes < need ||
                          reinterpret_cast<uintptr_t>(partials) % 16 != 0)) {
    plan.splits = 1;
    plan.k_split = p.K;
  }
  if (plan.splits > 1) {
    p.part = reinterpret_cast<float*>(partials);
    p.k_split = plan.k_split;
    const int rc = dispatch_nf4<SS_F32, EPI_PARTIAL>(p, plan.cfg, plan.splits, stream);
    if (rc) return rc;
    return splitk_reduce(p, (int)plan.splits, SS_F16, epi, stream);
  }
  if (epi == EPI_LORA) return dispatch_nf4<SS_F16, EPI_LORA>(p, plan.cfg, 1, stream);
  if (p.glu) {
    const int rc = dispatch_nf4<SS_F16, EPI_GLU>(p, plan.cfg, 1, stream);
    if (rc == SS_OK && p.glu_done) *p.glu_done = 1;
    return rc;
  }
  return dispatch_nf4<SS_F16, EPI_PLAIN>(p, plan.cfg, 1, stream);
}

// Fused dX (dY . Wdec, the weight decoded into the B tiles): 128x128 tiles,
// split over the weight rows until about 512 workgroups run, each split at
// least 512 rows deep.  For T up to two 128-row tiles, where each weight tile is
// decoded once or twice instead of being written to HBM and read back.
static NtPlan nf4t_plan(int64_t m, int64_t n, int64_t k) {
  NtPlan plan{2, 1, k};
  const int64_t tiles = cdiv(m, 128) * cdiv(n, 128);
  int64_t s = 512 / tiles;
  if (s > k / 512) s = k / 512;
  if (s < 1) s = 1;
  plan.k_split = cdiv(cdiv(k, s), 64) * 64;
  plan.splits = cdiv(k, plan.k_split);
  return plan;
}

bool gemm_nf4_dx_ok(const GemmParams& p, int epi) {
  // p.M = T, p.N = weight columns (dX columns), p.K = weight rows.
  if (p.M <= 0 || p.M > 256 || p.N <= 0 || p.N % 128 != 0 || p.K <= 0 || p.K % 64 != 0)
    return false;
  if (reinterpret_cast<uintptr_t>(p.A) % 16 != 0 || p.lda % 8 != 0 ||
      reinterpret_cast<uintptr_t>(p.w.packed) % 8 != 0)
    return false;
  // 32-bit offsets: A rows (DMA), code bytes and qabs from their bases.
  const int64_t kMaxOff = (int64_t)1 << 32;
  if (((p.M - 1) * p.lda + p.K) * 2 >= kMaxOff || p.K * (p.N / 2) >= kMaxOff) return false;
  if (epi != EPI_PLAIN && epi != EPI_RANK) return false;
  if (epi == EPI_RANK && reinterpret_cast<uintptr_t>(p.lz) % 16 != 0) return false;
  return true;
}

// Measured on MI355X (HIP graph, weights rotated through HBM): with 128 or
// more workgroups in its plan the fused dX is 1.2-2x ahead of decode-first
// (7B gate 18944 x 3584 at T = 128: 45.7 vs 75.6 us; q/o 3584 x 3584 at
// T = 32: 18.3 vs 36.3 us); with fewer (7B k/v 512 x 3584: 28 tiles and no
// split) it is behind (12.9 vs 11.6 us).
bool gemm_nf4_dx_preferred(const GemmParams& p) {
  const NtPlan plan = nf4t_plan(p.M, p.N, p.K);
  return cdiv(p.M, 128) * cdiv(p.N, 128) * plan.splits >= 128;
}

size_t nf4_dx_fused_partial_bytes(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || m > 256 || n <= 0 || k <= 0 || k % 64 != 0) return 0;
  const NtPlan plan = nf4t_plan(m, n, k);
  return plan.splits > 1 ? (size_t)(plan.splits * m * n) * sizeof(float) : 0;
}

int gemm_nf4_dx(const GemmParams& p0, int epi, hipStream_t stream, void* partials,
                size_t partial_bytes) {
  if (!gemm_nf4_dx_ok(p0, epi)) return SS_ERR_UNSUPPORTED;
  // Only the plain and rank-16 epilogues: a caller's SwiGLU epilogue and
  // rank-16 grad tails stay unrun (glu_done / tail_ran untouched), so the
  // caller runs them after the product, as after any path without them.
  GemmParams p = p0;
  p.glu = 0;
  p.tail_blocks = p.tail2_blocks = 0;
  p.c_vec = staged_epilogue_enabled() && !p.beta && p.N % 8 == 0 && p.ldc % 8 == 0 &&
            reinterpret_cast<uintptr_t>(p.C) % 16 == 0;
  NtPlan plan = nf4t_plan(p.M, p.N, p.K);
  const size_t need = (size_t)(plan.splits * p.M * p.N) * sizeof(float);
  if (plan.splits > 1 && (!partials || partial_bytes < need ||
                          reinterpret_cast<uintptr_t>(partials) % 16 != 0)) {
    plan.splits = 1;
    plan.k_split = p.K;
  }
  if (plan.splits > 1) {
    p.part = reinterpret_cast<float*>(partials);
    p.k_split = plan.k_split;
    // As the dense dX: split 0 adds the rank-16 update to its partial and the
    // reduce only sums.
    p.fold_rank = epi == EPI_RANK;
    p.lora_plane = nullptr;
    const int rc = dispatch_nf4t<SS_F32, EPI_PARTIAL>(p, plan.splits, stream);
    if (rc) return rc;
    if (epi == EPI_RANK) {
      p.alpha = 1.0f;
      p.bias = nullptr;
    }
    return splitk_reduce(p, (int)plan.splits, SS_F16, EPI_PLAIN, stream);
  }
  if (epi == EPI_RANK) return dispatch_nf4t<SS_F16, EPI_RANK>(p, 1, stream);
  return dispatch_nf4t<SS_F16, EPI_PLAIN>(p, 1, stream);
}

}  // namespace ss
