// Streaming NF4 backward for T <= 16 rows: dX[T, K] = dY[T, N] . Wdec[N, K].
//
// Reference: the backward of bnb.matmul_4bit (MatMul4Bit.backward: grad_A =
// grad_output @ dequantize_4bit(B).to(dtype).t(), with B the packed W^T;
// solution/nf4_patch.py:108-120 routes it).  At small T the product is
// bound by reading the packed weight once from HBM, as in the forward, but
// the reduction now runs over weight rows: an MFMA lane needs eight codes of
// one column from eight different rows, and the block scale changes along
// that reduction, so it cannot be applied after the MFMA.
//
// Transposed code reads.  gfx950's ds_read_b64_tr_b4 transposes 4-bit data
// within each 16-lane group: lanes 2j and 2j+1 each point at 8 bytes (16
// codes), and result lane L, byte j holds code L of lane 2j's bytes (low
// nibble) and code L of lane 2j+1's bytes (high nibble) (measured lane
// layout).  With lane L of group g pointing at weight row 16 g + L of the
// unit and all lanes at the same 16 columns, byte j of lane L holds rows
// 16 g + 2j and 16 g + 2j + 1 of one column: a pair along the reduction.
// One 256-entry LDS table lookup turns it into the fp16 pair {NF4[low],
// NF4[high]} (the same bank-replicated table as the forward, halves
// swapped), so four lookups give the eight-row B fragment of
// v_mfma_f32_16x16x32_f16 for column L (column 16 cc + (L ^ 1) of the
// chunk: a code byte holds element 2i in its high nibble); the lane's
// second dword gives rows 16 g + 8 .. 15 for a second MFMA.
//
// Scales.  W[n][k] = fp16(NF4[c]) * s[n][k / 64] up to the per-weight fp16
// rounding of the decode; the scale is folded into dY: the A operand of rows
// n for column block b is dY[t][n] * s[n][b] as a pair of fp16 fragments hi +
// lo (two MFMAs on the same B), exact to about 2^-22, reused by the block's
// four 16-column chunks.  A single fp16 fragment would add a second rounding
// per product and roughly double the error of the decode-first product.  s is
// the decoder's exact nested scale.
//
// Work split.  A workgroup owns 256 columns (4 blocks; grid.x) and a range of
// rows (grid.y, a multiple of 64); its 8 waves take the range's 64-row units
// in turn.  A unit (64 rows x 128 B of codes, plus the rows' qabs dwords and
// absmax2 values) moves into the wave's LDS slot with LDS DMAs of 8 rows x
// 128 B; the slot is refilled once the codes are in registers.  The waves'
// column sums are added through LDS at the end and each row range writes an
// fp32 partial plane; the split-K reduce adds the planes and applies the
// epilogue (rank-16 update, accumulate).

#include "gemm.h"

namespace ss {
namespace {

constexpr int kDxRows = 64;                       // weight rows per unit
constexpr int kDxCols = 256;                      // weight columns per workgroup
constexpr int kDxCodeBytes = kDxRows * kDxCols / 2;  // 8 KiB
constexpr int kDxSlotBytes = kDxCodeBytes + 512;  // + 64 qabs dwords + 64 absmax2 floats
constexpr int kDxWaves = 8;
constexpr int kDxLutRow = 256;
constexpr int kDxLutBytes = 256 * kDxLutRow;
constexpr int kDxCode2Off = kDxLutBytes;                          // per-wave code2 copies
constexpr int kDxScaleOff = kDxCode2Off + kDxWaves * 1024;        // per-wave [4 blocks][64 rows]
constexpr int kDxSlotOff = kDxScaleOff + kDxWaves * 1024;
constexpr int kDxSlotRegion = kDxWaves * kDxSlotBytes;
constexpr int kDxSmemBytes = kDxSlotOff + kDxSlotRegion;
static_assert(kDxSmemBytes <= 160 * 1024, "LDS");

typedef int v2i_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i_t lds_v2i;

struct StreamDxPlan {
  int ok;
  int64_t col_stages;   // grid.x
  int64_t groups;       // grid.y (row ranges)
  int64_t group_rows;   // rows per range (multiple of 64)
};

__global__ __launch_bounds__(kDxWaves * kWave) void nf4_stream_dx_kernel(GemmParams prm,
                                                                         int64_t group_rows) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kDxSmemBytes];
  uint8_t* const s_lut = smem;
  uint8_t* const s_slots = smem + kDxSlotOff;
  float* const s_red = reinterpret_cast<float*>(smem + kDxSlotOff);  // after the stream

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nw = blockDim.x >> 6;
  const int nthr = blockDim.x;
  const int c16 = lane & 15;
  const int g4 = lane >> 4;
  float* const s_code2 = reinterpret_cast<float*>(smem + kDxCode2Off + wave * 1024);
  float* const s_scale = reinterpret_cast<float*>(smem + kDxScaleOff + wave * 1024);
  uint8_t* const slot = s_slots + wave * kDxSlotBytes;
  const Nf4View& w = prm.w;
  const int t = (int)prm.M;
  const int64_t nr = prm.K;   // weight rows (the reduction)
  const int64_t nc = prm.N;   // weight columns (dX columns)
  const int64_t kb = nc >> 1;
  const int64_t kq = nc >> 6;

  const int64_t cs = blockIdx.x;                 // column stage (256 columns)
  const int64_t grp = blockIdx.y;
  const int64_t r0 = grp * group_rows;
  const int64_t r1 = r0 + group_rows < nr ? r0 + group_rows : nr;
  const int n_units = r0 < r1 ? (int)cdiv(r1 - r0, kDxRows) : 0;
  const int my_units = wave < n_units ? (n_units - wave + nw - 1) / nw : 0;

  // Decode table first (compile-time constants, one barrier): row e = 32
  // copies of {fp16(NF4[e & 15]), fp16(NF4[e >> 4])} -- low nibble = the
  // lower weight row of the transposed pair.
  const int nf4h = (int)nf4_half_bits_of(lane & 15);
  for (int i = tid; i < 256 * 8; i += nthr) {
    const int e = i >> 3;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute((e & 15) << 2, nf4h);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute((e >> 4) << 2, nf4h);
    const uint32_t d = lo | (hi << 16);
    *reinterpret_cast<u32x4*>(s_lut + e * kDxLutRow + (i & 7) * 16) = u32x4{d, d, d, d};
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);
  asm volatile("s_barrier" ::: "memory");

  // Loads of unit index i (this wave's i-th unit): eight code DMAs (8 rows x
  // 128 B; row pieces swizzled by (row >> 1) & 7), the 64 rows' qabs dwords
  // and absmax2 values (one lane per row), and this lane's dY fragment (row
  // t = c16 of dY, columns 16 g4 .. + 15 of the unit).  Rows past r1 re-read
  // row r1 - 1; their dY columns are zeroed.  Past T, row 0 is read and
  // zeroed.
  const uint32_t slot_lds = __builtin_amdgcn_readfirstlane(lds_address(slot));
  const int yrow = c16 < t ? c16 : 0;
  u32x4 ynext[2];
  auto issue = [&](int i) {
    const int64_t n0 = r0 + (int64_t)(wave + i * nw) * kDxRows;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int rl = 8 * q + (lane >> 3);
      int64_t row = n0 + rl;
      row = row < r1 ? row : r1 - 1;
      const int piece = (lane & 7) ^ ((rl >> 1) & 7);
      // 32-bit offset arithmetic (the voffset is 32 bits; the 64-bit form let
      // the compiler feed an arbitrary register into the unused high half).
      dma16((uint32_t)(row - r0) * (uint32_t)kb + (uint32_t)(piece * 16),
            w.packed + r0 * kb + cs * (kDxCols / 2), slot_lds + q * 1024);
    }
    int64_t row = n0 + lane;
    row = row < r1 ? row : r1 - 1;
    const int64_t blk = row * kq + cs * 4;
    dma4((uint32_t)(row - r0) * (uint32_t)kq, w.qabs + r0 * kq + cs * 4, slot_lds + kDxCodeBytes);
    dma4((uint32_t)(blk >> 8) * 4u, w.absmax2, slot_lds + kDxCodeBytes + 256);
    int64_t ycol = n0 + 16 * g4;
    ycol = ycol < nr ? ycol : nr - 16;  // a whole group past N (N % 16 == 0) is zeroed
    const half_t* ysrc = prm.A + (int64_t)yrow * prm.lda + ycol;
    ynext[0] = vload16(ysrc);
    ynext[1] = vload16(ysrc + 8);
  };

  // code2 copy, the offset, then the first unit.
  dma16((uint32_t)(lane * 16), w.code2, __builtin_amdgcn_readfirstlane(lds_address(s_code2)));
  uint32_t offset_bits = vload4(w.offset);
  if (my_units > 0) issue(0);

  float4v acc[16];
#pragma unroll
  for (int cc = 0; cc < 16; ++cc) acc[cc] = float4v{0.f, 0.f, 0.f, 0.f};
  const uint32_t lane4 = (uint32_t)(lane & 31) << 2;
  auto lut8 = [&](uint32_t d) -> half8 {
    u32x4 bv;
    bv[0] = *reinterpret_cast<const uint32_t*>(s_lut + __builtin_amdgcn_perm(d, lane4, 0x0C0C0400u));
    bv[1] = *reinterpret_cast<const uint32_t*>(s_lut + __builtin_amdgcn_perm(d, lane4, 0x0C0C0500u));
    bv[2] = *reinterpret_cast<const uint32_t*>(s_lut + __builtin_amdgcn_perm(d, lane4, 0x0C0C0600u));
    bv[3] = *reinterpret_cast<const uint32_t*>(s_lut + __builtin_amdgcn_perm(d, lane4, 0x0C0C0700u));
    return __builtin_bit_cast(half8, bv);
  };

  for (int i = 0; i < my_units; ++i) {
    wait_vm<0>();  // unit i (and, for i = 0, code2 and the offset) is in
    asm volatile("" ::: "memory");
    tie(offset_bits);
    tie(ynext[0]);
    tie(ynext[1]);
    const int64_t n0 = r0 + (int64_t)(wave + i * nw) * kDxRows;
    // dY fragment of this unit: columns n0 + 16 g4 + e, zeroed past T or past
    // the range (r1 is a multiple of 16, so a group is all in or all out).
    half8 y0, y1;
    {
      const bool live = c16 < t && n0 + 16 * g4 < r1;
      const u32x4 z = {0u, 0u, 0u, 0u};
      y0 = __builtin_bit_cast(half8, live ? ynext[0] : z);
      y1 = __builtin_bit_cast(half8, live ? ynext[1] : z);
    }
    // Codes of the 16 column chunks (transposed reads), the row's qabs and
    // absmax2.
    v2i_t cw[16];
    {
      const int rl = 16 * g4 + c16;  // lane's row of the unit
#pragma unroll
      for (int cc = 0; cc < 16; ++cc) {
        const int piece = (cc >> 1) ^ ((rl >> 1) & 7);
        cw[cc] = __builtin_amdgcn_ds_read_tr4_b64_v2i32(
            (lds_v2i*)(slot + rl * 128 + piece * 16 + 8 * (cc & 1)));
      }
    }
    const uint32_t qd = *reinterpret_cast<const uint32_t*>(slot + kDxCodeBytes + 4 * lane);
    const float a2 = *reinterpret_cast<const float*>(slot + kDxCodeBytes + 256 + 4 * lane);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // slot read into registers
    asm volatile("" ::: "memory");
    if (i + 1 < my_units) issue(i + 1);

    // Scales of the unit's 64 rows (row = lane) for its 4 blocks, through the
    // wave's LDS scale table [block][row].
    const float offset = __builtin_bit_cast(float, offset_bits);
#pragma unroll
    for (int b = 0; b < 4; ++b)
      s_scale[b * 64 + lane] = s_code2[(qd >> (8 * b)) & 0xffu] * a2 + offset;
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("" ::: "memory");

#pragma unroll
    for (int b = 0; b < 4; ++b) {
      // One block at a time (keeps its A / B fragments' live ranges short).
      __builtin_amdgcn_sched_barrier(0);
      // A fragments of block b: rows 16 g4 + 0..7 and + 8..15.
      const float4v* sp = reinterpret_cast<const float4v*>(s_scale + b * 64 + 16 * g4);
      float sc[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4v v = sp[q];
        sc[4 * q] = v[0];
        sc[4 * q + 1] = v[1];
        sc[4 * q + 2] = v[2];
        sc[4 * q + 3] = v[3];
      }
      // dY * s as an unevaluated fp16 pair hi + lo (hi = fp16(y s), lo =
      // fp16(y s - hi), each one fused multiply-add with a single rounding),
      // so the scaled operand carries no rounding beyond the reference's
      // decoded-weight rounding; both halves meet the same B fragment.
      half8 r0h, r0l, r1h, r1l;  // rows 16 g4 + 0..7 and + 8..15
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        r0h[e] = (half_t)((float)y0[e] * sc[e]);
        r0l[e] = (half_t)__builtin_fmaf((float)y0[e], sc[e], -(float)r0h[e]);
        r1h[e] = (half_t)((float)y1[e] * sc[8 + e]);
        r1l[e] = (half_t)__builtin_fmaf((float)y1[e], sc[8 + e], -(float)r1h[e]);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int cc = 4 * b + q;
        const half8 b0 = lut8((uint32_t)cw[cc][0]);
        const half8 b1 = lut8((uint32_t)cw[cc][1]);
        acc[cc] = __builtin_amdgcn_mfma_f32_16x16x32_f16(r0h, b0, acc[cc], 0, 0, 0);
        acc[cc] = __builtin_amdgcn_mfma_f32_16x16x32_f16(r0l, b0, acc[cc], 0, 0, 0);
        acc[cc] = __builtin_amdgcn_mfma_f32_16x16x32_f16(r1h, b1, acc[cc], 0, 0, 0);
        acc[cc] = __builtin_amdgcn_mfma_f32_16x16x32_f16(r1l, b1, acc[cc], 0, 0, 0);
      }
    }
  }
  wait_vm<0>();
  // A wave without units never consumed the offset load, and the last unit's
  // loop exit follows a skipped issue of the next unit's dY fragment: keep
  // those registers allocated until the wait above has retired every load.
  tie(offset_bits);
  tie(ynext[0]);
  tie(ynext[1]);

  // Cross-wave sums in rounds of column chunks through the slot region:
  // wave w's value for dY row m, chunk cc, lane column c at
  // s_red[((cc - ca) * nw + w) * t * 16 + m * 16 + c].  Lane (c16, g4) holds
  // rows 4 g4 + i of chunk column c16 (weight column 16 cc + (c16 ^ 1)).
  const int per_chunk = nw * t * 16;
  const int round_chunks = kDxSlotRegion / 4 / per_chunk;
  const int64_t plane = (int64_t)t * nc;
  for (int ca = 0; ca < 16; ca += round_chunks) {
    const int cb = ca + round_chunks < 16 ? ca + round_chunks : 16;
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("s_barrier" ::: "memory");
#pragma unroll
    for (int cc = 0; cc < 16; ++cc) {
      if (cc < ca || cc >= cb) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 4 * g4 + r;
        if (m < t) s_red[((cc - ca) * nw + wave) * t * 16 + m * 16 + c16] = acc[cc][r];
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("s_barrier" ::: "memory");
    const int outs = (cb - ca) * t * 16;
    for (int idx = tid; idx < outs; idx += nthr) {
      const int cl = idx / (t * 16);
      const int rem = idx - cl * t * 16;
      const int m = rem >> 4, c = rem & 15;
      float v = 0.f;
      for (int q = 0; q < nw; ++q) v += s_red[(cl * nw + q) * t * 16 + m * 16 + c];
      const int64_t col = cs * kDxCols + 16 * (ca + cl) + (c ^ 1);
      if (prm.part) {
        prm.part[grp * plane + m * nc + col] = v;
      } else {  // one row range: the plain epilogue here (no reduce launch)
        const float b = prm.bias ? (float)prm.bias[col] : 0.0f;
        store_c<SS_F16>(prm.C, m * prm.ldc + col, v * prm.alpha + b, prm.beta);
      }
    }
  }
}


// Column stages of 256; row ranges so that at most one workgroup per CU runs
// (the LDS holds one), each range at least 8 units (one per wave) when the
// rows allow.
StreamDxPlan stream_dx_plan(int64_t t, int64_t nr, int64_t nc) {
  StreamDxPlan plan{};
  if (t < 1 || t > kStreamDxMaxT || nr < 16 || nr % 16 != 0 || nc < kDxCols || nc % kDxCols != 0)
    return plan;
  const int64_t cus = device_cu_count();
  plan.col_stages = nc / kDxCols;
  int64_t g = cus / plan.col_stages;  // at most one workgroup per CU
  const int64_t g_max = cdiv(nr, kDxRows * kDxWaves);
  if (g > g_max) g = g_max;
  if (g < 1) g = 1;
  plan.group_rows = cdiv(cdiv(nr, g), kDxRows) * kDxRows;
  plan.groups = cdiv(nr, plan.group_rows);
  plan.ok = 1;
  return plan;
}

}  // namespace

size_t stream_dx_partial_bytes(int64_t t, int64_t n, int64_t k) {
  const StreamDxPlan plan = stream_dx_plan(t, n, k);
  return plan.ok ? (size_t)(plan.groups * t * k) * sizeof(float) : 0;
}

int nf4_stream_dx(const GemmParams& p0, int epi, void* partials, size_t partial_bytes,
                  hipStream_t stream) {
  // p0: M = T, N = weight columns (dX columns), K = weight rows (reduction).
  const StreamDxPlan plan = stream_dx_plan(p0.M, p0.K, p0.N);
  if (!plan.ok) return SS_ERR_UNSUPPORTED;
  auto misaligned = [](const void* ptr, uintptr_t a) {
    return reinterpret_cast<uintptr_t>(ptr) % a != 0;
  };
  const size_t need = stream_dx_partial_bytes(p0.M, p0.K, p0.N);
  if (!partials || partial_bytes < need || misaligned(partials, 16)) return SS_ERR_UNSUPPORTED;
  if (misaligned(p0.A, 16) || p0.lda % 8 != 0 || misaligned(p0.w.packed, 16) ||
      misaligned(p0.w.qabs, 4) || misaligned(p0.w.absmax2, 4) || misaligned(p0.w.code2, 16))
    return SS_ERR_UNSUPPORTED;
  // Per-lane DMA offsets are 32-bit, relative to a range's first row.
  if (plan.group_rows * (p0.N / 2) >= ((int64_t)1 << 31) || p0.K * (p0.N / 64) >= ((int64_t)1 << 31))
    return SS_ERR_UNSUPPORTED;
  GemmParams p = p0;
  p.part = reinterpret_cast<float*>(partials);
  // One row range and the plain epilogue: the kernel stores dX itself.
  const bool direct = plan.groups == 1 && epi == EPI_PLAIN;
  if (direct) p.part = nullptr;
  hipLaunchKernelGGL(nf4_stream_dx_kernel, dim3((unsigned)plan.col_stages, (unsigned)plan.groups),
                     dim3(kDxWaves * kWave), 0, stream, p, plan.group_rows);
  SS_CHECK_LAUNCH("nf4_stream_dx_kernel");
  if (direct) return SS_OK;
  p.part = reinterpret_cast<float*>(partials);
  return splitk_reduce(p, (int)plan.groups, SS_F16, epi, stream);
}

}  // namespace ss
