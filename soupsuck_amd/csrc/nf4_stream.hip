// Streaming NF4 forward for T <= 32 rows: Y[T, N] = X[T, K] . Wdec^T.
//
// Reference: bnb.matmul_4bit's forward for few rows (solution/nf4_patch.py:
// 108-120, solution/kernels/nf4_gemm.py:127-151).  At T <= 32 the product is
// bound by reading the packed weight (0.5 B per weight) once from HBM; every
// choice below serves that stream.
//
// Work split.  K is cut into stages of 256; a workgroup owns a contiguous
// range of at most 80 weight rows (one workgroup per CU, equal row counts,
// so every CU moves the same number of bytes) and wave w owns stage w of a
// stage group (grid.y; at most 16 stages per group) for every row of the
// range.  Its X fragments for that stage are loaded into registers once.  A
// unit is 16 rows x 256 k (2 KiB of codes); a wave walks its range's 16-row
// tiles in order, keeping one accumulator per tile in registers, with no
// barrier until the end, where the waves' tile sums are added through LDS
// (the bias / LoRA epilogue is applied there when there is one stage group;
// otherwise fp32 partial planes per group go to the split-K reduce).
//
// Weight stream.  A unit moves into one of the wave's two LDS slots with two
// LDS DMAs of 8 rows x 128 B (one DMA = 64 lanes x 16 B; on MI355X 128-byte
// row pieces stream from HBM at the rate of fully contiguous reads, 64-byte
// pieces at about 75% of it) and two dword DMAs for the rows' 4 qabs bytes
// and absmax2 values; the slot is refilled as soon as the wave has read it
// into registers.  Row pieces are XOR-swizzled (16-byte piece q of row r at
// slot q ^ ((r >> 1) & 7)) so the MFMA-layout reads are free of bank conflicts.
//
// Decode.  v_mfma_f32_16x16x32_f16 with the 16 weight rows of a tile as the
// output columns: lane (c = l % 16, g = l / 16) holds bytes 8 g .. 8 g + 7 of a
// row's 32-byte NF4 block, i.e. k 16 g .. 16 g + 15 of that block, and feeds
// two MFMAs.  Both MFMAs of a block stay inside one 64-element scale block,
// so the scale is applied to the MFMA result (fp32, one FMA per accumulator)
// and the MFMA consumes the unscaled code values fp16(NF4[c]).  A code byte
// (two weights) becomes a packed fp16 pair with one LDS lookup in a 256-entry
// table.  Random lookups into a 1 KiB table are 2.8x slower than
// conflict-free ones (bank conflicts), so the table is replicated across
// banks: entry e for lane l sits at e * 256 + (l % 32) * 4, and one v_perm_b32
// builds that address from the code byte and the lane.  Per weight: half a
// table lookup, half a v_perm and a sixteenth of an FMA.  The 64 block scales
// of a unit are computed once (one per lane) and shared with ds_bpermute.
//
// Numerics: y = sum over blocks of scale * sum(x * fp16(NF4[c])) with fp32
// accumulation, where scale = fp32(code2[qabs] * absmax2) + offset exactly as
// in the decoder.  The decode-first path rounds fp16(NF4[c] * scale) per
// weight instead; both are one fp16 rounding of the weight's code-value part
// away from the exact product, so the two differ by rounding only.

#include "gemm.h"

namespace ss {
namespace {

constexpr int kStK = 256;                          // k per stage
constexpr int kStTile = 16;                        // weight rows per unit / tile
constexpr int kStCodeBytes = kStTile * kStK / 2;   // 2 KiB
constexpr int kStSlotBytes = kStCodeBytes;
constexpr int kStSlots = 28;                       // LDS unit slots per workgroup
constexpr int kStMaxWaves = 16;
constexpr int kStMaxRange = 80;                    // weight rows per workgroup (at most)
constexpr int kStMaxTiles = kStMaxRange / kStTile;
constexpr int kStLoadsPerUnit = 2;                 // DMA instructions per unit
constexpr int kStA2Window = 128;                   // absmax2 entries a wave preloads
constexpr int kStLutRow = 256;                     // bytes per table entry row
constexpr int kStLutBytes = 256 * kStLutRow;
constexpr int kStCode2Off = kStLutBytes;                        // one code2 copy per wave
constexpr int kStSlotOff = kStCode2Off + kStMaxWaves * 1024;
constexpr int kStSlotRegion = kStSlots * kStSlotBytes;
constexpr int kStBiasOff = kStSlotOff + kStSlotRegion;
constexpr int kStLzOff = kStBiasOff + kStMaxRange * 2;
constexpr int kStLbOff = kStLzOff + kStreamMaxT * 32;
constexpr int kStSmemBytes = kStLbOff + 3072;       // lora_B rows: three 1 KiB DMAs
constexpr int64_t kStSmallBytes = (int64_t)8 << 20;  // small weight: codes bytes
static_assert(kStSmemBytes <= 160 * 1024, "LDS");

// Stage / wave plan.  mt = 0 when the kernel does not apply.
struct StreamPlan {
  int mt;           // 16-row M tiles (T <= 16: 1, T <= 32: 2)
  int waves;        // waves per workgroup = stages per group
  int d;            // LDS slots per wave
  int direct;       // one stage group: epilogue in the kernel
  int64_t groups;   // G
  int64_t sg;       // stages per group
  int64_t nwg;      // workgroups (row ranges) per group
};

// D = LDS slots per wave (1 or 2).
template <int MT, int D, int EPI>
__global__ __launch_bounds__(kStMaxWaves / MT * kWave) void nf4_stream_fwd_kernel(
    GemmParams prm, int64_t sg, int64_t nwg, int direct) {
  // One LDS object so that the table sits at LDS address 0: a lookup address
  // is then exactly the v_perm result (no base add; bases past 64 KiB do not
  // fit the ds_read offset field).
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kStSmemBytes];
  uint8_t* const s_lut = smem;

  uint8_t* const s_slots = smem + kStSlotOff;
  float* const s_red = reinterpret_cast<float*>(smem + kStSlotOff);  // after the stream
  half_t* const s_bias = reinterpret_cast<half_t*>(smem + kStBiasOff);
  half_t* const s_lz = reinterpret_cast<half_t*>(smem + kStLzOff);
  half_t* const s_lb = reinterpret_cast<half_t*>(smem + kStLbOff);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
  const int nw = blockDim.x >> 6;
  const int nthr = blockDim.x;
  const int c16 = lane & 15;
  const int g4 = lane >> 4;
  const Nf4View& w = prm.w;
  float* const s_code2 = reinterpret_cast<float*>(smem + kStCode2Off + wave * 1024);
  const int t = (int)prm.M;
  const int64_t n = prm.N, k = prm.K;
  const int64_t kb = k >> 1;   // bytes per weight row
  const int64_t kq = k >> 6;   // scale blocks per weight row

  // Rows [r0, r1) of stage group grp; this wave's stage kst.
  const int64_t grp = blockIdx.y;
  const int64_t r0 = (int64_t)blockIdx.x * n / nwg;
  const int64_t r1 = ((int64_t)blockIdx.x + 1) * n / nwg;
  const int rows = (int)(r1 - r0);
  const int n_tiles = (int)cdiv(rows, kStTile);
  const int64_t kst = grp * sg + wave;
  const bool has_stage = kst < k / kStK;  // the last group may be short
  const int n_units = has_stage ? n_tiles : 0;

  // DMA of tile u's codes into slot `slot`.  Lane offsets are fixed; the
  // tile goes into the scalar base pointer.  Rows past r1 (last tile) re-read
  // row r1 - 1; their results are never stored.
  const uint32_t slots0 = lds_address(s_slots);
  uint32_t code_off[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int rl = 8 * q + (lane >> 3);
    code_off[q] = (uint32_t)(rl * kb) + (uint32_t)(((lane & 7) ^ ((rl >> 1) & 7)) * 16);
  }
  auto issue = [&](int u, int slot) {
    const uint32_t lds =
        __builtin_amdgcn_readfirstlane(slots0 + (uint32_t)((wave * D + slot) * kStSlotBytes));
    const int64_t row0 = r0 + (int64_t)u * kStTile;
    if (row0 + kStTile <= r1) {
      const uint8_t* base = w.packed + row0 * kb + kst * (kStK / 2);
#pragma unroll
      for (int q = 0; q < 2; ++q) dma16(code_off[q], base, lds + q * 1024);
    } else {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int rl = 8 * q + (lane >> 3);
        int64_t row = row0 + rl;
        row = row < r1 ? row : r1 - 1;
        const int piece = (lane & 7) ^ ((rl >> 1) & 7);
        dma16((uint32_t)((row - r0) * kb + piece * 16), w.packed + r0 * kb + kst * (kStK / 2),
              lds + q * 1024);
      }
    }
  };

  // Decode table, first: row e = 32 copies of {fp16(NF4[e >> 4]),
  // fp16(NF4[e & 15])} (a code byte holds element 2j in its high nibble),
  // from compile-time constants.  Its barrier is the only one of the stream;
  // it comes before any memory instruction, whose issue can stall a wave for
  // a microsecond when every wave of the CU starts its loads at once.
  const int nf4h = (int)nf4_half_bits_of(lane & 15);
  for (int i = tid; i < 256 * 8; i += nthr) {
    const int e = i >> 3;
    const uint32_t first = (uint32_t)__builtin_amdgcn_ds_bpermute((e >> 4) << 2, nf4h);
    const uint32_t second = (uint32_t)__builtin_amdgcn_ds_bpermute((e & 15) << 2, nf4h);
    const uint32_t d = first | (second << 16);
    *reinterpret_cast<u32x4*>(s_lut + e * kStLutRow + (i & 7) * 16) = u32x4{d, d, d, d};
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): table writes done
  asm volatile("s_barrier" ::: "memory");

  // Issue order (the vector-memory counter completes in issue order; none of
  // these loads is tracked by the compiler, every wait is explicit):
  //   the wave's own code2 copy -> LDS (DMA), the double-quant offset, the
  //   epilogue operands (bias, lora_B rows, Z; used at the very end), X
  //   fragments, then the first D units.
  // The first unit's wait covers code2, the offset and X; the last wait the
  // epilogue operands.
  dma16((uint32_t)(lane * 16), w.code2, __builtin_amdgcn_readfirstlane(lds_address(s_code2)));
  const int e_rows = rows > 0 ? rows : 1;
  uint32_t bias_v;
  uint32_t offset_bits = vload4(w.offset);
  // This stage's qabs dword (4 blocks) of range rows lane and 64 + lane, and
  // the absmax2 window the range's blocks of this stage fall in (entry
  // a2_base + lane and + 64 + lane); looked up with ds_bpermute per unit.
  const int64_t kst_c = has_stage ? kst : 0;
  const int64_t a2_base = (r0 * kq + kst_c * 4) >> 8;
  const int64_t a2_last = (n * kq - 1) >> 8;
  uint32_t qd_v[2], a2_v[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int lr = 64 * h + lane;
    const int64_t row = r0 + (lr < rows ? lr : rows - 1);
    qd_v[h] = vload4(w.qabs + row * kq + kst_c * 4);
    const int64_t a2i = a2_base + lr < a2_last ? a2_base + lr : a2_last;
    a2_v[h] = vload4(w.absmax2 + a2i);
  }
  {
    const half_t* bsrc = prm.bias ? prm.bias + r0 + (tid < e_rows ? tid : e_rows - 1) : prm.A;
    bias_v = vload_u16(bsrc);
    if constexpr (EPI == EPI_LORA) {
      // lora_B rows of the range and Z straight into LDS (wave 0; 16-byte
      // chunks past the end re-read the last one).
      if (wave == 0) {
        const uint32_t lb_lds = __builtin_amdgcn_readfirstlane(lds_address(s_lb));
#pragma unroll
        for (int c = 0; c < 3; ++c) {
          const int chunk = c * 64 + lane;
          dma16((uint32_t)((chunk < 2 * e_rows ? chunk : 2 * e_rows - 1) * 16), prm.lb + r0 * 16,
                lb_lds + c * 1024);
        }
        dma16((uint32_t)((lane < 2 * t ? lane : 2 * t - 1) * 16), prm.lz,
              __builtin_amdgcn_readfirstlane(lds_address(s_lz)));
      }
    }
  }
  // X fragments of this wave's stage: xf[j][jj][mt] = X[16 mt + c16]
  // [k0 + 64 j + 16 g4 + 8 jj .. + 7]; lanes past T load row 0 and are zeroed
  // once the data is in.
  half8 xf[4][2][MT];
  {
    const int64_t k0 = (has_stage ? kst : 0) * kStK;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int row = 16 * mt + c16;
      const half_t* src = prm.A + (int64_t)(row < t ? row : 0) * prm.lda + k0 + 16 * g4;
      // Only rows below T load (row 16 mt < T always has a lane, so every
      // wave issues the loads and the wait counts hold).
      if (row < t) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int jj = 0; jj < 2; ++jj)
            xf[j][jj][mt] = __builtin_bit_cast(half8, vload16(src + 64 * j + 8 * jj));
      }
    }
  }
  int issued = 0;
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (issued < n_units) issue(issued++, d);


  const uint32_t lane4 = (uint32_t)(lane & 31) << 2;
  // Lane l computes the scale of (row l % 16, block l / 16) of each unit;
  // lane (c16, g4) fetches block j's from lane c16 + 16 j.
  auto lut8 = [&](uint32_t d) -> half8 {
    u32x4 bv;
    bv[0] = *reinterpret_cast<const uint32_t*>(s_lut + __builtin_amdgcn_perm(d, lane4, 0x0C0C0400u));
    bv[1] = *reinterpret_cast<const uint32_t*>(s_lut + __builtin_amdgcn_perm(d, lane4, 0x0C0C0500u));
    bv[2] = *reinterpret_cast<const uint32_t*>(s_lut + __builtin_amdgcn_perm(d, lane4, 0x0C0C0600u));
    bv[3] = *reinterpret_cast<const uint32_t*>(s_lut + __builtin_amdgcn_perm(d, lane4, 0x0C0C0700u));
    return __builtin_bit_cast(half8, bv);
  };

  float4v acc[kStMaxTiles][MT];
#pragma unroll
  for (int u = 0; u < kStMaxTiles; ++u)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[u][mt] = float4v{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int u = 0; u < kStMaxTiles; ++u) {
    if (u >= n_units) break;
    const int slot = u % D;
    // Outstanding DMAs issued after this unit: at most D - 1 units.
    if (D > 1 && issued - u > 1)
      wait_vm<kStLoadsPerUnit>();
    else
      wait_vm<0>();
    asm volatile("" ::: "memory");
    if (u == 0) {  // code2, the offset, qabs, absmax2 and X are in (issued before the units)
      tie(offset_bits);
      tie(qd_v[0]);
      tie(qd_v[1]);
      tie(a2_v[0]);
      tie(a2_v[1]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const bool live = 16 * mt + c16 < t;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) {
            tie(xf[j][jj][mt]);
            if (!live) xf[j][jj][mt] = half8{};
          }
      }
    }
    const uint8_t* sl = s_slots + (wave * D + slot) * kStSlotBytes;
    // Codes: tile row c16, block j, bytes 8 g4 .. + 7.
    u32x2 cw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int piece = 2 * j + (g4 >> 1);
      cw[j] = *reinterpret_cast<const u32x2*>(sl + c16 * 128 + ((piece ^ ((c16 >> 1) & 7)) << 4) +
                                              8 * (g4 & 1));
    }
    // Scale of (tile row c16, block g4): qabs byte g4 of the row's dword,
    // absmax2 entry of the row's blocks of this stage.
    const int lr = u * kStTile + c16;  // row within the range (< 128)
    const uint32_t qd =
        (uint32_t)__builtin_amdgcn_ds_bpermute((lr & 63) << 2, (int)qd_v[u >> 2]);
    const int a2i = (int)((((r0 + lr) * kq + kst * 4) >> 8) - a2_base);
    const uint32_t a2b_lo = (uint32_t)__builtin_amdgcn_ds_bpermute((a2i & 63) << 2, (int)a2_v[0]);
    const uint32_t a2b_hi = (uint32_t)__builtin_amdgcn_ds_bpermute((a2i & 63) << 2, (int)a2_v[1]);
    const float a2 = __builtin_bit_cast(float, a2i < 64 ? a2b_lo : a2b_hi);
    const uint32_t qbyte = (qd >> (8 * g4)) & 0xffu;
    // The slot is free once these reads have returned: refill it.
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("" ::: "memory");
    if (issued < n_units) issue(issued++, slot);

    const float my_scale = s_code2[qbyte] * a2 + __builtin_bit_cast(float, offset_bits);
    float sc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      sc[j] = __builtin_bit_cast(
          float, __builtin_amdgcn_ds_bpermute((c16 + 16 * j) << 2, __builtin_bit_cast(int, my_scale)));
    // Four blocks; the table lookups of block j + 1 are issued before the
    // MFMAs of block j.
    half8 bn0 = lut8(cw[0][0]), bn1 = lut8(cw[0][1]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const half8 b0 = bn0, b1 = bn1;
      if (j < 3) {
        bn0 = lut8(cw[j + 1][0]);
        bn1 = lut8(cw[j + 1][1]);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        float4v tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[j][0][mt], b0,
                                                              float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        tmp = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[j][1][mt], b1, tmp, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[u][mt][i] = __builtin_fmaf(tmp[i], sc[j], acc[u][mt][i]);
      }
    }
  }
  wait_vm<0>();
  tie(bias_v);
  if (direct && tid < rows)  // the host guarantees nthr >= rows
    s_bias[tid] = prm.bias ? __builtin_bit_cast(half_t, (uint16_t)bias_v) : (half_t)0.0f;

  // Cross-wave sums, in rounds of as many tiles as the slot region holds:
  // wave w's value for X row m, tile u, column col at
  // s_red[((u - ua) * nw + w) * t * 16 + m * 16 + col].  Lane (c16, g4)
  // holds rows 16 mt + 4 g4 + i of column c16.
  const int per_tile = nw * t * kStTile;  // floats
  const int round_tiles = kStSlotRegion / 4 / per_tile;
  const int64_t plane = (int64_t)t * n;
  for (int ua = 0; ua < n_tiles; ua += round_tiles) {
    const int ub = ua + round_tiles < n_tiles ? ua + round_tiles : n_tiles;
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("s_barrier" ::: "memory");  // slots / previous round free
#pragma unroll
    for (int u = 0; u < kStMaxTiles; ++u) {
      if (u < ua || u >= ub) continue;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = 16 * mt + 4 * g4 + i;
          if (m < t) s_red[((u - ua) * nw + wave) * t * kStTile + m * kStTile + c16] = acc[u][mt][i];
        }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("s_barrier" ::: "memory");
    const int outs = (ub - ua) * t * kStTile;
    for (int idx = tid; idx < outs; idx += nthr) {
      const int ul = idx / (t * kStTile);
      const int rem = idx - ul * t * kStTile;
      const int m = rem >> 4, col = rem & 15;
      const int lr = (ua + ul) * kStTile + col;  // row within the range
      float v = 0.f;
      for (int q = 0; q < nw; ++q) v += s_red[(ul * nw + q) * t * kStTile + m * kStTile + col];
      if (lr >= rows) continue;
      const int64_t wrow = r0 + lr;
      if (direct) {
        const float b = (float)s_bias[lr];
        half_t o;
        if constexpr (EPI == EPI_LORA) {
          float l = 0.0f;
#pragma unroll
          for (int r = 0; r < 16; ++r) l += (float)s_lz[m * 16 + r] * (float)s_lb[lr * 16 + r];
          const float y = (float)f32_to_f16(v * prm.alpha + b);
          const float scaled = (float)f32_to_f16((float)f32_to_f16(l) * prm.lscale);
          o = f32_to_f16(y + scaled);
        } else {
          o = f32_to_f16(v * prm.alpha + b);
        }
        reinterpret_cast<half_t*>(prm.C)[m * prm.ldc + wrow] = o;
      } else {
        prm.part[grp * plane + m * n + wrow] = v;
      }
    }
  }
}


// Stage groups: one stage per wave, at most 16 waves (T <= 16) or 8 (T <= 32:
// twice the X fragments and accumulators); more groups while there are too
// few 32-row ranges to give every CU one.  Ranges: one workgroup per CU.
// Two LDS slots per wave when they fit, else one.
StreamPlan stream_plan(int64_t t, int64_t n, int64_t k) {
  StreamPlan plan{};
  if (t < 1 || t > kStreamMaxT || n < 1 || k < kStK || k % kStK != 0) return plan;
  const int64_t cus = device_cu_count();
  const int64_t s = k / kStK;
  const int mt = t <= 16 ? 1 : 2;
  const int64_t max_waves = mt == 1 ? kStMaxWaves : kStMaxWaves / 2;
  // Row ranges of at least 32 rows; 16 for a small weight (below), whose
  // latency-bound stream gains from spreading over twice the CUs (7B k/v at
  // T = 1: 7.1 -> 6.1 us, q/o 7.6 -> 6.6 us).
  const bool small_w = n * (k / 2) <= kStSmallBytes && s <= max_waves;
  const int64_t n_ranges = cdiv(n, small_w ? 16 : 32);
  int64_t g = cdiv(s, max_waves);
  int64_t g_fill = cdiv(cus, n_ranges);
  if (g_fill > s) g_fill = s;
  if (g_fill > g) g = g_fill;
  // A small weight (at most 8 MiB of codes) is latency-bound, not
  // bandwidth-bound: every stage in one workgroup, so the epilogue runs in
  // the kernel and no partial planes or reduce launch follow (7B k/v at T =
  // 1: 10.8 -> 7.0 us, q/o: 9.8 -> 7.6 us, although fewer CUs stream it).
  if (small_w) g = 1;
  plan.sg = cdiv(s, g);
  plan.groups = cdiv(s, plan.sg);
  plan.waves = (int)plan.sg;
  plan.d = 2 * plan.waves <= kStSlots ? 2 : 1;
  int64_t nwg = cus / plan.groups;
  if (nwg > n_ranges) nwg = n_ranges;
  if (nwg < 1) nwg = 1;
  const int64_t max_rows = cdiv(n, nwg);
  if (max_rows > kStMaxRange) return StreamPlan{};  // rows per range beyond the tile registers
  // The absmax2 entries of a range's blocks in one stage must fit the
  // preloaded window.
  if ((kStMaxRange * (k / 64)) / 256 + 2 > kStA2Window) return StreamPlan{};
  plan.nwg = nwg;
  plan.mt = mt;
  // In-kernel epilogue: one group, and enough threads to stage the range's
  // bias.
  plan.direct = plan.groups == 1 && plan.waves * kWave >= max_rows;
  return plan;
}

template <int MT, int D>
void launch_stream(const GemmParams& p, const StreamPlan& plan, int epi, hipStream_t stream) {
  const dim3 grid((unsigned)plan.nwg, (unsigned)plan.groups);
  const dim3 block((unsigned)(plan.waves * kWave));
  if (plan.direct && epi == EPI_LORA)
    hipLaunchKernelGGL((nf4_stream_fwd_kernel<MT, D, EPI_LORA>), grid, block, 0, stream, p,
                       plan.sg, plan.nwg, plan.direct);
  else
    hipLaunchKernelGGL((nf4_stream_fwd_kernel<MT, D, EPI_PLAIN>), grid, block, 0, stream, p,
                       plan.sg, plan.nwg, plan.direct);
}

}  // namespace

size_t stream_partial_bytes(int64_t t, int64_t n, int64_t k) {
  const StreamPlan plan = stream_plan(t, n, k);
  return plan.mt && !plan.direct ? (size_t)(plan.groups * t * n) * sizeof(float) : 0;
}

int nf4_stream_fwd(const GemmParams& p0, int epi, void* partials, size_t partial_bytes,
                   hipStream_t stream) {
  const StreamPlan plan = stream_plan(p0.M, p0.N, p0.K);
  if (!plan.mt || (epi != EPI_PLAIN && epi != EPI_LORA) || p0.beta) return SS_ERR_UNSUPPORTED;
  const size_t need = stream_partial_bytes(p0.M, p0.N, p0.K);
  auto misaligned = [](const void* ptr, uintptr_t a) {
    return reinterpret_cast<uintptr_t>(ptr) % a != 0;
  };
  if (need && (!partials || partial_bytes < need || misaligned(partials, 16)))
    return SS_ERR_UNSUPPORTED;
  if (misaligned(p0.A, 16) || p0.lda % 8 != 0 || misaligned(p0.w.packed, 16) ||
      misaligned(p0.w.qabs, 4) || misaligned(p0.w.absmax2, 4) || misaligned(p0.w.code2, 16))
    return SS_ERR_UNSUPPORTED;
  if (epi == EPI_LORA && (misaligned(p0.lz, 16) || misaligned(p0.lb, 16))) return SS_ERR_UNSUPPORTED;
  // Per-lane DMA offsets are 32-bit, relative to a workgroup's first row.
  if (cdiv(p0.N, plan.nwg) * (p0.K / 2) >= ((int64_t)1 << 31) ||
      p0.N * (p0.K / 64) >= ((int64_t)1 << 31))
    return SS_ERR_UNSUPPORTED;
  GemmParams p = p0;
  p.part = reinterpret_cast<float*>(partials);
  if (plan.mt == 1) {
    if (plan.d == 1)
      launch_stream<1, 1>(p, plan, epi, stream);
    else
      launch_stream<1, 2>(p, plan, epi, stream);
  } else {
    launch_stream<2, 2>(p, plan, epi, stream);
  }
  SS_CHECK_LAUNCH("nf4_stream_fwd_kernel");
  if (plan.direct) return SS_OK;
  return splitk_reduce(p, (int)plan.groups, SS_F16, epi, stream);
}

}  // namespace ss
