// Causal attention over packed rows (varlen), forward and backward, head_dim 128.
//
// Replaces the reference's per-row SDPA loop over a packed batch
// (solution/unpad.py:359-410: each real row of length L attends causally to
// itself only; GQA by repeating the KV heads; scale 1/sqrt(head_dim)).  Rows
// are given by cu_seqlens (int32 [rows + 1], offsets into the packed token
// axis); a query attends to the keys of its own row at positions <= its own.
//
// Layout (HBM): q [T, Hq, 128], k / v [T, Hk, 128] with any token and head
// strides (unit last stride), o [T, Hq, 128] likewise, fp16; lse2 fp32 [Hq, T]
// holds m + log2(l) of the base-2 scaled scores (the backward's softmax
// statistic).  Scores are s = (q . k) * scale in fp32 (MFMA accumulate),
// softmax in fp32 with an online maximum, P rounded to fp16 for the P.V MFMA,
// O accumulated in fp32 and rounded once.
//
// MFMA: gfx950's v_mfma_f32_16x16x32_f16 (lane l supplies k 8 (l / 16) .. + 7
// of row / column l % 16; the accumulator gives lane l rows 4 (l / 16) + i of
// column l % 16).  The k order inside one MFMA is free as long as both operands
// use it, so two 16-key score tiles' accumulators (keys 4 (l / 16) + i and
// 16 + 4 (l / 16) + i of one column) form the 8-slot B operand P^T of O^T +=
// V^T . P^T in registers, with no shuffle, and V^T supplies the same keys in the
// same slots.  Each wave owns 16 queries (forward, dQ) or 16 keys (dK / dV); 4
// waves per workgroup share the LDS tiles of the other operand.
//
// Operands whose MFMA layout runs along the token axis of a row-major LDS tile
// (V in O^T += V^T . P^T, K in dQ += dS . K, Q and dO in dK / dV) are read
// straight from that tile with gfx950's ds_read_b64_tr_b16 (ld4_tr): no
// transposed copy of any tile is built.
//
// Backward: a dQ kernel per (row, 64 queries, q head), which also writes
// delta = rowsum(dO . O); then a dK / dV kernel per (row, 64 keys, q head)
// over the causal query tiles; with GQA each q head writes fp32 partials that
// a reduce kernel adds in head order (no atomics, deterministic).
#include "common.h"

namespace ss {
namespace {

constexpr int kD = 128;        // head dimension
constexpr int kBlk = 64;       // queries / keys per workgroup (4 waves x 16)
constexpr int kLdRow = kD + 8; // padded LDS row of a [token][d] tile (halfs, 16-byte rows)
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
  const half_t* q; int64_t q_tok, q_head;
  const half_t* k; int64_t k_tok, k_head;
  const half_t* v; int64_t v_tok, v_head;
  const half_t* o; int64_t o_tok, o_head;     // forward output / backward input
  const half_t* dout; int64_t do_tok, do_head;
  half_t* out; int64_t out_tok, out_head;     // forward O, or backward dQ
  half_t* dk; int64_t dk_tok, dk_head;
  half_t* dv; int64_t dv_tok, dv_head;
  float* lse2;      // [hq][total]
  float* delta;     // [hq][total]
  const int* cu;    // [rows + 1]
  int64_t total;
  int hq, hk;
  float scale;      // softmax scale (1/sqrt(128) for Qwen2)
};

__device__ __forceinline__ float4v mfma32(half8 a, half8 b, float4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ half8 cat8(half4 lo, half4 hi) {
  return half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}


typedef short attn_short4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) attn_short4 attn_lds_short4;

// MFMA 16x16x16 operand of a row-major LDS tile T[token][d] along its token
// axis: lane l (column c = l % 16, group g = l / 16) receives T[t0 + 4 g + j][d0 +
// c] for j = 0..3.  One ds_read_b64_tr_b16: in each 16-lane group the lanes'
// 8-byte reads form a 16 x 4 matrix M (row = reading lane) and lane i receives
// M[4 j + i / 4][i % 4] (measured on gfx950), so lane r of the group points at
// T[t0 + 4 g + r / 4][d0 + 4 (r % 4)].
__device__ __forceinline__ half4 ld4_tr(const half_t (*tile)[kLdRow], int t0, int d0, int lane) {
  const int r = lane & 15, g = lane >> 4;
  const half_t* p = &tile[t0 + 4 * g + (r >> 2)][d0 + 4 * (r & 3)];
  const attn_short4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((attn_lds_short4*)p);
  return __builtin_bit_cast(half4, v);
}
__device__ __forceinline__ half8 ld8(const half_t* p) { return *reinterpret_cast<const half8*>(p); }

__device__ __forceinline__ float xor_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, kWave));
  return fmaxf(v, __shfl_xor(v, 32, kWave));
}
__device__ __forceinline__ float xor_sum(float v) {
  v += __shfl_xor(v, 16, kWave);
  return v + __shfl_xor(v, 32, kWave);
}

// Register staging of ROWS token rows [t0, t0 + ROWS) of two operands of one
// head (K and V, or Q and dO): fetch() issues the global loads (rows past the
// row end re-read the last row; their results are masked), stage() writes
// them into row-major LDS tiles.  The loops fetch the next tile before
// computing on the current one, so its loads are in flight meanwhile.
template <int ROWS>
struct TilePair {
  static constexpr int kPer = ROWS * (kD / 8) / 256;  // 16-byte chunks per thread and operand
  half8 a[kPer], b[kPer];
  __device__ __forceinline__ void fetch(const half_t* base_a, int64_t tok_a, const half_t* base_b,
                                        int64_t tok_b, int start, int len, int t0) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + 256 * i;
      const int r = c >> 4, ch = c & 15;
      const int64_t t = start + min(t0 + r, len - 1);
      a[i] = ld8(base_a + t * tok_a + ch * 8);
      b[i] = ld8(base_b + t * tok_b + ch * 8);
    }
  }
  __device__ __forceinline__ void stage(half_t (*ta)[kLdRow], half_t (*tb)[kLdRow]) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = threadIdx.x + 256 * i;
      const int r = c >> 4, ch = c & 15;
      *reinterpret_cast<half8*>(&ta[r][ch * 8]) = a[i];
      *reinterpret_cast<half8*>(&tb[r][ch * 8]) = b[i];
    }
  }
};

// ------------------------------------------------------------------ forward

__global__ __launch_bounds__(256) void attn_fwd_kernel(AttnArgs a) {
  const int row = blockIdx.z, h = blockIdx.y;
  const int start = a.cu[row], len = a.cu[row + 1] - start;
  const int q0 = blockIdx.x * kBlk;
  if (q0 >= len) return;
  const int kvh = h / (a.hq / a.hk);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, grp = lane >> 4;
  const int myq = q0 + wave * 16 + col;  // the query of this lane's column
  const float sl2 = a.scale * kLog2e;

  __shared__ __align__(16) half_t sK[kBlk][kLdRow];
  __shared__ __align__(16) half_t sV[kBlk][kLdRow];

  half8 qf[4];  // B operand of S^T = K . Q^T: Q[myq][32 ks + 8 grp + j]
  {
    const half_t* qp = a.q + (int64_t)(start + min(myq, len - 1)) * a.q_tok + (int64_t)h * a.q_head;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) qf[ks] = ld8(qp + ks * 32 + grp * 8);
  }
  float4v acc[8];  // O^T tiles: [d = 16 dt + 4 grp + i][q = myq]
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) acc[dt] = float4v{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;

  const int kend = min(len, q0 + kBlk);  // causal: keys beyond the block's last query unused
  const half_t* kbase = a.k + (int64_t)kvh * a.k_head;
  const half_t* vbase = a.v + (int64_t)kvh * a.v_head;
  // Two tiles in flight: block kb computes while blocks kb + 64 and kb + 128 load.
  TilePair<kBlk> kv0, kv1;
  kv0.fetch(kbase, a.k_tok, vbase, a.v_tok, start, len, 0);
  if (kBlk < kend) kv1.fetch(kbase, a.k_tok, vbase, a.v_tok, start, len, kBlk);
  auto block = [&](int kb, TilePair<kBlk>& kv) {
    __syncthreads();
    kv.stage(sK, sV);
    __syncthreads();
    if (kb + 2 * kBlk < kend)
      kv.fetch(kbase, a.k_tok, vbase, a.v_tok, start, len, kb + 2 * kBlk);
    float4v s[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      s[kt] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        s[kt] = mfma32(ld8(&sK[kt * 16 + col][ks * 32 + grp * 8]), qf[ks], s[kt]);
    }
    // s[kt][i] = S^T[key = kb + 16 kt + 4 grp + i][q = myq]; base-2 scaled, masked.
    float mx = m;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kb + kt * 16 + grp * 4 + i;
        const float x = (key <= myq && key < len) ? s[kt][i] * sl2 : -INFINITY;
        s[kt][i] = x;
        mx = fmaxf(mx, x);
      }
    mx = xor_max(mx);
    const float alpha = exp2f(m - mx);
    float rs = 0.f;
    half4 p[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = exp2f(s[kt][i] - mx);
        rs += e;
        p[kt][i] = f32_to_f16(e);
      }
    rs = xor_sum(rs);
    l = l * alpha + rs;
    m = mx;
    // O^T += V^T . P^T over the block's 64 keys in two 32-deep steps: step u pairs
    // key tiles 2u and 2u + 1 (k slots 8 grp + i <-> key 32 u + 4 grp + i, 8 grp + 4 + i
    // <-> key 32 u + 16 + 4 grp + i), the same slot order for V^T (two transposed
    // reads) and P^T (the two score tiles' registers).
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      acc[dt] *= alpha;
#pragma unroll
      for (int u = 0; u < 2; ++u)
        acc[dt] = mfma32(cat8(ld4_tr(sV, 32 * u, dt * 16, lane),
                              ld4_tr(sV, 32 * u + 16, dt * 16, lane)),
                         cat8(p[2 * u], p[2 * u + 1]), acc[dt]);
    }
  };
  for (int kb = 0; kb < kend; kb += 2 * kBlk) {
    block(kb, kv0);
    if (kb + kBlk < kend) block(kb + kBlk, kv1);
  }
  if (myq < len) {
    const float inv = 1.0f / l;
    half_t* op = a.out + (int64_t)(start + myq) * a.out_tok + (int64_t)h * a.out_head;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      half4 v;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = f32_to_f16(acc[dt][i] * inv);
      *reinterpret_cast<half4*>(op + dt * 16 + grp * 4) = v;
    }
    if (grp == 0) a.lse2[(int64_t)h * a.total + start + myq] = m + __log2f(l);
  }
}

// --------------------------------------------------------------- backward dQ

__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(AttnArgs a) {
  const int row = blockIdx.z, h = blockIdx.y;
  const int start = a.cu[row], len = a.cu[row + 1] - start;
  const int q0 = blockIdx.x * kBlk;
  if (q0 >= len) return;
  const int kvh = h / (a.hq / a.hk);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, grp = lane >> 4;
  const int q0w = q0 + wave * 16;
  const int myq = q0w + col;
  const int qc = min(myq, len - 1);
  const float sl2 = a.scale * kLog2e;

  __shared__ __align__(16) half_t sK[kBlk][kLdRow];
  __shared__ __align__(16) half_t sV[kBlk][kLdRow];

  half8 qf[4], df[4];  // Q[myq][32 ks + 8 grp + j], dO[myq][...]
  float dsum = 0.f;    // this lane's part of rowsum(dO . O)
  {
    const half_t* qp = a.q + (int64_t)(start + qc) * a.q_tok + (int64_t)h * a.q_head;
    const half_t* dp = a.dout + (int64_t)(start + qc) * a.do_tok + (int64_t)h * a.do_head;
    const half_t* op = a.o + (int64_t)(start + qc) * a.o_tok + (int64_t)h * a.o_head;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      qf[ks] = ld8(qp + ks * 32 + grp * 8);
      df[ks] = ld8(dp + ks * 32 + grp * 8);
      const half8 ov = ld8(op + ks * 32 + grp * 8);
#pragma unroll
      for (int j = 0; j < 8; ++j) dsum += (float)df[ks][j] * (float)ov[j];
    }
  }
  const float delta = xor_sum(dsum);
  const float lse = a.lse2[(int64_t)h * a.total + start + qc];
  if (myq < len && grp == 0) a.delta[(int64_t)h * a.total + start + myq] = delta;

  float4v dq[8];  // dQ tiles: [q = q0w + 4 grp + i][d = 16 dt + col]
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) dq[dt] = float4v{0.f, 0.f, 0.f, 0.f};

  const int kend = min(len, q0 + kBlk);
  const half_t* kbase = a.k + (int64_t)kvh * a.k_head;
  const half_t* vbase = a.v + (int64_t)kvh * a.v_head;
  // One tile ahead (a second one in flight measured slower here: more registers).
  TilePair<kBlk> kv;
  kv.fetch(kbase, a.k_tok, vbase, a.v_tok, start, len, 0);
  for (int kb = 0; kb < kend; kb += kBlk) {
    __syncthreads();
    kv.stage(sK, sV);
    __syncthreads();
    if (kb + kBlk < kend) kv.fetch(kbase, a.k_tok, vbase, a.v_tok, start, len, kb + kBlk);
    half4 ds[4];  // dS^T[key = kb + 16 kt + 4 grp + i][q = myq] = A of dS (rows q)
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      float4v s = float4v{0.f, 0.f, 0.f, 0.f}, dp = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        s = mfma32(ld8(&sK[kt * 16 + col][ks * 32 + grp * 8]), qf[ks], s);   // S^T
        dp = mfma32(ld8(&sV[kt * 16 + col][ks * 32 + grp * 8]), df[ks], dp); // dP^T
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kb + kt * 16 + grp * 4 + i;
        const float p = (key <= myq && key < len) ? exp2f(s[i] * sl2 - lse) : 0.f;
        ds[kt][i] = f32_to_f16(p * (dp[i] - delta));
      }
    }
    // dQ += dS . K over the block's keys in two 32-deep steps (the forward's P.V slot order).
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int u = 0; u < 2; ++u)
        dq[dt] = mfma32(cat8(ds[2 * u], ds[2 * u + 1]),
                        cat8(ld4_tr(sK, 32 * u, dt * 16, lane),
                             ld4_tr(sK, 32 * u + 16, dt * 16, lane)), dq[dt]);
  }
  half_t* base = a.out + (int64_t)h * a.out_head;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int q = q0w + grp * 4 + i;
    if (q < len) {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
        base[(int64_t)(start + q) * a.out_tok + dt * 16 + col] = f32_to_f16(dq[dt][i] * a.scale);
    }
  }
}

// ------------------------------------------------------------ backward dK/dV

constexpr int kQt = 64;           // queries per LDS tile of the dK / dV kernel

// One workgroup per (row, 64 keys, q head): 4 waves of 16 keys walk the row's
// causal query tiles.  With GQA (hq > hk) the q heads of a group write fp32
// partial dK / dV planes that attn_bwd_reduce_kernel adds in head order;
// without it dK / dV are written directly.
__global__ __launch_bounds__(256) void attn_bwd_dkdv_kernel(AttnArgs a, float* part_k,
                                                            float* part_v) {
  const int row = blockIdx.z, h = blockIdx.y;
  const int start = a.cu[row], len = a.cu[row + 1] - start;
  const int k0 = blockIdx.x * kBlk;
  if (k0 >= len) return;
  const int kvh = h / (a.hq / a.hk);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 15, grp = lane >> 4;
  const int k0w = k0 + wave * 16;
  const int mykey = k0w + col;
  const int kc = min(mykey, len - 1);
  const float sl2 = a.scale * kLog2e;

  __shared__ __align__(16) half_t sQ[kQt][kLdRow];
  __shared__ __align__(16) half_t sO[kQt][kLdRow];    // dO rows
  __shared__ float sL[kQt], sDl[kQt];                 // lse2 and delta of the tile's queries

  half8 kf[4], vf[4];  // K[mykey][32 ks + 8 grp + j], V[mykey][...]
  {
    const half_t* kp = a.k + (int64_t)(start + kc) * a.k_tok + (int64_t)kvh * a.k_head;
    const half_t* vp = a.v + (int64_t)(start + kc) * a.v_tok + (int64_t)kvh * a.v_head;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      kf[ks] = ld8(kp + ks * 32 + grp * 8);
      vf[ks] = ld8(vp + ks * 32 + grp * 8);
    }
  }
  float4v dk[8], dv[8];  // [key = k0w + 4 grp + i][d = 16 dt + col]
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) {
    dk[dt] = float4v{0.f, 0.f, 0.f, 0.f};
    dv[dt] = float4v{0.f, 0.f, 0.f, 0.f};
  }

  const half_t* qbase = a.q + (int64_t)h * a.q_head;
  const half_t* dbase = a.dout + (int64_t)h * a.do_head;
  // Query tile [qt, qt + kQt): Q and dO rows, lse2, delta (fetched one tile ahead).
  TilePair<kQt> qo;
  float nl = 0.f, nd = 0.f;
  auto fetch = [&](int qt) {
    qo.fetch(qbase, a.q_tok, dbase, a.do_tok, start, len, qt);
    if (threadIdx.x < kQt) {
      const int64_t idx = (int64_t)h * a.total + start + min(qt + (int)threadIdx.x, len - 1);
      nl = a.lse2[idx];
      nd = a.delta[idx];
    }
  };
  fetch(k0);
  for (int qt = k0; qt < len; qt += kQt) {
    __syncthreads();
    qo.stage(sQ, sO);
    if (threadIdx.x < kQt) {
      sL[threadIdx.x] = nl;
      sDl[threadIdx.x] = nd;
    }
    __syncthreads();
    if (qt + kQt < len) fetch(qt + kQt);
    // P^T / dS^T as A operands: [key = mykey][q = qt + 16 sub + 4 grp + i]
    half4 p16[kQt / 16], ds16[kQt / 16];
#pragma unroll
    for (int sub = 0; sub < kQt / 16; ++sub) {
      float4v s = float4v{0.f, 0.f, 0.f, 0.f}, dp = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        s = mfma32(ld8(&sQ[sub * 16 + col][ks * 32 + grp * 8]), kf[ks], s);   // S[q][key]
        dp = mfma32(ld8(&sO[sub * 16 + col][ks * 32 + grp * 8]), vf[ks], dp); // dP[q][key]
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ql = sub * 16 + grp * 4 + i;
        const int q = qt + ql;
        const float p = (mykey <= q && q < len && mykey < len)
                            ? exp2f(s[i] * sl2 - sL[ql]) : 0.f;
        p16[sub][i] = f32_to_f16(p);
        ds16[sub][i] = f32_to_f16(p * (dp[i] - sDl[ql]));
      }
    }
    // dV += P^T . dO and dK += dS^T . Q over the tile's queries, 32 per step (the
    // forward's P.V slot order).
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int u = 0; u < kQt / 32; ++u) {
        dv[dt] = mfma32(cat8(p16[2 * u], p16[2 * u + 1]),
                        cat8(ld4_tr(sO, 32 * u, dt * 16, lane),
                             ld4_tr(sO, 32 * u + 16, dt * 16, lane)), dv[dt]);
        dk[dt] = mfma32(cat8(ds16[2 * u], ds16[2 * u + 1]),
                        cat8(ld4_tr(sQ, 32 * u, dt * 16, lane),
                             ld4_tr(sQ, 32 * u + 16, dt * 16, lane)), dk[dt]);
      }
  }
  const bool direct = a.hq == a.hk;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = k0w + grp * 4 + i;
    if (key >= len) continue;
    if (direct) {
      half_t* kb = a.dk + (int64_t)kvh * a.dk_head + (int64_t)(start + key) * a.dk_tok;
      half_t* vb = a.dv + (int64_t)kvh * a.dv_head + (int64_t)(start + key) * a.dv_tok;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        kb[dt * 16 + col] = f32_to_f16(dk[dt][i] * a.scale);
        vb[dt * 16 + col] = f32_to_f16(dv[dt][i]);
      }
    } else {
      float* kp = part_k + ((int64_t)h * a.total + start + key) * kD;
      float* vp = part_v + ((int64_t)h * a.total + start + key) * kD;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        kp[dt * 16 + col] = dk[dt][i];
        vp[dt * 16 + col] = dv[dt][i];
      }
    }
  }
}

// dK / dV of a GQA group: the q heads' fp32 partials added in head order
// (deterministic), dK scaled; four consecutive d per thread.
__global__ __launch_bounds__(256) void attn_bwd_reduce_kernel(AttnArgs a, const float* part_k,
                                                              const float* part_v) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (token, kv head, d / 4)
  const int64_t per_tok = (int64_t)a.hk * (kD / 4);
  if (i >= a.total * per_tok) return;
  const int64_t t = i / per_tok;
  const int kvh = (int)((i % per_tok) / (kD / 4));
  const int d = (int)(i % (kD / 4)) * 4;
  const int group = a.hq / a.hk;
  float4v sk = float4v{0.f, 0.f, 0.f, 0.f}, sv = float4v{0.f, 0.f, 0.f, 0.f};
  for (int hh = 0; hh < group; ++hh) {
    const int64_t off = ((int64_t)(kvh * group + hh) * a.total + t) * kD + d;
    sk += *reinterpret_cast<const float4v*>(part_k + off);
    sv += *reinterpret_cast<const float4v*>(part_v + off);
  }
  half4 ok, ov;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    ok[j] = f32_to_f16(sk[j] * a.scale);
    ov[j] = f32_to_f16(sv[j]);
  }
  *reinterpret_cast<half4*>(a.dk + t * a.dk_tok + (int64_t)kvh * a.dk_head + d) = ok;
  *reinterpret_cast<half4*>(a.dv + t * a.dv_tok + (int64_t)kvh * a.dv_head + d) = ov;
}

bool al8(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

int check_common(const char* fn, int rows, int max_len, int hq, int hk, int head_dim,
                 int64_t total, const int* cu) {
  SS_CHECK_ARG(rows >= 0 && max_len >= 0 && total >= 0, "%s: negative sizes", fn);
  SS_CHECK_ARG(head_dim == kD, "%s: head_dim %d unsupported (only %d)", fn, head_dim, kD);
  SS_CHECK_ARG(hq > 0 && hk > 0 && hq % hk == 0, "%s: hq=%d must be a positive multiple of hk=%d",
               fn, hq, hk);
  SS_CHECK_ARG(rows <= 65535 && hq <= 65535, "%s: rows / heads exceed the grid", fn);
  SS_CHECK_ARG(rows == 0 || cu, "%s: null cu_seqlens", fn);
  return SS_OK;
}

// Token / head strides (elements) of a tensor must keep every 16-byte load aligned.
bool strides_ok(const void* p, int64_t tok, int64_t head) {
  return p && al8(p) && tok % 8 == 0 && head % 8 == 0;
}

}  // namespace
}  // namespace ss

using namespace ss;

extern "C" int ss_attn_varlen_fwd(const void* q, int64_t q_tok, int64_t q_head, const void* k,
                                  int64_t k_tok, int64_t k_head, const void* v, int64_t v_tok,
                                  int64_t v_head, const int* cu_seqlens, int rows, int max_len,
                                  int64_t total, int hq, int hk, int head_dim, float scale,
                                  void* o, int64_t o_tok, int64_t o_head, float* lse2,
                                  void* stream) {
  const char* fn = "ss_attn_varlen_fwd";
  int rc = check_common(fn, rows, max_len, hq, hk, head_dim, total, cu_seqlens);
  if (rc) return rc;
  if (rows == 0 || max_len == 0) return SS_OK;
  SS_CHECK_ARG(strides_ok(q, q_tok, q_head) && strides_ok(k, k_tok, k_head) &&
                   strides_ok(v, v_tok, v_head) && strides_ok(o, o_tok, o_head) && lse2,
               "%s: q/k/v/o need 16-byte aligned bases and strides that are multiples of 8", fn);
  AttnArgs a{};
  a.q = (const half_t*)q; a.q_tok = q_tok; a.q_head = q_head;
  a.k = (const half_t*)k; a.k_tok = k_tok; a.k_head = k_head;
  a.v = (const half_t*)v; a.v_tok = v_tok; a.v_head = v_head;
  a.out = (half_t*)o; a.out_tok = o_tok; a.out_head = o_head;
  a.lse2 = lse2; a.cu = cu_seqlens; a.total = total; a.hq = hq; a.hk = hk; a.scale = scale;
  const dim3 grid((unsigned)cdiv(max_len, kBlk), (unsigned)hq, (unsigned)rows);
  hipLaunchKernelGGL(attn_fwd_kernel, grid, dim3(256), 0, (hipStream_t)stream, a);
  SS_CHECK_LAUNCH("attn_fwd_kernel");
  return SS_OK;
}

static size_t round256(size_t b) { return (b + 255) / 256 * 256; }

extern "C" size_t ss_attn_varlen_bwd_workspace_size(int hq, int hk, int64_t total) {
  if (hq <= 0 || hk <= 0 || total <= 0) return 0;
  const size_t delta = round256((size_t)hq * total * sizeof(float));
  const size_t part = hq == hk ? 0 : round256((size_t)hq * total * kD * sizeof(float));
  return delta + 2 * part;
}

extern "C" int ss_attn_varlen_bwd(const void* q, int64_t q_tok, int64_t q_head, const void* k,
                                  int64_t k_tok, int64_t k_head, const void* v, int64_t v_tok,
                                  int64_t v_head, const void* o, int64_t o_tok, int64_t o_head,
                                  const void* dout, int64_t do_tok, int64_t do_head,
                                  const float* lse2, const int* cu_seqlens, int rows, int max_len,
                                  int64_t total, int hq, int hk, int head_dim, float scale,
                                  void* dq, int64_t dq_tok, int64_t dq_head, void* dk,
                                  int64_t dk_tok, int64_t dk_head, void* dv, int64_t dv_tok,
                                  int64_t dv_head, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  const char* fn = "ss_attn_varlen_bwd";
  int rc = check_common(fn, rows, max_len, hq, hk, head_dim, total, cu_seqlens);
  if (rc) return rc;
  if (rows == 0 || max_len == 0) return SS_OK;
  SS_CHECK_ARG(strides_ok(q, q_tok, q_head) && strides_ok(k, k_tok, k_head) &&
                   strides_ok(v, v_tok, v_head) && strides_ok(o, o_tok, o_head) &&
                   strides_ok(dout, do_tok, do_head) && strides_ok(dq, dq_tok, dq_head) &&
                   strides_ok(dk, dk_tok, dk_head) && strides_ok(dv, dv_tok, dv_head) && lse2,
               "%s: q/k/v/o/dO/dq/dk/dv need 16-byte aligned bases and strides that are "
               "multiples of 8", fn);
  const size_t need = ss_attn_varlen_bwd_workspace_size(hq, hk, total);
  SS_CHECK_ARG(workspace && workspace_bytes >= need && al8(workspace),
               "%s: workspace of %zu bytes (16-byte aligned) needed, %zu given", fn, need,
               workspace_bytes);
  AttnArgs a{};
  a.q = (const half_t*)q; a.q_tok = q_tok; a.q_head = q_head;
  a.k = (const half_t*)k; a.k_tok = k_tok; a.k_head = k_head;
  a.v = (const half_t*)v; a.v_tok = v_tok; a.v_head = v_head;
  a.o = (const half_t*)o; a.o_tok = o_tok; a.o_head = o_head;
  a.dout = (const half_t*)dout; a.do_tok = do_tok; a.do_head = do_head;
  a.out = (half_t*)dq; a.out_tok = dq_tok; a.out_head = dq_head;
  a.dk = (half_t*)dk; a.dk_tok = dk_tok; a.dk_head = dk_head;
  a.dv = (half_t*)dv; a.dv_tok = dv_tok; a.dv_head = dv_head;
  a.lse2 = const_cast<float*>(lse2);
  a.delta = static_cast<float*>(workspace);
  a.cu = cu_seqlens; a.total = total; a.hq = hq; a.hk = hk; a.scale = scale;
  char* base = static_cast<char*>(workspace) + round256((size_t)hq * total * sizeof(float));
  const size_t part = round256((size_t)hq * total * kD * sizeof(float));
  float* part_k = hq == hk ? nullptr : reinterpret_cast<float*>(base);
  float* part_v = hq == hk ? nullptr : reinterpret_cast<float*>(base + part);
  const unsigned blocks = (unsigned)cdiv(max_len, kBlk);
  hipStream_t st = (hipStream_t)stream;
  hipLaunchKernelGGL(attn_bwd_dq_kernel, dim3(blocks, (unsigned)hq, (unsigned)rows), dim3(256), 0,
                     st, a);
  SS_CHECK_LAUNCH("attn_bwd_dq_kernel");
  hipLaunchKernelGGL(attn_bwd_dkdv_kernel, dim3(blocks, (unsigned)hq, (unsigned)rows), dim3(256),
                     0, st, a, part_k, part_v);
  SS_CHECK_LAUNCH("attn_bwd_dkdv_kernel");
  if (hq != hk) {
    const int64_t work = total * hk * (kD / 4);
    hipLaunchKernelGGL(attn_bwd_reduce_kernel, dim3((unsigned)cdiv(work, 256)), dim3(256), 0, st,
                       a, part_k, part_v);
    SS_CHECK_LAUNCH("attn_bwd_reduce_kernel");
  }
  return SS_OK;
}
