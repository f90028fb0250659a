// Fused residual add + Qwen2 RMSNorm, forward / backward / dgamma (A13-A14).
//
// Reference: solution/kernels/add_rmsnorm.py:1-24,37-81 and
// solution/kernels/rmsnorm.py:73-102.  Every cast follows the reference
// order; the file is built without contraction (enable_fp_fusion=False in
// the reference).
//
// Layout: one wave64 per row, four rows per 256-thread workgroup.  Lane l
// owns the 8-element chunks starting at (c*64 + l)*8, so each wave-wide
// access is 64 x 16 B contiguous for fp16 rows.  The row stays in registers
// (NCH chunks per lane, H <= 512*NCH), so the forward reads r and d once and
// writes s and y once: (2+2+2+2)*H + 4 bytes per fp16 row, the HBM floor.

#include "elementwise.h"

namespace ss {

struct F8 {
  float v[8];
};

// Load 8 consecutive logical elements starting at element offset `off`
// (contiguous), `valid` of which exist.
__device__ __forceinline__ F8 load8(const void* p, int dt, int64_t off, int valid, bool vec) {
  F8 r;
  if (vec && valid == 8) {
    if (dt == SS_F16) {
      union {
        uint4 u;
        half8 h;
      } t;
      t.u = *reinterpret_cast<const uint4*>(reinterpret_cast<const half_t*>(p) + off);
#pragma unroll
      for (int j = 0; j < 8; ++j) r.v[j] = (float)t.h[j];
    } else {
      const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + off);
      const float4 b =
          *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + off + 4);
      r.v[0] = a.x; r.v[1] = a.y; r.v[2] = a.z; r.v[3] = a.w;
      r.v[4] = b.x; r.v[5] = b.y; r.v[6] = b.z; r.v[7] = b.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) r.v[j] = j < valid ? ld_elem(p, dt, off + j) : 0.0f;
  }
  return r;
}

// Strided variant: element j at p[row_off + (col0 + j) * col_stride].
__device__ __forceinline__ F8 load8s(const void* p, int dt, int64_t row_off, int64_t col0,
                                     int64_t col_stride, int valid, bool vec) {
  if (col_stride == 1) return load8(p, dt, row_off + col0, valid, vec);
  F8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    r.v[j] = j < valid ? ld_elem(p, dt, row_off + (col0 + j) * col_stride) : 0.0f;
  return r;
}

__device__ __forceinline__ void store8(void* p, int dt, int64_t off, int valid, const float* v,
                                       bool vec) {
  if (vec && valid == 8) {
    if (dt == SS_F16) {
      union {
        uint4 u;
        half8 h;
      } t;
#pragma unroll
      for (int j = 0; j < 8; ++j) t.h[j] = f32_to_f16(v[j]);
      *reinterpret_cast<uint4*>(reinterpret_cast<half_t*>(p) + off) = t.u;
    } else {
      float* q = reinterpret_cast<float*>(p) + off;
      *reinterpret_cast<float4*>(q) = make_float4(v[0], v[1], v[2], v[3]);
      *reinterpret_cast<float4*>(q + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j < valid) st_elem(p, dt, off + j, v[j]);
  }
}

// d == nullptr: the standalone RMSNorm (s = r, read with row stride r_row,
// not stored when s == nullptr).
struct FwdArgs {
  const void* r; int rd;
  int64_t r_row;
  const void* d; int dd;
  const void* w; int wd; int64_t w_stride;
  void* s; int sd;
  void* y; int yd;
  float* rstd;
  int64_t rows, h;
  float eps;
  int vec;
};

__device__ __forceinline__ int chunk_valid(int64_t h, int64_t col0) {
  const int64_t left = h - col0;
  return left <= 0 ? 0 : (left >= 8 ? 8 : (int)left);
}

template <int NCH>
__global__ __launch_bounds__(256) void add_rmsnorm_fwd_kernel(FwdArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int64_t base = row * a.h;
  float sv[NCH][8];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t col0 = ((int64_t)c * 64 + lane) * 8;
    const int valid = chunk_valid(a.h, col0);
    if (valid > 0) {
      const F8 r = load8(a.r, a.rd, row * a.r_row + col0, valid, a.vec);
      if (a.d) {
        const F8 d = load8(a.d, a.dd, base + col0, valid, a.vec);
#pragma unroll
        for (int j = 0; j < 8; ++j) sv[c][j] = round_to(a.sd, r.v[j] + d.v[j]);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) sv[c][j] = r.v[j];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float sq = sv[c][j] * sv[c][j];
        ss += sq;
      }
      if (a.s) store8(a.s, a.sd, base + col0, valid, sv[c], a.vec);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) sv[c][j] = 0.0f;
    }
  }
  ss = wave_sum(ss);
  const float mean = ss / (float)a.h;
  const float rstd = rsqrtf(mean + a.eps);
  if (lane == 0) a.rstd[row] = rstd;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t col0 = ((int64_t)c * 64 + lane) * 8;
    const int valid = chunk_valid(a.h, col0);
    if (valid > 0) {
      const F8 w = load8s(a.w, a.wd, 0, col0, a.w_stride, valid, a.vec);
      float y[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float q = round_to(a.sd, sv[c][j] * rstd);
        y[j] = q * w.v[j];
      }
      store8(a.y, a.yd, base + col0, valid, y, a.vec);
    }
  }
}

// Fast forward: fp16 r (and d), s and y with 16-byte aligned rows, h = 512 NCH
// (every lane chunk full) and a contiguous gamma (fp16, or fp32 with WF32).  A
// lane issues all its loads -- its chunks of r and d and of gamma -- before the
// first use with no branch between them, so a row costs one memory round trip
// (the generic kernel's per-chunk dtype and length branches made each load wait
// for the previous one).  The arithmetic is the generic kernel's, in the same
// order, so the results are the same bits.
template <int NCH, bool HAS_D, bool WF32>
__global__ __launch_bounds__(256) void add_rmsnorm_fwd_fast_kernel(FwdArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int64_t base = row * a.h;
  const half_t* rp = reinterpret_cast<const half_t*>(a.r) + row * a.r_row;
  half8 rv[NCH], dv[NCH], wh[NCH];
  float4v wf[WF32 ? NCH : 1][2];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int col0 = (c * 64 + lane) * 8;
    rv[c] = *reinterpret_cast<const half8*>(rp + col0);
    if constexpr (HAS_D)
      dv[c] = *reinterpret_cast<const half8*>(reinterpret_cast<const half_t*>(a.d) + base + col0);
    if constexpr (WF32) {
      const float* wp = reinterpret_cast<const float*>(a.w) + col0;
      wf[c][0] = *reinterpret_cast<const float4v*>(wp);
      wf[c][1] = *reinterpret_cast<const float4v*>(wp + 4);
    } else {
      wh[c] = *reinterpret_cast<const half8*>(reinterpret_cast<const half_t*>(a.w) + col0);
    }
  }
  float sv[NCH][8];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if constexpr (HAS_D)
        sv[c][j] = (float)f32_to_f16((float)rv[c][j] + (float)dv[c][j]);
      else
        sv[c][j] = (float)rv[c][j];
      const float sq = sv[c][j] * sv[c][j];
      ss += sq;
    }
    if (HAS_D && a.s) {
      half8 o;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = f32_to_f16(sv[c][j]);
      *reinterpret_cast<half8*>(reinterpret_cast<half_t*>(a.s) + base + (c * 64 + lane) * 8) = o;
    }
  }
  ss = wave_sum(ss);
  const float mean = ss / (float)a.h;
  const float rstd = rsqrtf(mean + a.eps);
  if (lane == 0) a.rstd[row] = rstd;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    half8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float w;
      if constexpr (WF32)
        w = j < 4 ? wf[c][0][j] : wf[c][1][j - 4];
      else
        w = (float)wh[c][j];
      const float q = (float)f32_to_f16(sv[c][j] * rstd);
      o[j] = f32_to_f16(q * w);
    }
    *reinterpret_cast<half8*>(reinterpret_cast<half_t*>(a.y) + base + (c * 64 + lane) * 8) = o;
  }
}

struct BwdArgs {
  const void* s; int sd;
  const void* w; int wd; int64_t w_stride;
  const float* rstd;
  const void* gs; int gsd; int64_t gs_row, gs_col;
  const void* gy; int gyd; int64_t gy_row, gy_col;
  void* dr; int drd;
  void* dd; int ddd;
  int64_t rows, h;
  int vec;
  int vec_gs, vec_gy;
};

// One row of the backward, on one wave: ds into dr / dd (when present) and,
// with DG, gy * cast_s(s * rstd) added to the lane's column sums dg
// (rounded to fp16 first when half_products).
template <int NCH, bool DG>
__device__ __forceinline__ void bwd_row(const BwdArgs& a, int64_t row, int lane,
                                        float (&dg)[NCH][8], int half_products) {
  const int64_t base = row * a.h;
  float ds[NCH][8];
  if (a.gy) {
    const float rstd = a.rstd[row];
    float av[NCH][8];
    float dot = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int64_t col0 = ((int64_t)c * 64 + lane) * 8;
      const int valid = chunk_valid(a.h, col0);
      if (valid > 0) {
        const F8 s = load8(a.s, a.sd, base + col0, valid, a.vec);
        const F8 g = load8s(a.gy, a.gyd, row * a.gy_row, col0, a.gy_col, valid, a.vec_gy);
        const F8 w = load8s(a.w, a.wd, 0, col0, a.w_stride, valid, a.vec);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float av_ = s.v[j] * rstd;
          const float u = round_to(a.sd, g.v[j] * w.v[j]);
          av[c][j] = av_;
          ds[c][j] = u;
          const float ua = u * av_;
          dot += ua;
          if constexpr (DG) {
            float prod = g.v[j] * round_to(a.sd, av_);
            if (half_products) prod = round_to(SS_F16, prod);
            dg[c][j] += prod;
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          av[c][j] = 0.0f;
          ds[c][j] = 0.0f;
        }
      }
    }
    dot = wave_sum(dot);
    const float proj = dot / (float)a.h;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float t = av[c][j] * proj;
        const float diff = ds[c][j] - t;
        ds[c][j] = round_to(a.sd, rstd * diff);
      }
  } else {
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) ds[c][j] = 0.0f;
  }
  if (!a.dr && !a.dd) return;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t col0 = ((int64_t)c * 64 + lane) * 8;
    const int valid = chunk_valid(a.h, col0);
    if (valid <= 0) continue;
    float out[8];
    F8 gs;
    if (a.gs) gs = load8s(a.gs, a.gsd, row * a.gs_row, col0, a.gs_col, valid, a.vec_gs);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float v = ds[c][j];
      if (a.gs) v += gs.v[j];
      out[j] = round_to(a.sd, v);
    }
    if (a.dr) store8(a.dr, a.drd, base + col0, valid, out, a.vec);
    if (a.dd) store8(a.dd, a.ddd, base + col0, valid, out, a.vec);
  }
}

// Fast backward row: fp16 s, gy, gs, dr and dd, 16-byte aligned contiguous
// rows, h = 512 NCH and a contiguous gamma (fp16, or fp32 with WF32).  Every
// load of the row (s, gy, gamma and gs; without gs the lane re-reads s and
// ignores it) is issued before the first use with no branch between them.  The
// arithmetic is bwd_row's, in the same order.
template <int NCH, bool DG, bool WF32>
__device__ __forceinline__ void bwd_row_fast(const BwdArgs& a, int64_t row, int lane,
                                             float (&dg)[NCH][8], int half_products) {
  const int64_t base = row * a.h;
  const half_t* sp = reinterpret_cast<const half_t*>(a.s) + base;
  const half_t* gp = reinterpret_cast<const half_t*>(a.gy) + row * a.gy_row;
  const half_t* gsp = a.gs ? reinterpret_cast<const half_t*>(a.gs) + row * a.gs_row : sp;
  half8 sv[NCH], gv[NCH], gsv[NCH], wh[NCH];
  float4v wf[WF32 ? NCH : 1][2];
  const float rstd = a.rstd[row];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int col0 = (c * 64 + lane) * 8;
    sv[c] = *reinterpret_cast<const half8*>(sp + col0);
    gv[c] = *reinterpret_cast<const half8*>(gp + col0);
    gsv[c] = *reinterpret_cast<const half8*>(gsp + col0);
    if constexpr (WF32) {
      const float* wp = reinterpret_cast<const float*>(a.w) + col0;
      wf[c][0] = *reinterpret_cast<const float4v*>(wp);
      wf[c][1] = *reinterpret_cast<const float4v*>(wp + 4);
    } else {
      wh[c] = *reinterpret_cast<const half8*>(reinterpret_cast<const half_t*>(a.w) + col0);
    }
  }
  float av[NCH][8], ds[NCH][8];
  float dot = 0.0f;
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float w;
      if constexpr (WF32)
        w = j < 4 ? wf[c][0][j] : wf[c][1][j - 4];
      else
        w = (float)wh[c][j];
      const float g = (float)gv[c][j];
      const float av_ = (float)sv[c][j] * rstd;
      const float u = (float)f32_to_f16(g * w);
      av[c][j] = av_;
      ds[c][j] = u;
      const float ua = u * av_;
      dot += ua;
      if constexpr (DG) {
        float prod = g * (float)f32_to_f16(av_);
        if (half_products) prod = (float)f32_to_f16(prod);
        dg[c][j] += prod;
      }
    }
  dot = wave_sum(dot);
  const float proj = dot / (float)a.h;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    half8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float t = av[c][j] * proj;
      const float diff = ds[c][j] - t;
      float v = (float)f32_to_f16(rstd * diff);
      if (a.gs) v += (float)gsv[c][j];
      o[j] = f32_to_f16(v);
    }
    const int64_t off = base + (c * 64 + lane) * 8;
    if (a.dr) *reinterpret_cast<half8*>(reinterpret_cast<half_t*>(a.dr) + off) = o;
    if (a.dd) *reinterpret_cast<half8*>(reinterpret_cast<half_t*>(a.dd) + off) = o;
  }
}

// MODE: 0 the generic row, 1 the fast row with an fp16 gamma, 2 with an fp32 gamma.
template <int NCH, bool DG, int MODE>
__device__ __forceinline__ void bwd_row_any(const BwdArgs& a, int64_t row, int lane,
                                            float (&dg)[NCH][8], int half_products) {
  if constexpr (MODE == 0)
    bwd_row<NCH, DG>(a, row, lane, dg, half_products);
  else
    bwd_row_fast<NCH, DG, MODE == 2>(a, row, lane, dg, half_products);
}

template <int NCH, int MODE>
__global__ __launch_bounds__(256) void add_rmsnorm_bwd_kernel(BwdArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  float unused[NCH][8];
  bwd_row_any<NCH, false, MODE>(a, row, lane, unused, 0);
}

// Backward with the weight gradient in the same pass over s and gy: a
// workgroup of kDgWaves waves owns kDgWaves consecutive rows (one per wave,
// like the plain backward) and keeps fp32 column sums of gy * cast_s(s *
// rstd); the waves' sums are added through LDS in wave order into
// partial[workgroup][h].
constexpr int kDgWaves = 8;

template <int NCH, int MODE>
__global__ __launch_bounds__(kDgWaves * 64) void add_rmsnorm_bwd_dg_kernel(
    BwdArgs a, int half_products, float* __restrict__ partial) {
  extern __shared__ float s_dg[];  // [kDgWaves][h]
  const int lane = threadIdx.x & 63;
  const int k = threadIdx.x >> 6;
  float dg[NCH][8];
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) dg[c][j] = 0.0f;
  const int64_t row = (int64_t)blockIdx.x * kDgWaves + k;
  if (row < a.rows) bwd_row_any<NCH, true, MODE>(a, row, lane, dg, half_products);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t col0 = ((int64_t)c * 64 + lane) * 8;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (col0 + j < a.h) s_dg[k * a.h + col0 + j] = dg[c][j];
  }
  __syncthreads();
  for (int64_t col = threadIdx.x; col < a.h; col += kDgWaves * 64) {
    float v = s_dg[col];
#pragma unroll
    for (int q = 1; q < kDgWaves; ++q) v += s_dg[q * a.h + col];
    partial[(int64_t)blockIdx.x * a.h + col] = v;
  }
}

// dw[c] = sum over g = 0 .. groups-1 of partial[g][c]: 64 columns per
// workgroup of 16 waves; wave k takes g = k, k + 16, ... in batches of eight
// loads (in flight together) added in order, and the 16 wave sums are added
// in wave order.
__global__ __launch_bounds__(1024) void dgamma_groups_final_kernel(
    const float* __restrict__ partial, int64_t groups, int64_t h, void* dw, int dwd) {
  __shared__ float part[16][64];
  const int lane = threadIdx.x & 63;
  const int k = threadIdx.x >> 6;
  const int64_t c = (int64_t)blockIdx.x * 64 + lane;
  const int64_t cc = c < h ? c : h - 1;
  float acc = 0.0f;
  int64_t g = k;
  for (; g + 16 * 7 < groups; g += 16 * 8) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = partial[(g + 16 * j) * h + cc];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += v[j];
  }
  for (; g < groups; g += 16) acc += partial[g * h + cc];
  part[k][lane] = acc;
  __syncthreads();
  if (k == 0 && c < h) {
    float v = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; ++q) v += part[q][lane];
    st_elem(dw, dwd, c, v);
  }
}

// Partial rows of the fused backward + dgamma pass (one per workgroup).  One
// row per wave: a wave's rows would run one after the other (each a chain of
// loads, a wave reduction and stores), cutting the waves in flight more than
// it saves in partial rows (measured at T = 16384: 196 us with four rows per
// wave).
int64_t dgamma_groups(int64_t rows) { return rows > 0 ? cdiv(rows, kDgWaves) : 0; }

__global__ __launch_bounds__(256) void dgamma_partial_kernel(
    const void* __restrict__ s, int sd, const float* __restrict__ rstd, const void* __restrict__ gy,
    int gyd, int64_t gy_row, int64_t gy_col, int half_products, float* __restrict__ partial,
    int64_t rows, int64_t h) {
  const int64_t c = (int64_t)blockIdx.y * 256 + threadIdx.x;
  if (c >= h) return;
  const int64_t r0 = (int64_t)blockIdx.x * 32;
  const int64_t r1 = r0 + 32 < rows ? r0 + 32 : rows;
  float acc = 0.0f;
  for (int64_t r = r0; r < r1; ++r) {
    const float q = round_to(sd, ld_elem(s, sd, r * h + c) * rstd[r]);
    float prod = ld_elem(gy, gyd, r * gy_row + c * gy_col) * q;
    if (half_products) prod = round_to(SS_F16, prod);
    acc += prod;
  }
  partial[blockIdx.x * h + c] = acc;
}

__global__ __launch_bounds__(256) void dgamma_final_kernel(const float* __restrict__ partial,
                                                           int64_t groups, int64_t h, void* dw,
                                                           int dwd) {
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= h) return;
  float acc = 0.0f;
  for (int64_t g = 0; g < groups; ++g) acc += partial[g * h + c];
  st_elem(dw, dwd, c, acc);
}

constexpr int kMaxChunks = 16;  // h <= 8192

static bool al16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace ss

using namespace ss;

#define SS_ROW_KERNEL_SWITCH(KERNEL, NCH, ARGS, GRID, STREAM)                                   \
  switch (NCH) {                                                                                \
    case 1: hipLaunchKernelGGL(KERNEL<1>, GRID, dim3(256), 0, STREAM, ARGS); break;             \
    case 2: hipLaunchKernelGGL(KERNEL<2>, GRID, dim3(256), 0, STREAM, ARGS); break;             \
    case 3: hipLaunchKernelGGL(KERNEL<3>, GRID, dim3(256), 0, STREAM, ARGS); break;             \
    case 4: hipLaunchKernelGGL(KERNEL<4>, GRID, dim3(256), 0, STREAM, ARGS); break;             \
    case 5: hipLaunchKernelGGL(KERNEL<5>, GRID, dim3(256), 0, STREAM, ARGS); break;             \
    case 6: hipLaunchKernelGGL(KERNEL<6>, GRID, dim3(256), 0, STREAM, ARGS); break;             \
    case 7: hipLaunchKernelGGL(KERNEL<7>, GRID, dim3(256), 0, STREAM, ARGS); break;             \
    case 8: hipLaunchKernelGGL(KERNEL<8>, GRID, dim3(256), 0, STREAM, ARGS); break;             \
    default: hipLaunchKernelGGL(KERNEL<16>, GRID, dim3(256), 0, STREAM, ARGS); break;           \
  }

// The fast forward applies to fp16 rows (r, d, s, y), 16-byte aligned, with h a
// multiple of 512 up to 4096 and a contiguous fp16 or fp32 gamma.
static bool fwd_fast_ok(const FwdArgs& a, bool has_d) {
  const bool rows16 = a.rd == SS_F16 && a.sd == SS_F16 && a.yd == SS_F16 &&
                      (!has_d || a.dd == SS_F16);
  return rows16 && a.vec && a.w_stride == 1 && a.h % 512 == 0 && a.h <= 4096;
}

template <bool HAS_D, bool WF32>
static void launch_fwd_fast(const FwdArgs& a, dim3 grid, hipStream_t st) {
  switch (a.h / 512) {
#define SS_FAST_CASE(N)                                                                        \
  case N:                                                                                      \
    hipLaunchKernelGGL((add_rmsnorm_fwd_fast_kernel<N, HAS_D, WF32>), grid, dim3(256), 0, st,  \
                       a);                                                                     \
    break;
    SS_FAST_CASE(1) SS_FAST_CASE(2) SS_FAST_CASE(3) SS_FAST_CASE(4) SS_FAST_CASE(5)
    SS_FAST_CASE(6) SS_FAST_CASE(7) SS_FAST_CASE(8)
#undef SS_FAST_CASE
  }
}

static void launch_fwd(const FwdArgs& a, bool has_d, dim3 grid, hipStream_t st) {
  if (fwd_fast_ok(a, has_d)) {
    if (has_d)
      a.wd == SS_F32 ? launch_fwd_fast<true, true>(a, grid, st)
                     : launch_fwd_fast<true, false>(a, grid, st);
    else
      a.wd == SS_F32 ? launch_fwd_fast<false, true>(a, grid, st)
                     : launch_fwd_fast<false, false>(a, grid, st);
    return;
  }
  const int nch = (int)cdiv(a.h, 512);
  SS_ROW_KERNEL_SWITCH(add_rmsnorm_fwd_kernel, nch, a, grid, st);
}

// Backward row mode (bwd_row_any): the fast row for fp16 s, gy, gs, dr and dd in
// 16-byte aligned contiguous rows, h a multiple of 512 up to 4096 and a
// contiguous gamma; else the generic row.
static int bwd_mode(const BwdArgs& a) {
  const bool f16 = a.sd == SS_F16 && a.gy && a.gyd == SS_F16 && a.vec_gy &&
                   (!a.gs || (a.gsd == SS_F16 && a.vec_gs)) && (!a.dr || a.drd == SS_F16) &&
                   (!a.dd || a.ddd == SS_F16);
  if (!f16 || !a.vec || a.w_stride != 1 || a.h % 512 != 0 || a.h > 4096) return 0;
  return a.wd == SS_F32 ? 2 : 1;
}

template <int MODE>
static void launch_bwd_mode(const BwdArgs& a, dim3 grid, hipStream_t st) {
  switch (cdiv(a.h, 512)) {
#define SS_BWD_CASE(N)                                                                         \
  case N:                                                                                      \
    hipLaunchKernelGGL((add_rmsnorm_bwd_kernel<N, MODE>), grid, dim3(256), 0, st, a);          \
    break;
    SS_BWD_CASE(1) SS_BWD_CASE(2) SS_BWD_CASE(3) SS_BWD_CASE(4) SS_BWD_CASE(5)
    SS_BWD_CASE(6) SS_BWD_CASE(7) SS_BWD_CASE(8)
#undef SS_BWD_CASE
    default:
      if constexpr (MODE == 0)
        hipLaunchKernelGGL((add_rmsnorm_bwd_kernel<16, 0>), grid, dim3(256), 0, st, a);
      break;
  }
}

template <int MODE>
static void launch_dg_mode(const BwdArgs& a, int half_products, float* partial, dim3 grid,
                           size_t lds, hipStream_t st) {
  const dim3 block(kDgWaves * 64);
  switch (cdiv(a.h, 512)) {
#define SS_DG_CASE(N)                                                                          \
  case N:                                                                                      \
    hipLaunchKernelGGL((add_rmsnorm_bwd_dg_kernel<N, MODE>), grid, block, lds, st, a,          \
                       half_products, partial);                                                \
    break;
    SS_DG_CASE(1) SS_DG_CASE(2) SS_DG_CASE(3) SS_DG_CASE(4) SS_DG_CASE(5) SS_DG_CASE(6)
    SS_DG_CASE(7) SS_DG_CASE(8)
#undef SS_DG_CASE
    default:
      if constexpr (MODE == 0)
        hipLaunchKernelGGL((add_rmsnorm_bwd_dg_kernel<16, 0>), grid, block, lds, st, a,
                           half_products, partial);
      break;
  }
}

extern "C" int ss_add_rmsnorm_fwd(const void* r, int r_dtype, const void* d, int d_dtype,
                                  const void* w, int w_dtype, int64_t w_stride, void* s,
                                  int s_dtype, void* y, int y_dtype, float* rstd, int64_t rows,
                                  int64_t h, float eps, void* stream) {
  const char* fn = "ss_add_rmsnorm_fwd";
  SS_CHECK_ARG(rows >= 0 && h > 0, "%s: need rows >= 0 and h > 0", fn);
  SS_CHECK_ARG(valid_dtype(r_dtype) && valid_dtype(d_dtype) && valid_dtype(w_dtype) &&
                   valid_dtype(s_dtype) && valid_dtype(y_dtype),
               "%s: dtype must be SS_F16 or SS_F32", fn);
  SS_CHECK_ARG(s_dtype == promote(r_dtype, d_dtype), "%s: s dtype must be promote(r, d)", fn);
  SS_CHECK_ARG(y_dtype == promote(s_dtype, w_dtype) || y_dtype == SS_F16,
               "%s: y dtype must be promote(s, w) or fp16", fn);
  SS_CHECK_ARG(eps >= 0.0f, "%s: eps must be >= 0", fn);
  if (h > 512 * kMaxChunks) {
    ss::set_error("%s: h=%lld exceeds the register-resident row limit %d", fn, (long long)h,
                  512 * kMaxChunks);
    return SS_ERR_UNSUPPORTED;
  }
  if (rows == 0) return SS_OK;
  SS_CHECK_ARG(r && d && w && s && y && rstd, "%s: null pointer", fn);
  FwdArgs a{r, r_dtype, h, d, d_dtype, w, w_dtype, w_stride, s, s_dtype, y, y_dtype, rstd, rows,
            h, eps, 0};
  a.vec = (h % 8 == 0) && al16(r) && al16(d) && al16(s) && al16(y) && (w_stride != 1 || al16(w));
  const dim3 grid((unsigned)cdiv(rows, 4));
  launch_fwd(a, true, grid, (hipStream_t)stream);
  SS_CHECK_LAUNCH("add_rmsnorm_fwd_kernel");
  return SS_OK;
}

extern "C" int ss_rmsnorm_fwd(const void* x, int x_dtype, int64_t x_row, const void* w,
                              int w_dtype, int64_t w_stride, void* y, int y_dtype, float* rstd,
                              int64_t rows, int64_t h, float eps, void* stream) {
  const char* fn = "ss_rmsnorm_fwd";
  SS_CHECK_ARG(rows >= 0 && h > 0, "%s: need rows >= 0 and h > 0", fn);
  SS_CHECK_ARG(valid_dtype(x_dtype) && valid_dtype(w_dtype) && valid_dtype(y_dtype),
               "%s: dtype must be SS_F16 or SS_F32", fn);
  SS_CHECK_ARG(y_dtype == promote(x_dtype, w_dtype) || y_dtype == SS_F16,
               "%s: y dtype must be promote(x, w) or fp16", fn);
  SS_CHECK_ARG(eps >= 0.0f, "%s: eps must be >= 0", fn);
  SS_CHECK_ARG(x_row >= h, "%s: row stride %lld < h", fn, (long long)x_row);
  if (h > 512 * kMaxChunks) {
    ss::set_error("%s: h=%lld exceeds the register-resident row limit %d", fn, (long long)h,
                  512 * kMaxChunks);
    return SS_ERR_UNSUPPORTED;
  }
  if (rows == 0) return SS_OK;
  SS_CHECK_ARG(x && w && y && rstd, "%s: null pointer", fn);
  FwdArgs a{x, x_dtype, x_row, nullptr, x_dtype, w, w_dtype, w_stride, nullptr, x_dtype, y,
            y_dtype, rstd, rows, h, eps, 0};
  const int64_t xs = x_dtype == SS_F16 ? 2 : 4;
  a.vec = (h % 8 == 0) && al16(x) && (x_row * xs) % 16 == 0 && al16(y) &&
          (w_stride != 1 || al16(w));
  const dim3 grid((unsigned)cdiv(rows, 4));
  launch_fwd(a, false, grid, (hipStream_t)stream);
  SS_CHECK_LAUNCH("add_rmsnorm_fwd_kernel");
  return SS_OK;
}

extern "C" int ss_add_rmsnorm_bwd(const void* s, int s_dtype, const void* w, int w_dtype,
                                  int64_t w_stride, const float* rstd, const void* gs,
                                  int gs_dtype, int64_t gs_row, int64_t gs_col, const void* gy,
                                  int gy_dtype, int64_t gy_row, int64_t gy_col, void* dr,
                                  int dr_dtype, void* dd, int dd_dtype, int64_t rows, int64_t h,
                                  void* stream) {
  const char* fn = "ss_add_rmsnorm_bwd";
  SS_CHECK_ARG(rows >= 0 && h > 0, "%s: need rows >= 0 and h > 0", fn);
  SS_CHECK_ARG(valid_dtype(s_dtype) && valid_dtype(w_dtype), "%s: bad s/w dtype", fn);
  SS_CHECK_ARG(!gs || valid_dtype(gs_dtype), "%s: bad gs dtype", fn);
  SS_CHECK_ARG(!gy || valid_dtype(gy_dtype), "%s: bad gy dtype", fn);
  SS_CHECK_ARG(!dr || valid_dtype(dr_dtype), "%s: bad dr dtype", fn);
  SS_CHECK_ARG(!dd || valid_dtype(dd_dtype), "%s: bad dd dtype", fn);
  if (h > 512 * kMaxChunks) {
    ss::set_error("%s: h=%lld exceeds the register-resident row limit %d", fn, (long long)h,
                  512 * kMaxChunks);
    return SS_ERR_UNSUPPORTED;
  }
  if (rows == 0 || (!dr && !dd)) return SS_OK;
  SS_CHECK_ARG(s && w && rstd, "%s: null pointer", fn);
  BwdArgs a{s, s_dtype, w, w_dtype, w_stride, rstd, gs, gs_dtype, gs_row, gs_col, gy, gy_dtype,
            gy_row, gy_col, dr, dr_dtype, dd, dd_dtype, rows, h, 0, 0, 0};
  a.vec = (h % 8 == 0) && al16(s) && (!dr || al16(dr)) && (!dd || al16(dd)) &&
          (w_stride != 1 || al16(w));
  a.vec_gs = gs && gs_col == 1 && gs_row % 8 == 0 && al16(gs) && a.vec;
  a.vec_gy = gy && gy_col == 1 && gy_row % 8 == 0 && al16(gy) && a.vec;
  const dim3 grid((unsigned)cdiv(rows, 4));
  hipStream_t st = (hipStream_t)stream;
  switch (bwd_mode(a)) {
    case 1: launch_bwd_mode<1>(a, grid, st); break;
    case 2: launch_bwd_mode<2>(a, grid, st); break;
    default: launch_bwd_mode<0>(a, grid, st); break;
  }
  SS_CHECK_LAUNCH("add_rmsnorm_bwd_kernel");
  return SS_OK;
}

extern "C" int64_t ss_add_rmsnorm_dgamma_waves(int64_t rows) { return ss::dgamma_groups(rows); }

extern "C" int ss_add_rmsnorm_bwd_dgamma(const void* s, int s_dtype, const void* w, int w_dtype,
                                         int64_t w_stride, const float* rstd, const void* gs,
                                         int gs_dtype, int64_t gs_row, int64_t gs_col,
                                         const void* gy, int gy_dtype, int64_t gy_row,
                                         int64_t gy_col, void* dr, int dr_dtype, void* dd,
                                         int dd_dtype, int half_products, float* partial,
                                         void* dw, int dw_dtype, int64_t rows, int64_t h,
                                         void* stream) {
  const char* fn = "ss_add_rmsnorm_bwd_dgamma";
  SS_CHECK_ARG(rows >= 0 && h > 0, "%s: need rows >= 0 and h > 0", fn);
  SS_CHECK_ARG(valid_dtype(s_dtype) && valid_dtype(w_dtype) && valid_dtype(dw_dtype),
               "%s: bad s/w/dw dtype", fn);
  SS_CHECK_ARG(!gs || valid_dtype(gs_dtype), "%s: bad gs dtype", fn);
  SS_CHECK_ARG(!gy || valid_dtype(gy_dtype), "%s: bad gy dtype", fn);
  SS_CHECK_ARG(!dr || valid_dtype(dr_dtype), "%s: bad dr dtype", fn);
  SS_CHECK_ARG(!dd || valid_dtype(dd_dtype), "%s: bad dd dtype", fn);
  if (h > 512 * kMaxChunks) {
    ss::set_error("%s: h=%lld exceeds the register-resident row limit %d", fn, (long long)h,
                  512 * kMaxChunks);
    return SS_ERR_UNSUPPORTED;
  }
  SS_CHECK_ARG(dw, "%s: null dw", fn);
  hipStream_t st = (hipStream_t)stream;
  if ((size_t)kDgWaves * h * sizeof(float) > 160 * 1024) {
    // Rows too wide for the LDS combine: the backward, then the two-stage
    // dgamma (ceil(rows / 32) partial rows, within the partial scratch).
    const int rc = ss_add_rmsnorm_bwd(s, s_dtype, w, w_dtype, w_stride, rstd, gs, gs_dtype, gs_row,
                                      gs_col, gy, gy_dtype, gy_row, gy_col, dr, dr_dtype, dd,
                                      dd_dtype, rows, h, stream);
    if (rc) return rc;
    if (!gy) {
      hipLaunchKernelGGL(dgamma_final_kernel, dim3((unsigned)cdiv(h, 256)), dim3(256), 0, st,
                         partial, (int64_t)0, h, dw, dw_dtype);
      SS_CHECK_LAUNCH("dgamma_final_kernel");
      return SS_OK;
    }
    return ss_rmsnorm_dgamma(s, s_dtype, rstd, gy, gy_dtype, gy_row, gy_col, half_products,
                             partial, dw, dw_dtype, rows, h, stream);
  }
  const int64_t groups = dgamma_groups(rows);
  if (rows > 0) {
    SS_CHECK_ARG(s && w && rstd && partial, "%s: null pointer", fn);
    BwdArgs a{s, s_dtype, w, w_dtype, w_stride, rstd, gs, gs_dtype, gs_row, gs_col, gy,
              gy_dtype, gy_row, gy_col, dr, dr_dtype, dd, dd_dtype, rows, h, 0, 0, 0};
    a.vec = (h % 8 == 0) && al16(s) && (!dr || al16(dr)) && (!dd || al16(dd)) &&
            (w_stride != 1 || al16(w));
    a.vec_gs = gs && gs_col == 1 && gs_row % 8 == 0 && al16(gs) && a.vec;
    a.vec_gy = gy && gy_col == 1 && gy_row % 8 == 0 && al16(gy) && a.vec;
    const size_t lds = (size_t)kDgWaves * h * sizeof(float);
    const dim3 grid((unsigned)groups);
    switch (bwd_mode(a)) {
      case 1: launch_dg_mode<1>(a, half_products, partial, grid, lds, st); break;
      case 2: launch_dg_mode<2>(a, half_products, partial, grid, lds, st); break;
      default: launch_dg_mode<0>(a, half_products, partial, grid, lds, st); break;
    }
    SS_CHECK_LAUNCH("add_rmsnorm_bwd_dg_kernel");
  }
  hipLaunchKernelGGL(dgamma_groups_final_kernel, dim3((unsigned)cdiv(h, 64)), dim3(1024), 0, st,
                     partial, groups, h, dw, dw_dtype);
  SS_CHECK_LAUNCH("dgamma_groups_final_kernel");
  return SS_OK;
}

extern "C" int ss_rmsnorm_dgamma(const void* s, int s_dtype, const float* rstd, const void* gy,
                                 int gy_dtype, int64_t gy_row, int64_t gy_col, int half_products,
                                 float* partial, void* dw, int dw_dtype, int64_t rows, int64_t h,
                                 void* stream) {
  const char* fn = "ss_rmsnorm_dgamma";
  SS_CHECK_ARG(rows >= 0 && h > 0, "%s: need rows >= 0 and h > 0", fn);
  SS_CHECK_ARG(valid_dtype(s_dtype) && valid_dtype(gy_dtype) && valid_dtype(dw_dtype),
               "%s: dtype must be SS_F16 or SS_F32", fn);
  SS_CHECK_ARG(dw, "%s: null dw", fn);
  const int64_t groups = cdiv(rows, 32);
  hipStream_t st = (hipStream_t)stream;
  if (groups > 0) {
    SS_CHECK_ARG(s && rstd && gy && partial, "%s: null pointer", fn);
    hipLaunchKernelGGL(dgamma_partial_kernel, dim3((unsigned)groups, (unsigned)cdiv(h, 256)),
                       dim3(256), 0, st, s, s_dtype, rstd, gy, gy_dtype, gy_row, gy_col,
                       half_products, partial, rows, h);
    SS_CHECK_LAUNCH("dgamma_partial_kernel");
  }
  hipLaunchKernelGGL(dgamma_final_kernel, dim3((unsigned)cdiv(h, 256)), dim3(256), 0, st,
                     partial, groups, h, dw, dw_dtype);
  SS_CHECK_LAUNCH("dgamma_final_kernel");
  return SS_OK;
}
