// Vocabulary-chunk kernels of the fused linear cross-entropy (A17-A18).
//
// Reference: solution/kernels/cross_entropy.py:1-43 (semantics), :51-89
// (statistics), :92-105 (outputs), :108-122 (derivative), :193-210 (dX
// rescale and scatter).  The logits of a chunk are fp16 (the reference
// rounds logits before any statistic); all statistics are fp32.
//
// ce_stats: one 256-thread workgroup per row; pass 1 finds the chunk max and
// its first index, pass 2 accumulates sum exp(z - m) and sum exp(z - m) * z
// against the merged running max.  Lanes read 8 consecutive fp16 logits
// (16 B), so a wave reads 1 KiB contiguous per access.  Chunks up to 8192 wide
// are read once, all of a lane's loads issued together into registers, and both
// passes run from there (one memory round trip per row instead of one per
// 2048 logits and pass); wider chunks re-read the row in pass 2.  Both forms
// add in the same order, so they give the same bits.

#include "elementwise.h"

namespace ss {

struct MaxArg {
  float m;
  int64_t a;
};

__device__ __forceinline__ MaxArg better(MaxArg x, MaxArg y) {
  // Larger value wins; equal values keep the lower vocabulary index.
  if (y.m > x.m || (y.m == x.m && y.a < x.a)) return y;
  return x;
}

__device__ __forceinline__ MaxArg wave_maxarg(MaxArg v) {
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) {
    MaxArg o;
    o.m = __shfl_xor(v.m, s, kWave);
    o.a = __shfl_xor(v.a, s, kWave);
    v = better(v, o);
  }
  return v;
}

constexpr int64_t kNoIndex = 0x7fffffffffffffffLL;

__device__ __forceinline__ void load_logits8(const half_t* __restrict__ row, int64_t c,
                                             int64_t width, bool vec, float* v) {
  if (vec && c + 8 <= width) {
    union {
      uint4 u;
      half8 h;
    } t;
    t.u = *reinterpret_cast<const uint4*>(row + c);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (float)t.h[j];
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = c + j < width ? (float)row[c + j] : -INFINITY;
  }
}

constexpr int kStatsHeld = 4;  // 2048-logit steps a lane holds in registers (width <= 8192)

template <bool HELD>
__global__ __launch_bounds__(256) void ce_stats_kernel(const half_t* __restrict__ z, int64_t ldz,
                                                       const int64_t* __restrict__ targets,
                                                       float* __restrict__ state,
                                                       int64_t* __restrict__ best, int64_t width,
                                                       int64_t start, int64_t ignore, int first,
                                                       int vec) {
  __shared__ MaxArg s_ma[4];
  __shared__ float s_sum[4][3];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const half_t* zr = z + row * ldz;
  // The lane's steps, logits c = 8 tid + 2048 i .. + 7 for c < width, in order.
  // HELD: all of them loaded up front (load_logits8 touches no memory at or
  // past `width`, so the loads of absent steps read nothing).
  float held[HELD ? kStatsHeld : 1][8];
  if constexpr (HELD) {
#pragma unroll
    for (int i = 0; i < kStatsHeld; ++i)
      load_logits8(zr, (int64_t)tid * 8 + 2048 * i, width, vec, held[i]);
  }
  // The row's running state, read before the passes so its latency overlaps them.
  float old_m = -INFINITY, old_s = 0.0f, old_t = 0.0f, tz = 0.0f;
  int64_t old_arg = kNoIndex;
  if (!first) {
    old_m = state[row * 4 + 0];
    old_s = state[row * 4 + 1];
    old_t = state[row * 4 + 2];
    tz = state[row * 4 + 3];
    old_arg = best[row];
  }
  const int64_t tgt = targets[row];
  auto each_step = [&](auto&& f) {
    if constexpr (HELD) {
#pragma unroll
      for (int i = 0; i < kStatsHeld; ++i) {
        const int64_t c = (int64_t)tid * 8 + 2048 * i;
        if (c < width) f(c, held[i]);
      }
    } else {
      for (int64_t c = (int64_t)tid * 8; c < width; c += 2048) {
        float v[8];
        load_logits8(zr, c, width, vec, v);
        f(c, v);
      }
    }
  };

  MaxArg ma{-INFINITY, kNoIndex};
  each_step([&](int64_t c, const float* v) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (c + j < width && v[j] > ma.m) {
        ma.m = v[j];
        ma.a = start + c + j;
      }
    }
  });
  ma = wave_maxarg(ma);
  if (lane == 0) s_ma[wave] = ma;
  __syncthreads();
  MaxArg tile = s_ma[0];
#pragma unroll
  for (int w = 1; w < 4; ++w) tile = better(tile, s_ma[w]);
  const float new_m = fmaxf(old_m, tile.m);

  float sp = 0.0f, spz = 0.0f, found = 0.0f;
  each_step([&](int64_t c, const float* v) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (c + j < width) {
        const float p = __expf(v[j] - new_m);
        sp += p;
        const float pz = p * v[j];
        spz += pz;
        if (tgt != ignore && tgt == start + c + j) found += v[j];
      }
    }
  });
  sp = wave_sum(sp);
  spz = wave_sum(spz);
  found = wave_sum(found);
  if (lane == 0) {
    s_sum[wave][0] = sp;
    s_sum[wave][1] = spz;
    s_sum[wave][2] = found;
  }
  __syncthreads();
  if (tid == 0) {
    float a = 0.f, b = 0.f, f = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      a += s_sum[w][0];
      b += s_sum[w][1];
      f += s_sum[w][2];
    }
    const float rescale = __expf(old_m - new_m);
    const float total_s = old_s * rescale + a;
    const float total_t = old_t * rescale + b;
    int64_t arg;
    if (tile.m > old_m)
      arg = tile.a;
    else if (tile.m == old_m)
      arg = old_arg < tile.a ? old_arg : tile.a;
    else
      arg = old_arg;
    state[row * 4 + 0] = new_m;
    state[row * 4 + 1] = total_s;
    state[row * 4 + 2] = total_t;
    state[row * 4 + 3] = tz + f;
    best[row] = arg;
  }
}

__global__ __launch_bounds__(256) void ce_outputs_kernel(const float* __restrict__ state,
                                                         const int64_t* __restrict__ targets,
                                                         float* __restrict__ loss,
                                                         float* __restrict__ entropy,
                                                         float* __restrict__ lse, int64_t n,
                                                         int64_t ignore) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= n) return;
  const float m = state[r * 4 + 0];
  const float s = state[r * 4 + 1];
  const float t = state[r * 4 + 2];
  const float zt = state[r * 4 + 3];
  const float l = m + __logf(s);
  lse[r] = l;
  entropy[r] = l - t / s;
  loss[r] = targets[r] != ignore ? l - zt : 0.0f;
}

__global__ __launch_bounds__(256) void ce_derivative_kernel(
    const half_t* __restrict__ z, int64_t ldz, const int64_t* __restrict__ z_rows,
    const int64_t* __restrict__ targets,
    const float* __restrict__ lse, const float* __restrict__ grad, half_t* __restrict__ dz,
    half_t* __restrict__ dzg, const float* __restrict__ global_gain_p, int64_t width,
    int64_t start, int64_t ignore, int vec) {
  const int64_t row = blockIdx.x;
  const int64_t c = ((int64_t)blockIdx.y * 256 + threadIdx.x) * 8;
  if (c >= width) return;
  const int64_t tgt = targets[row];
  const bool valid = tgt != ignore;
  const float g = valid ? grad[row] : 0.0f;
  const float gain = fmaxf(fabsf(g), 1e-30f) / 1024.0f;
  const float global_gain = dzg ? *global_gain_p : 1.0f;
  const float l = lse[row];
  float v[8];
  load_logits8(z + (z_rows ? z_rows[row] : row) * ldz, c, width, vec, v);
  union {
    uint4 u;
    half8 h;
  } o, og;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float d = 0.0f;
    if (valid && c + j < width) {
      const float p = __expf(v[j] - l);
      const float onehot = (start + c + j == tgt) ? 1.0f : 0.0f;
      d = (p - onehot) * g;
    }
    o.h[j] = f32_to_f16(d / gain);
    og.h[j] = f32_to_f16(d / global_gain);
  }
  half_t* out = dz + row * width + c;
  half_t* outg = dzg ? dzg + row * width + c : nullptr;
  if (vec && c + 8 <= width) {
    *reinterpret_cast<uint4*>(out) = o.u;
    if (outg) *reinterpret_cast<uint4*>(outg) = og.u;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (c + j < width) {
        out[j] = o.h[j];
        if (outg) outg[j] = og.h[j];
      }
  }
}

__global__ __launch_bounds__(256) void ce_finalize_kernel(const float* __restrict__ acc,
                                                          const float* __restrict__ grad,
                                                          const int32_t* __restrict__ inverse,
                                                          void* __restrict__ out, int od,
                                                          int64_t h, int64_t valid_n) {
  const int64_t r = blockIdx.x;
  const int64_t c = (int64_t)blockIdx.y * 256 + threadIdx.x;
  if (c >= h) return;
  const int32_t j = inverse[r];
  float v = 0.0f;
  if (j >= 0 && j < valid_n) {
    const float gain = fmaxf(fabsf(grad[r]), 1e-30f) / 1024.0f;
    v = acc[(int64_t)j * h + c] * gain;
  }
  st_elem(out, od, r * h + c, v);
}

static bool al16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace ss

using namespace ss;

extern "C" int ss_ce_stats(const uint16_t* z, int64_t ldz, const int64_t* targets, float* state,
                           int64_t* best, int64_t n, int64_t width, int64_t start,
                           int64_t ignore_index, int first, void* stream) {
  SS_CHECK_ARG(n >= 0 && width > 0 && start >= 0 && ldz >= width, "ss_ce_stats: bad sizes");
  if (n == 0) return SS_OK;
  SS_CHECK_ARG(z && targets && state && best, "ss_ce_stats: null pointer");
  const int vec = al16(z) && ldz % 8 == 0;
  if (width <= 2048 * kStatsHeld)
    hipLaunchKernelGGL(ce_stats_kernel<true>, dim3((unsigned)n), dim3(256), 0,
                       (hipStream_t)stream, reinterpret_cast<const half_t*>(z), ldz, targets,
                       state, best, width, start, ignore_index, first ? 1 : 0, vec);
  else
    hipLaunchKernelGGL(ce_stats_kernel<false>, dim3((unsigned)n), dim3(256), 0,
                       (hipStream_t)stream, reinterpret_cast<const half_t*>(z), ldz, targets,
                       state, best, width, start, ignore_index, first ? 1 : 0, vec);
  SS_CHECK_LAUNCH("ce_stats_kernel");
  return SS_OK;
}

extern "C" int ss_ce_outputs(const float* state, const int64_t* targets, float* loss,
                             float* entropy, float* lse, int64_t n, int64_t ignore_index,
                             void* stream) {
  SS_CHECK_ARG(n >= 0, "ss_ce_outputs: negative n");
  if (n == 0) return SS_OK;
  SS_CHECK_ARG(state && targets && loss && entropy && lse, "ss_ce_outputs: null pointer");
  hipLaunchKernelGGL(ce_outputs_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0,
                     (hipStream_t)stream, state, targets, loss, entropy, lse, n, ignore_index);
  SS_CHECK_LAUNCH("ce_outputs_kernel");
  return SS_OK;
}

extern "C" int ss_ce_derivative(const uint16_t* z, int64_t ldz, const int64_t* z_rows,
                                const int64_t* targets, const float* lse, const float* grad,
                                uint16_t* dz, uint16_t* dz_global, const float* global_gain,
                                int64_t n, int64_t width, int64_t start, int64_t ignore_index,
                                void* stream) {
  SS_CHECK_ARG(n >= 0 && width > 0 && ldz >= width, "ss_ce_derivative: bad sizes");
  SS_CHECK_ARG(!dz_global || global_gain, "ss_ce_derivative: dz_global needs global_gain");
  if (n == 0) return SS_OK;
  SS_CHECK_ARG(z && targets && lse && grad && dz, "ss_ce_derivative: null pointer");
  const int vec = al16(z) && ldz % 8 == 0 && al16(dz) && width % 8 == 0 &&
                  (!dz_global || al16(dz_global));
  SS_CHECK_ARG(cdiv(width, 256 * 8) < 65536, "ss_ce_derivative: width too large");
  const dim3 grid((unsigned)n, (unsigned)cdiv(width, 256 * 8));
  hipLaunchKernelGGL(ce_derivative_kernel, grid, dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<const half_t*>(z), ldz, z_rows, targets, lse, grad,
                     reinterpret_cast<half_t*>(dz), reinterpret_cast<half_t*>(dz_global),
                     global_gain, width, start, ignore_index, vec);
  SS_CHECK_LAUNCH("ce_derivative_kernel");
  return SS_OK;
}

extern "C" int ss_ce_finalize_dx(const float* acc, int64_t valid_n, const float* grad,
                                 const int32_t* inverse, void* out, int out_dtype, int64_t n,
                                 int64_t h, void* stream) {
  SS_CHECK_ARG(n >= 0 && h > 0 && valid_n >= 0, "ss_ce_finalize_dx: bad sizes");
  SS_CHECK_ARG(valid_dtype(out_dtype), "ss_ce_finalize_dx: bad out dtype");
  if (n == 0) return SS_OK;
  SS_CHECK_ARG(grad && inverse && out && (valid_n == 0 || acc), "ss_ce_finalize_dx: null pointer");
  SS_CHECK_ARG(cdiv(h, 256) < 65536, "ss_ce_finalize_dx: h too large");
  const dim3 grid((unsigned)n, (unsigned)cdiv(h, 256));
  hipLaunchKernelGGL(ce_finalize_kernel, grid, dim3(256), 0, (hipStream_t)stream, acc, grad,
                     inverse, out, out_dtype, h, valid_n);
  SS_CHECK_LAUNCH("ce_finalize_kernel");
  return SS_OK;
}
