// Vocabulary-chunk kernels of the fused linear cross-entropy (A17-A18).
//
// Reference: solution/kernels/cross_entropy.py:1-43 (semantics), :51-89
// (statistics), :92-105 (outputs), :108-122 (derivative), :193-210 (dX
// rescale and scatter).  The logits of a chunk are fp16 (the reference
// rounds logits before any statistic); all statistics are fp32.
//
// ce_stats: one 256-thread workgroup per (row, piece), a piece being up to
// kStatsPiece consecutive logits of the row; one launch covers any number of
// pieces (every chunk of the kept logits).  A lane's four 16-byte loads (8
// consecutive fp16 logits per 2048-logit step) go out together with no branch
// between them; one pass keeps the lane's running max m and its sums of
// exp(z - m) and exp(z - m) * z, rescaled when a step raises m; lanes and
// waves merge as the pieces do.  The piece's partial state goes to its slot of
// partial[row, slots]; ce_outputs folds a row's slots in a fixed order (one
// wave per row: lane-strided, then an xor butterfly of a commutative fold), so
// the results depend only on where the pieces start, not on how many a launch
// covered.

#include "elementwise.h"

namespace ss {

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

constexpr int kStatsHeld = 4;                  // 2048-logit steps a lane holds in registers
constexpr int64_t kStatsPiece = 2048 * kStatsHeld;  // widest piece one workgroup reduces

struct Partial {
  float m, s, t, f;  // max, sum exp(z - m), sum exp(z - m) * z, target logit
  int64_t a;         // first index of the max
};

// State a folded with the next piece b: both sums rescaled to the larger max (a
// side whose max is -inf holds no finite logit and contributes nothing); the
// argmax keeps the lower index on ties.
__device__ __forceinline__ Partial fold(Partial a, const Partial& b) {
  const float m = fmaxf(a.m, b.m);
  const float ra = a.m == -INFINITY ? 0.0f : __expf(a.m - m);
  const float rb = b.m == -INFINITY ? 0.0f : __expf(b.m - m);
  int64_t arg = a.a;
  if (b.m > a.m)
    arg = b.a;
  else if (b.m == a.m && b.a < a.a)
    arg = b.a;
  return Partial{m, a.s * ra + b.s * rb, a.t * ra + b.t * rb, a.f + b.f, arg};
}

// Local index standing for "no max": the piece holds no finite logit.
constexpr int kNoLocal = 0x7fffffff;

// The lane's logits c = 8 tid + 2048 i .. + 7 of one piece (c < w), as fp16.
// No branch around a load (a lane past w reads column 0 again), so a wave's
// loads are all in flight together.  VEC: rows and pieces 16-byte aligned and
// w % 8 == 0, so a lane's 8 logits are all present or all absent (a step with
// c >= w is skipped whole) and columns 0 .. 7 exist; otherwise absent logits
// read as -inf.
template <bool VEC>
__device__ __forceinline__ void stats_load(const half_t* __restrict__ zr, int w, int tid,
                                           half8 (&held)[kStatsHeld]) {
  const half_t ninf = (half_t)-INFINITY;
#pragma unroll
  for (int i = 0; i < kStatsHeld; ++i) {
    const int c = tid * 8 + 2048 * i;
    if constexpr (VEC) {
      held[i] = *reinterpret_cast<const half8*>(zr + (c < w ? c : 0));
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const half_t v = zr[c + j < w ? c + j : 0];
        held[i][j] = c + j < w ? v : ninf;
      }
    }
  }
}

constexpr float kLog2e = 1.4426950408889634f;

// One workgroup per (row, piece).  The lane's logits, 4 steps of 8, are loaded
// together; each step takes its max with packed fp16 max (NaN loses, as in an
// ordered compare; fp16 order is the fp32 order), and its terms as
// p = 2^(z log2e - m log2e) with z read from fp16 by the fused multiply-add.
// The running state (max m, sums against m) rescales when a step raises m.
// The first index of the max and the target logit are picked once per piece.
template <bool VEC>
__global__ __launch_bounds__(256) void ce_stats_kernel(const half_t* __restrict__ z, int64_t ldz,
                                                       const int64_t* __restrict__ targets,
                                                       float4* __restrict__ partial,
                                                       int64_t* __restrict__ partial_arg,
                                                       int64_t width, int64_t piece,
                                                       int64_t start, int64_t slot0,
                                                       int64_t slots, int64_t ignore) {
  __shared__ Partial s_state[4];
  __shared__ float s_found;
  const int64_t row = blockIdx.x;
  const int64_t c0 = (int64_t)blockIdx.y * piece;  // the piece's first column in z
  const int w = (int)(width - c0 < piece ? width - c0 : piece);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t first_index = start + c0;  // vocabulary index of the piece's column 0
  half8 held[kStatsHeld];
  stats_load<VEC>(z + row * ldz + c0, w, tid, held);
  const int64_t tgt = targets[row];
  const int local_t = tgt != ignore && tgt >= first_index && tgt < first_index + w
                          ? (int)(tgt - first_index) : -1;

  float m = -INFINITY, sum = 0.0f, wsum = 0.0f;
  int best_step = -1;
#pragma unroll
  for (int i = 0; i < kStatsHeld; ++i) {
    const int c = tid * 8 + 2048 * i;
    if (c < w) {
      const half8 h = held[i];
      half2_t q = __builtin_elementwise_max(__builtin_elementwise_max(h.s01, h.s23),
                                            __builtin_elementwise_max(h.s45, h.s67));
      const float gm = (float)__builtin_elementwise_max(q.x, q.y);
      if (gm > m) {
        const float r = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m - gm) * kLog2e);
        sum *= r;
        wsum *= r;
        m = gm;
        best_step = i;
      }
      // 2^(z log2e - sh); sh = 0 while no finite logit was seen (its -inf terms add 0)
      const float sh = m == -INFINITY ? 0.0f : m * kLog2e;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (!VEC && c + j >= w) continue;
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf((float)h[j], kLog2e, -sh));
        sum += p;
        wsum = __builtin_fmaf(p, (float)h[j], wsum);
      }
    }
  }
  // The lane's first index of m (only its best step can hold it).
  int arg = kNoLocal;
  if (best_step >= 0) {
    half8 h = held[0];
#pragma unroll
    for (int i = 1; i < kStatsHeld; ++i)
      if (best_step == i) h = held[i];
    const half_t hm = (half_t)m;
#pragma unroll
    for (int j = 7; j >= 0; --j)
      if (h[j] == hm) arg = tid * 8 + 2048 * best_step + j;
  }
  // The target's logit, from the lane that holds it.
  if (local_t >= 0 && tid == (local_t & 2047) >> 3) {
    const int ti = local_t >> 11, tj = local_t & 7;
    half8 h = held[0];
#pragma unroll
    for (int i = 1; i < kStatsHeld; ++i)
      if (ti == i) h = held[i];
    float v = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (tj == j) v = (float)h[j];
    s_found = v;
  }
  Partial st{m, sum, wsum, 0.0f, arg};
  // Lanes, then waves, merged as the pieces are folded.
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    Partial other{__shfl_xor(st.m, o, kWave), __shfl_xor(st.s, o, kWave),
                  __shfl_xor(st.t, o, kWave), 0.0f, (int64_t)__shfl_xor((int)st.a, o, kWave)};
    st = fold(st, other);
  }
  if (lane == 0) s_state[wave] = st;
  __syncthreads();
  if (tid == 0) {
    Partial b = s_state[0];
#pragma unroll
    for (int v = 1; v < 4; ++v) b = fold(b, s_state[v]);
    const int64_t slot = row * slots + slot0 + blockIdx.y;
    // s_found was written before the barrier by the one lane holding the target.
    partial[slot] = make_float4(b.m, b.s, b.t, local_t >= 0 ? s_found : 0.0f);
    partial_arg[slot] = b.a == kNoLocal ? kNoIndex : first_index + b.a;
  }
}

// One wave per row: lane l folds slots l, l + 64, ... in order, then the lanes
// fold pairwise (xor butterfly; fold is commutative, so every lane ends with the
// same state).  The fold order is fixed by the slot count alone.
__global__ __launch_bounds__(256) void ce_outputs_kernel(const float4* __restrict__ partial,
                                                         const int64_t* __restrict__ partial_arg,
                                                         int64_t slots,
                                                         const int64_t* __restrict__ targets,
                                                         float* __restrict__ loss,
                                                         float* __restrict__ entropy,
                                                         float* __restrict__ lse,
                                                         int64_t* __restrict__ best, int64_t n,
                                                         int64_t ignore) {
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= n) return;  // uniform per wave
  const int lane = threadIdx.x & 63;
  const float4* pr = partial + r * slots;
  const int64_t* ar = partial_arg + r * slots;
  Partial st{-INFINITY, 0.0f, 0.0f, 0.0f, kNoIndex};
  for (int64_t k = lane; k < slots; k += kWave) {
    const float4 q = pr[k];
    st = fold(st, Partial{q.x, q.y, q.z, q.w, ar[k]});
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const int64_t oa = __shfl_xor(st.a, o, kWave);
    Partial other{__shfl_xor(st.m, o, kWave), __shfl_xor(st.s, o, kWave),
                  __shfl_xor(st.t, o, kWave), __shfl_xor(st.f, o, kWave), oa};
    st = fold(st, other);
  }
  if (lane == 0) {
    const float l = st.m + __logf(st.s);
    lse[r] = l;
    entropy[r] = l - st.t / st.s;
    loss[r] = targets[r] != ignore ? l - st.f : 0.0f;
    best[r] = st.a;
  }
}

__global__ __launch_bounds__(256) void ce_derivative_kernel(
    const half_t* __restrict__ z, int64_t ldz, const int64_t* __restrict__ z_rows,
    const int64_t* __restrict__ targets,
    const float* __restrict__ lse, const float* __restrict__ grad, half_t* __restrict__ dz,
    half_t* __restrict__ dzg, const float* __restrict__ global_gain_p, int64_t width,
    int64_t start, int64_t ignore, int vec, int64_t n) {
  const int64_t row = blockIdx.x;
  const int64_t c = ((int64_t)blockIdx.y * 256 + threadIdx.x) * 8;
  if (c >= width) return;
  if (row >= n) {
    // Rows n .. of dz_global (its padding up to the head-gradient product's depth):
    // zeros, so the product needs no separate fill.
    half_t* outg = dzg + row * width + c;
    if (vec && c + 8 <= width) {
      *reinterpret_cast<uint4*>(outg) = make_uint4(0, 0, 0, 0);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (c + j < width) outg[j] = (half_t)0.0f;
    }
    return;
  }
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

// Labelled rows and target validation in one workgroup: thread t takes rows
// [t per, (t + 1) per); pass 1 counts its labelled rows and checks its targets,
// a scan over the threads places them, pass 2 writes the labelled rows' indices
// in row order; the rest of `order` is filled with -1.
constexpr int kRowsThreads = 1024;

__global__ __launch_bounds__(kRowsThreads) void ce_rows_kernel(
    const int64_t* __restrict__ targets, int64_t n, int64_t vocab, int64_t ignore,
    int64_t* __restrict__ order, int64_t order_len, int64_t* __restrict__ count,
    uint8_t* __restrict__ ok) {
  __shared__ int64_t s_scan[kRowsThreads];
  __shared__ int s_bad;
  const int tid = threadIdx.x;
  if (tid == 0) s_bad = 0;
  const int64_t per = (n + kRowsThreads - 1) / kRowsThreads;
  const int64_t r0 = tid * per < n ? tid * per : n;
  const int64_t r1 = r0 + per < n ? r0 + per : n;
  int64_t mine = 0;
  bool bad = false;
  for (int64_t r = r0; r < r1; ++r) {
    const int64_t t = targets[r];
    if (t != ignore) {
      ++mine;
      bad = bad || t < 0 || t >= vocab;
    }
  }
  s_scan[tid] = mine;
  __syncthreads();
  if (bad) s_bad = 1;  // benign race: every writer stores 1
  // Inclusive scan (Hillis-Steele) over the thread counts.
  for (int off = 1; off < kRowsThreads; off <<= 1) {
    const int64_t v = tid >= off ? s_scan[tid - off] : 0;
    __syncthreads();
    s_scan[tid] += v;
    __syncthreads();
  }
  const int64_t total = s_scan[kRowsThreads - 1];
  int64_t kept_at = s_scan[tid] - mine;   // labelled rows before this thread's
  for (int64_t r = r0; r < r1; ++r)
    if (targets[r] != ignore) order[kept_at++] = r;
  for (int64_t i = total + tid; i < order_len; i += kRowsThreads) order[i] = -1;
  if (tid == 0) {
    count[0] = total;
    ok[0] = s_bad ? 0 : 1;
  }
}

// gain[0] = max(max_r |grad[r]|, 1e-30) / 1024, NaN when a grad is NaN.
__global__ __launch_bounds__(256) void ce_head_gain_kernel(const float* __restrict__ grad,
                                                           int64_t n, float* __restrict__ gain) {
  __shared__ float s_max[4];
  __shared__ int s_nan[4];
  float m = 0.0f;
  int nan = 0;
  for (int64_t r = threadIdx.x; r < n; r += 256) {
    const float v = fabsf(grad[r]);
    nan |= v != v;
    m = fmaxf(m, v);
  }
  m = wave_max(m);
  for (int o = 32; o >= 1; o >>= 1) nan |= __shfl_xor(nan, o, kWave);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    s_max[wave] = m;
    s_nan[wave] = nan;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = s_max[0];
    int any_nan = s_nan[0];
    for (int w = 1; w < 4; ++w) {
      v = fmaxf(v, s_max[w]);
      any_nan |= s_nan[w];
    }
    gain[0] = any_nan ? __int_as_float(0x7fc00000) : fmaxf(v, 1e-30f) / 1024.0f;
  }
}

static bool al16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

}  // namespace ss

using namespace ss;

extern "C" int ss_ce_stats(const uint16_t* z, int64_t ldz, const int64_t* targets,
                           float* partial, int64_t* partial_arg, int64_t n, int64_t width,
                           int64_t piece, int64_t start, int64_t slot0, int64_t slots,
                           int64_t ignore_index, void* stream) {
  SS_CHECK_ARG(n >= 0 && width > 0 && start >= 0 && ldz >= width, "ss_ce_stats: bad sizes");
  SS_CHECK_ARG(piece > 0 && piece <= kStatsPiece, "ss_ce_stats: piece outside [1, 8192]");
  const int64_t pieces = cdiv(width, piece);
  SS_CHECK_ARG(pieces < 65536 && slot0 >= 0 && slot0 + pieces <= slots,
               "ss_ce_stats: pieces outside the partial row");
  SS_CHECK_ARG(n < (int64_t)1 << 31, "ss_ce_stats: too many rows");
  if (n == 0) return SS_OK;
  SS_CHECK_ARG(z && targets && partial && partial_arg, "ss_ce_stats: null pointer");
  SS_CHECK_ARG(al16(partial), "ss_ce_stats: partial not 16-byte aligned");
  const bool vec = al16(z) && ldz % 8 == 0 && piece % 8 == 0 && width % 8 == 0;
  const dim3 grid((unsigned)n, (unsigned)pieces);
  if (vec)
    hipLaunchKernelGGL(ce_stats_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream,
                       reinterpret_cast<const half_t*>(z), ldz, targets,
                       reinterpret_cast<float4*>(partial), partial_arg, width, piece, start,
                       slot0, slots, ignore_index);
  else
    hipLaunchKernelGGL(ce_stats_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream,
                       reinterpret_cast<const half_t*>(z), ldz, targets,
                       reinterpret_cast<float4*>(partial), partial_arg, width, piece, start,
                       slot0, slots, ignore_index);
  SS_CHECK_LAUNCH("ce_stats_kernel");
  return SS_OK;
}

extern "C" int ss_ce_outputs(const float* partial, const int64_t* partial_arg, int64_t slots,
                             const int64_t* targets, float* loss, float* entropy, float* lse,
                             int64_t* best, int64_t n, int64_t ignore_index, void* stream) {
  SS_CHECK_ARG(n >= 0 && slots > 0, "ss_ce_outputs: bad sizes");
  if (n == 0) return SS_OK;
  SS_CHECK_ARG(partial && partial_arg && targets && loss && entropy && lse && best,
               "ss_ce_outputs: null pointer");
  SS_CHECK_ARG(al16(partial), "ss_ce_outputs: partial not 16-byte aligned");
  SS_CHECK_ARG(cdiv(n, 4) < (int64_t)1 << 31, "ss_ce_outputs: too many rows");
  hipLaunchKernelGGL(ce_outputs_kernel, dim3((unsigned)cdiv(n, 4)), dim3(256), 0,
                     (hipStream_t)stream, reinterpret_cast<const float4*>(partial), partial_arg,
                     slots, targets, loss, entropy, lse, best, n, ignore_index);
  SS_CHECK_LAUNCH("ce_outputs_kernel");
  return SS_OK;
}

extern "C" int ss_ce_derivative(const uint16_t* z, int64_t ldz, const int64_t* z_rows,
                                const int64_t* targets, const float* lse, const float* grad,
                                uint16_t* dz, uint16_t* dz_global, const float* global_gain,
                                int64_t n, int64_t global_rows, int64_t width, int64_t start,
                                int64_t ignore_index, void* stream) {
  SS_CHECK_ARG(n >= 0 && width > 0 && ldz >= width, "ss_ce_derivative: bad sizes");
  SS_CHECK_ARG(!dz_global || global_gain, "ss_ce_derivative: dz_global needs global_gain");
  SS_CHECK_ARG(global_rows >= n && (dz_global || global_rows == n),
               "ss_ce_derivative: global_rows must be >= n (and n without dz_global)");
  SS_CHECK_ARG(global_rows < (int64_t)1 << 31, "ss_ce_derivative: too many rows");
  if (n == 0 && global_rows == 0) return SS_OK;
  SS_CHECK_ARG(z && targets && lse && grad && dz, "ss_ce_derivative: null pointer");
  const int vec = al16(z) && ldz % 8 == 0 && al16(dz) && width % 8 == 0 &&
                  (!dz_global || al16(dz_global));
  SS_CHECK_ARG(cdiv(width, 256 * 8) < 65536, "ss_ce_derivative: width too large");
  const dim3 grid((unsigned)global_rows, (unsigned)cdiv(width, 256 * 8));
  hipLaunchKernelGGL(ce_derivative_kernel, grid, dim3(256), 0, (hipStream_t)stream,
                     reinterpret_cast<const half_t*>(z), ldz, z_rows, targets, lse, grad,
                     reinterpret_cast<half_t*>(dz), reinterpret_cast<half_t*>(dz_global),
                     global_gain, width, start, ignore_index, vec, n);
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

extern "C" int ss_ce_rows(const int64_t* targets, int64_t n, int64_t vocab, int64_t ignore_index,
                          int64_t* order, int64_t order_len, int64_t* count, uint8_t* ok,
                          void* stream) {
  SS_CHECK_ARG(n >= 0 && vocab > 0 && order_len >= n, "ss_ce_rows: bad sizes");
  SS_CHECK_ARG(count && ok && (n == 0 || targets) && (order_len == 0 || order),
               "ss_ce_rows: null pointer");
  hipLaunchKernelGGL(ce_rows_kernel, dim3(1), dim3(kRowsThreads), 0, (hipStream_t)stream,
                     targets, n, vocab, ignore_index, order, order_len, count, ok);
  SS_CHECK_LAUNCH("ce_rows_kernel");
  return SS_OK;
}

extern "C" int ss_ce_head_gain(const float* grad, int64_t n, float* gain, void* stream) {
  SS_CHECK_ARG(n >= 0, "ss_ce_head_gain: negative n");
  SS_CHECK_ARG(gain && (n == 0 || grad), "ss_ce_head_gain: null pointer");
  hipLaunchKernelGGL(ce_head_gain_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, grad, n,
                     gain);
  SS_CHECK_LAUNCH("ce_head_gain_kernel");
  return SS_OK;
}
