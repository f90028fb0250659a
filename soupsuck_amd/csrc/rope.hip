// Joint q/k rotary position embedding, forward and input gradients.
//
// Rows are (batch, head, token) with the q heads first, then the k heads; one
// wave handles one row, its lanes over the half width (lane c holds columns
// c and c + half, looping when half > 64).  With x1 = x[c], x2 = x[c + half]:
//   forward   y1 = R(x1 c1) + R(-x2 s1),  y2 = R(x2 c2) + R(x1 s2)
//             R = rounding to the output dtype promote(x, cos), sums rounded
//             on store (solution/kernels/rope.py:24-56);
//   backward  d1 = R'(g1 c1) + R'(g2 s2),  d2 = R'(g2 c2) - R'(g1 s1)
//             R' = rounding to the input's dtype (:59-98).
// fp32 arithmetic, no contraction (-ffp-contract=off), so the results equal
// the numpy restatement bit for bit.  Inputs take runtime strides (batch,
// head, token; the last dimension stride is given for gradients and must be
// 1 for q / k / cos / sin); cos / sin have 1 or B batches; forward outputs
// are contiguous [B, H, S, D], the backward's gradients take the caller's
// (batch, head, token) strides, so they can share the memory layout of the
// forward's inputs (the transposed projection views).  HBM-bound: 2 x 2 B per fp16 element of q / k
// plus cos / sin (shared by all heads of a token, mostly cache hits).
// Aligned layouts take the vector kernel (4 columns per thread).

#include "common.h"
#include "elementwise.h"

namespace ss {
namespace {

struct RopeOperand {
  const void* x;  // q / k (forward) or its output gradient (backward); null: skip
  int xd;
  int64_t sb, sh, st, sd;  // element strides: batch, head, token, last dim
  void* y;
  int yd;
  int64_t heads;
  int64_t yb, yh, yt;  // output element strides: batch, head, token (last dim 1)
};

struct RopeArgs {
  RopeOperand q, k;
  const void* c;
  const void* s;
  int cd;
  int64_t cb, ct, sb, st;  // cos / sin strides (batch, token); last stride 1
  int64_t c_batches;
  int64_t batches, tokens, half;
};

template <bool BWD>
__global__ __launch_bounds__(256) void rope_kernel(RopeArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t heads = a.q.heads + a.k.heads;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.batches * heads * a.tokens) return;
  const int64_t token = row % a.tokens;
  const int64_t head = (row / a.tokens) % heads;
  const int64_t batch = row / (heads * a.tokens);
  const bool is_q = head < a.q.heads;
  const RopeOperand& o = is_q ? a.q : a.k;
  const int64_t h = is_q ? head : head - a.q.heads;
  if (!o.x) return;
  const int64_t cbatch = a.c_batches == 1 ? 0 : batch;
  const int64_t coff = cbatch * a.cb + token * a.ct;
  const int64_t soff = cbatch * a.sb + token * a.st;
  const int64_t xoff = batch * o.sb + h * o.sh + token * o.st;
  const int64_t yoff = batch * o.yb + h * o.yh + token * o.yt;
  for (int64_t c = lane; c < a.half; c += 64) {
    const float c1 = ld_elem(a.c, a.cd, coff + c), c2 = ld_elem(a.c, a.cd, coff + c + a.half);
    const float s1 = ld_elem(a.s, a.cd, soff + c), s2 = ld_elem(a.s, a.cd, soff + c + a.half);
    const float x1 = ld_elem(o.x, o.xd, xoff + c * o.sd);
    const float x2 = ld_elem(o.x, o.xd, xoff + (c + a.half) * o.sd);
    float lo, hi;
    if (BWD) {
      lo = round_to(o.yd, x1 * c1) + round_to(o.yd, x2 * s2);
      hi = round_to(o.yd, x2 * c2) - round_to(o.yd, x1 * s1);
    } else {
      lo = round_to(o.yd, x1 * c1) + round_to(o.yd, -x2 * s1);
      hi = round_to(o.yd, x2 * c2) + round_to(o.yd, x1 * s2);
    }
    st_elem(o.y, o.yd, yoff + c, lo);
    st_elem(o.y, o.yd, yoff + c + a.half, hi);
  }
}

__device__ __forceinline__ void load4(const void* p, int dt, int64_t off, float (&v)[4]) {
  if (dt == SS_F16) {
    const half4 h = *reinterpret_cast<const half4*>(static_cast<const half_t*>(p) + off);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = (float)h[e];
  } else {
    const float4v f = *reinterpret_cast<const float4v*>(static_cast<const float*>(p) + off);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = f[e];
  }
}

__device__ __forceinline__ void store4(void* p, int dt, int64_t off, const float (&v)[4]) {
  if (dt == SS_F16) {
    half4 h;
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = f32_to_f16(v[e]);
    *reinterpret_cast<half4*>(static_cast<half_t*>(p) + off) = h;
  } else {
    float4v f;
#pragma unroll
    for (int e = 0; e < 4; ++e) f[e] = v[e];
    *reinterpret_cast<float4v*>(static_cast<float*>(p) + off) = f;
  }
}

template <int DT>
__device__ __forceinline__ void load4t(const void* p, int64_t off, float (&v)[4]) {
  if constexpr (DT == SS_F16) {
    const half4 h = *reinterpret_cast<const half4*>(static_cast<const half_t*>(p) + off);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = (float)h[e];
  } else {
    const float4v f = *reinterpret_cast<const float4v*>(static_cast<const float*>(p) + off);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = f[e];
  }
}

// Vector form: each thread takes 4 consecutive columns of one row's half
// width (8- or 16-byte accesses), half / 4 threads per row, rows packed
// across the workgroup.  Needs half % 4 == 0, unit last-dimension strides,
// every other stride a multiple of 4 and 16-byte aligned bases (vec_ok).
// CD: the cos / sin dtype, or -1 to read it (and every other dtype) at run
// time; with CD set, q / k and their outputs are fp16, and the six loads of a
// thread go out together (a run-time dtype branch around each load makes it
// wait for the previous one).
template <bool BWD, int CD>
__global__ __launch_bounds__(256) void rope_vec_kernel(RopeArgs a) {
  const int64_t quads = a.half / 4;
  const int64_t heads = a.q.heads + a.k.heads;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = gid / quads;
  if (row >= a.batches * heads * a.tokens) return;
  const int64_t c = (gid - row * quads) * 4;
  const int64_t token = row % a.tokens;
  const int64_t head = (row / a.tokens) % heads;
  const int64_t batch = row / (heads * a.tokens);
  const bool is_q = head < a.q.heads;
  // The operand's fields picked one by one (each a select of two kernel
  // arguments), not through a reference chosen at run time, which would be
  // read from the argument segment by a dependent load before the data loads.
  const void* ox = is_q ? a.q.x : a.k.x;
  if (!ox) return;
  void* oy = is_q ? a.q.y : a.k.y;
  const int xd = is_q ? a.q.xd : a.k.xd;
  const int yd_rt = is_q ? a.q.yd : a.k.yd;
  const int64_t h = is_q ? head : head - a.q.heads;
  const int64_t cbatch = a.c_batches == 1 ? 0 : batch;
  const int64_t coff = cbatch * a.cb + token * a.ct + c;
  const int64_t soff = cbatch * a.sb + token * a.st + c;
  const int64_t xoff = batch * (is_q ? a.q.sb : a.k.sb) + h * (is_q ? a.q.sh : a.k.sh) +
                       token * (is_q ? a.q.st : a.k.st) + c;
  const int64_t yoff = batch * (is_q ? a.q.yb : a.k.yb) + h * (is_q ? a.q.yh : a.k.yh) +
                       token * (is_q ? a.q.yt : a.k.yt) + c;
  float c1[4], c2[4], s1[4], s2[4], x1[4], x2[4], lo[4], hi[4];
  if constexpr (CD < 0) {
    load4(ox, xd, xoff, x1);
    load4(ox, xd, xoff + a.half, x2);
    load4(a.c, a.cd, coff, c1);
    load4(a.c, a.cd, coff + a.half, c2);
    load4(a.s, a.cd, soff, s1);
    load4(a.s, a.cd, soff + a.half, s2);
  } else {
    load4t<SS_F16>(ox, xoff, x1);
    load4t<SS_F16>(ox, xoff + a.half, x2);
    load4t<CD>(a.c, coff, c1);
    load4t<CD>(a.c, coff + a.half, c2);
    load4t<CD>(a.s, soff, s1);
    load4t<CD>(a.s, soff + a.half, s2);
  }
  const int yd = CD < 0 ? yd_rt : SS_F16;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (BWD) {
      lo[e] = round_to(yd, x1[e] * c1[e]) + round_to(yd, x2[e] * s2[e]);
      hi[e] = round_to(yd, x2[e] * c2[e]) - round_to(yd, x1[e] * s1[e]);
    } else {
      lo[e] = round_to(yd, x1[e] * c1[e]) + round_to(yd, -x2[e] * s1[e]);
      hi[e] = round_to(yd, x2[e] * c2[e]) + round_to(yd, x1[e] * s2[e]);
    }
  }
  store4(oy, yd, yoff, lo);
  store4(oy, yd, yoff + a.half, hi);
}

bool al16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

bool vec_ok(const RopeArgs& a) {
  if (a.half % 4 || !al16(a.c) || !al16(a.s) || a.cb % 4 || a.ct % 4 || a.sb % 4 || a.st % 4)
    return false;
  for (const RopeOperand* o : {&a.q, &a.k}) {
    if (!o->x) continue;
    if (o->sd != 1 || !al16(o->x) || !al16(o->y) || o->sb % 4 || o->sh % 4 || o->st % 4 ||
        o->yb % 4 || o->yh % 4 || o->yt % 4)
      return false;
  }
  return true;
}

int launch_rope(bool bwd, const RopeArgs& a, void* stream, const char* fn) {
  SS_CHECK_ARG(a.batches >= 0 && a.tokens >= 0 && a.half > 0 && a.q.heads >= 0 &&
                   a.k.heads >= 0 && (a.c_batches == 1 || a.c_batches == a.batches),
               "%s: bad shape", fn);
  SS_CHECK_ARG(valid_dtype(a.cd) && (!a.q.x || (valid_dtype(a.q.xd) && valid_dtype(a.q.yd))) &&
                   (!a.k.x || (valid_dtype(a.k.xd) && valid_dtype(a.k.yd))),
               "%s: dtype must be SS_F16 or SS_F32", fn);
  const int64_t rows = a.batches * (a.q.heads + a.k.heads) * a.tokens;
  if (rows == 0) return SS_OK;
  SS_CHECK_ARG(a.c && a.s && (!a.q.x || a.q.y) && (!a.k.x || a.k.y), "%s: null pointer", fn);
  SS_CHECK_ARG(cdiv(rows, 4) <= 0x7fffffff, "%s: too many rows", fn);
  if (vec_ok(a) && cdiv(rows * (a.half / 4), 256) <= 0x7fffffff) {
    // fp16 q / k in and out: the dtypes are template arguments.
    const bool f16 = (!a.q.x || (a.q.xd == SS_F16 && a.q.yd == SS_F16)) &&
                     (!a.k.x || (a.k.xd == SS_F16 && a.k.yd == SS_F16));
    auto kern = !f16 ? (bwd ? rope_vec_kernel<true, -1> : rope_vec_kernel<false, -1>)
                : a.cd == SS_F16 ? (bwd ? rope_vec_kernel<true, SS_F16> : rope_vec_kernel<false, SS_F16>)
                                 : (bwd ? rope_vec_kernel<true, SS_F32> : rope_vec_kernel<false, SS_F32>);
    hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(rows * (a.half / 4), 256)), dim3(256), 0,
                       (hipStream_t)stream, a);
    SS_CHECK_LAUNCH(fn);
    return SS_OK;
  }
  auto kern = bwd ? rope_kernel<true> : rope_kernel<false>;
  hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(rows, 4)), dim3(256), 0, (hipStream_t)stream, a);
  SS_CHECK_LAUNCH(fn);
  return SS_OK;
}

}  // namespace
}  // namespace ss

using namespace ss;

extern "C" int ss_rope_fwd(const void* q, int q_dtype, int64_t qb, int64_t qh, int64_t qt,
                           const void* k, int k_dtype, int64_t kb, int64_t kh, int64_t kt,
                           const void* cos, const void* sin, int cs_dtype, int64_t cb, int64_t ct,
                           int64_t sb, int64_t st, int64_t c_batches, void* yq, int yq_dtype,
                           void* yk, int yk_dtype, int64_t batches, int64_t qheads,
                           int64_t kheads, int64_t tokens, int64_t half, void* stream) {
  const char* fn = "ss_rope_fwd";
  SS_CHECK_ARG(yq_dtype == promote(q_dtype, cs_dtype) && yk_dtype == promote(k_dtype, cs_dtype),
               "%s: outputs must be promote(x, cos)", fn);
  // Contiguous [B, H, S, D] outputs.
  const int64_t d = 2 * half;
  RopeArgs a{{q, q_dtype, qb, qh, qt, 1, yq, yq_dtype, qheads, qheads * tokens * d, tokens * d, d},
             {k, k_dtype, kb, kh, kt, 1, yk, yk_dtype, kheads, kheads * tokens * d, tokens * d, d},
             cos, sin, cs_dtype, cb, ct, sb, st, c_batches, batches, tokens, half};
  return launch_rope(false, a, stream, fn);
}

extern "C" int ss_rope_bwd(const void* gq, int gq_dtype, int64_t qb, int64_t qh, int64_t qt,
                           int64_t qd, const void* gk, int gk_dtype, int64_t kb, int64_t kh,
                           int64_t kt, int64_t kd, const void* cos, const void* sin,
                           int cs_dtype, int64_t cb, int64_t ct, int64_t sb, int64_t st,
                           int64_t c_batches, void* dq, int dq_dtype, int64_t dqb, int64_t dqh,
                           int64_t dqt, void* dk, int dk_dtype, int64_t dkb, int64_t dkh,
                           int64_t dkt, int64_t batches, int64_t qheads, int64_t kheads,
                           int64_t tokens, int64_t half, void* stream) {
  const char* fn = "ss_rope_bwd";
  RopeArgs a{{gq, gq_dtype, qb, qh, qt, qd, dq, dq_dtype, qheads, dqb, dqh, dqt},
             {gk, gk_dtype, kb, kh, kt, kd, dk, dk_dtype, kheads, dkb, dkh, dkt},
             cos, sin, cs_dtype, cb, ct, sb, st, c_batches, batches, tokens, half};
  return launch_rope(true, a, stream, fn);
}
