/* soupsuck_amd: C ABI of the MI355X (gfx950) QLoRA NF4 hot path.
 *
 * Conventions
 *   - Every entry point is extern "C", takes plain device pointers, element
 *     counts and a HIP stream (passed as void*, a hipStream_t; NULL = the
 *     default stream), enqueues work on that stream and returns immediately.
 *   - Return value: 0 on success, a negative SS_ERR_* code otherwise.  Invalid
 *     arguments are rejected BEFORE any launch; ss_last_error() then returns a
 *     thread-local message.  No entry point throws, allocates device memory or
 *     synchronizes the stream, and none keeps mutable global state except
 *     ss_nf4_gemm_fwd_noalloc, whose fixed device scratch and per-device
 *     pointer cache are described at its declaration.
 *   - fp16 tensors are passed as uint16_t* (IEEE binary16 bits); "dtype" codes
 *     are SS_F16 / SS_F32.
 *   - Reference citations are file:line in the reference tree (Khasuetolog/
 *     soupsuck); each entry point replaces the Triton launch or the library
 *     call named there, behind the same Python-level interface.
 */
#ifndef SOUPSUCK_AMD_H
#define SOUPSUCK_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SS_ABI_VERSION 1

enum ss_status {
  SS_OK = 0,
  SS_ERR_INVALID_ARGUMENT = -1,
  SS_ERR_LAUNCH = -2,
  SS_ERR_UNSUPPORTED = -3
};

enum ss_dtype { SS_F16 = 0, SS_F32 = 1 };

/* Library identity and the last error message of the calling thread. */
int ss_abi_version(void);
const char* ss_last_error(void);

/* ---------------------------------------------------------------- NF4 ---
 * Nested (double-quantized) NF4 state, bitsandbytes 0.50.2 layout
 * (reference solution/kernels/nf4.py:140-168): packed uint8[ceil(n/2)] with
 * element 2j in the HIGH nibble of byte j; qabs uint8[ceil(n/64)];
 * absmax2 fp32[ceil(n/16384)]; code2 fp32[256]; offset fp32[1] (device).
 */

/* A2. out[i] = fp16(NF4[nib(i)] * fp32(fp32(code2[qabs[i/64]] * absmax2[i/16384]) + offset[0])),
 * bit-exact, no FMA.  Replaces nf4_decode_kernel[NESTED=True] launched by
 * dequantize_nf4 (solution/kernels/nf4.py:41-59,190-203).  Any n >= 0 and any
 * pointer alignment (an aligned vector path is used when possible). */
int ss_nf4_dequant_nested(const uint8_t* packed, const uint8_t* qabs, const float* absmax2,
                          const float* code2, const float* offset, uint16_t* out, int64_t n,
                          void* stream);

/* A2, transposed: out[kk][nn] = Wdec[nn][kk] for a weight of shape [rows, cols]
 * (out is [cols, rows] row-major), bit-exact like ss_nf4_dequant_nested.  The
 * backward's large-T path decodes W^T once and runs dX = dY . W as a
 * K-contiguous GEMM.  Needs cols % 64 == 0, 8-byte aligned packed and 16-byte
 * aligned out (SS_ERR_UNSUPPORTED otherwise). */
int ss_nf4_dequant_nested_t(const uint8_t* packed, const uint8_t* qabs, const float* absmax2,
                            const float* code2, const float* offset, uint16_t* out,
                            int64_t rows, int64_t cols, void* stream);

/* A3. out[i] = fp16(NF4[nib(i)] * absmax[i/64]) with an already reconstructed
 * fp32 absmax.  Replaces _dequantize_flat_into / nf4_decode_kernel[NESTED=False]
 * (solution/kernels/nf4.py:181-187), the bnb backend _dequantize_4bit_impl
 * entry (solution/nf4_patch.py:89-106). */
int ss_nf4_dequant_flat(const uint8_t* packed, const float* absmax, uint16_t* out, int64_t n,
                        void* stream);

/* A7/A9 forward. y[t,n] = fp16(sum_k x[t,k] * Wdec[n,k] + bias[n]) with
 * Wdec the A2-decoded weight [N,K] (row-major, element n*K+k), fp32
 * accumulation, bias (fp16, may be NULL) added to the accumulator.
 * Replaces bnb.matmul_4bit -> gemm_4bit / _dequant_linear_fallback
 * (solution/nf4_patch.py:108-120) and nf4_tile_matmul_kernel[TRANSPOSE=False]
 * (solution/kernels/nf4_gemm.py:35-96).  x is [T,K] row-major with row
 * stride ldx >= K; y is [T,N] with row stride ldy >= N.
 * workspace: device scratch of at least ss_nf4_gemm_workspace_size(t,n,k)
 * bytes (may be NULL when that size is 0); used by the large-T path, which
 * decodes W once into it. */
int ss_nf4_gemm_fwd(const uint16_t* x, int64_t ldx, int64_t t, const uint8_t* packed,
                    const uint8_t* qabs, const float* absmax2, const float* code2,
                    const float* offset, int64_t n, int64_t k, const uint16_t* bias,
                    uint16_t* y, int64_t ldy, void* workspace, size_t workspace_bytes,
                    void* stream);

/* ss_nf4_gemm_fwd without a workspace: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * result and kernels as ss_nf4_gemm_fwd (bit-identical output); its scratch is
 * a fixed 64 MiB device array per GPU, held until the process ends.  Shapes
 * whose forward needs more scratch than that (T >= 256 with a large weight)
 * are rejected with SS_ERR_INVALID_ARGUMENT; every T < 256 at the Qwen2.5
 * 1.5B/7B projection shapes fits.  Nothing is allocated and no library routine
 * that allocates is called.  Calls that overlap in time on one GPU share the
 * scratch and race: issue them on one stream, or serialise them. */
int ss_nf4_gemm_fwd_noalloc(const uint16_t* x, int64_t ldx, int64_t t, const uint8_t* packed,
                            const uint8_t* qabs, const float* absmax2, const float* code2,
                            const float* offset, int64_t n, int64_t k, const uint16_t* bias,
                            uint16_t* y, int64_t ldy, void* stream);

/* A8/A9 backward.  dx[t,k] = fp16(sum_n dy[t,n] * Wdec[n,k]).  Replaces
 * MatMul4Bit.backward's dequantize_4bit + torch.matmul(dY, W)
 * (solution/nf4_patch.py:62-87; tasks/RUNTIME_AUDIT.md:113) and
 * nf4_tile_matmul_kernel[TRANSPOSE=True] (solution/kernels/nf4_gemm.py:35-118).
 * If accumulate != 0, dx is read and the result is fp16(dx_old + sum). */
int ss_nf4_gemm_dx(const uint16_t* dy, int64_t lddy, int64_t t, const uint8_t* packed,
                   const uint8_t* qabs, const float* absmax2, const float* code2,
                   const float* offset, int64_t n, int64_t k, uint16_t* dx, int64_t lddx,
                   int accumulate, void* workspace, size_t workspace_bytes, void* stream);

/* NF4 encoder (weight preparation, not on the training path).  Restates
 * bitsandbytes 0.50.2 quantize_4bit(w, blocksize=64, compress_statistics=True,
 * quant_type="nf4"), which the reference calls to build its states
 * (solution/tests/test_nf4.py:40-44; Params4bit in solution/tests/test_unpad.py:
 * 261-266).  w is fp16/fp32 [n]; code2 (input) is the 256-entry signed dynamic
 * map; outputs packed, qabs, absmax2 and offset as in the state above;
 * absmax_workspace is fp32[ceil(n/64)] scratch (it holds the first-level absmax). */
int ss_nf4_quantize(const void* w, int w_dtype, int64_t n, uint8_t* packed, uint8_t* qabs,
                    float* absmax2, const float* code2, float* offset, float* absmax_workspace,
                    void* stream);

/* Workspace bytes the NF4 GEMM entry points (forward, dX, LoRA-fused) use
 * for this shape: split-K partial planes of the small-T and fused
 * decode-in-GEMM kernels, or the decoded weight (W, or W^T for dX) plus the
 * dense GEMM's partials.  A smaller workspace (or NULL) selects a path that
 * fits. */
size_t ss_nf4_gemm_workspace_size(int64_t t, int64_t n, int64_t k);

/* A7+A10+A11 fused: the QLoRA projection forward of one Linear4bit with its
 * LoRA adapter (reference solution/lora.py:135-163 with
 * solution/kernels/lora_epilogue.py:24-34 under fp16 autocast):
 *   y = fp16( fp16(x . Wdec^T + bias) + fp16( fp16(z . lora_b^T) * scale ) )
 * z = fp16(drop(x) . lora_a^T) is [t, 16] contiguous (ss_lora_project);
 * lora_b is [n, 16] contiguous; rank 16.  Same workspace rule as above. */
int ss_qlora_fwd(const uint16_t* x, int64_t ldx, int64_t t, const uint8_t* packed,
                 const uint8_t* qabs, const float* absmax2, const float* code2,
                 const float* offset, int64_t n, int64_t k, const uint16_t* bias,
                 const uint16_t* z, const uint16_t* lora_b, float scale, uint16_t* y,
                 int64_t ldy, void* workspace, size_t workspace_bytes, void* stream);

/* A8+A12 fused: dx = fp16(dy . Wdec + dz . lora_a), the base dX of
 * MatMul4Bit.backward plus the LoRA input gradient in one accumulator
 * (reference solution/lora_pair.py:52-65 sums them in fp16 after two
 * roundings).  dz is [t, 16] contiguous, lora_a is [16, k] contiguous. */
int ss_qlora_dx(const uint16_t* dy, int64_t lddy, int64_t t, const uint8_t* packed,
                const uint8_t* qabs, const float* absmax2, const float* code2,
                const float* offset, int64_t n, int64_t k, const uint16_t* dz,
                const uint16_t* lora_a, uint16_t* dx, int64_t lddx, void* workspace,
                size_t workspace_bytes, void* stream);

/* A10-A12 as one projection step (forward / backward of the rank-16 QLoRA
 * projection out = fp16(X . Wdec^T + bias) + fp16(fp16(Z . lora_b^T) * scale),
 * Z = fp16(X . lora_a^T); reference solution/lora.py:135-163 forward and
 * solution/lora_pair.py:34-65 backward order).  The rank-16 jobs that do not
 * depend on each other run in one launch with the NF4 decode of the
 * decode-first path, ahead of the NF4 GEMM:
 * ss_qlora_forward: z [t,16] (written, kept for the backward) and y [t,n] as
 *   ss_lora_project (Z) followed by ss_qlora_fwd.
 * ss_qlora_backward: dz [t,16] = fp16(fp16(dy*scale) . lora_b), db [n,16] =
 *   fp16(fp16(dy*scale)^T . z), dx [t,k] = fp16(dy . Wdec + dz . lora_a),
 *   da [16,k] = fp16(dz^T . x), as ss_lora_project, ss_lora_grad (twice) and
 *   ss_qlora_dx.
 * x, lora_a [16,k], lora_b [n,16], z, dz contiguous rows; workspace as for
 * ss_qlora_fwd / ss_qlora_dx (ss_nf4_gemm_workspace_size); rank_workspace:
 * ss_qlora_rank_workspace_size(t, n, k) bytes with the contract of the
 * rank-16 products' workspace below (zero-filled once, left zero).  No
 * counterpart in the reference: it is the fused form of the entry points it
 * composes. */
size_t ss_qlora_rank_workspace_size(int64_t t, int64_t n, int64_t k);
int ss_qlora_forward(const uint16_t* x, int64_t ldx, int64_t t, const uint8_t* packed,
                     const uint8_t* qabs, const float* absmax2, const float* code2,
                     const float* offset, int64_t n, int64_t k, const uint16_t* bias,
                     const uint16_t* lora_a, const uint16_t* lora_b, float scale, uint16_t* z,
                     uint16_t* y, int64_t ldy, void* workspace, size_t workspace_bytes,
                     void* rank_workspace, size_t rank_workspace_bytes, void* stream);
int ss_qlora_backward(const uint16_t* dy, int64_t lddy, int64_t t, const uint8_t* packed,
                      const uint8_t* qabs, const float* absmax2, const float* code2,
                      const float* offset, int64_t n, int64_t k, const uint16_t* x, int64_t ldx,
                      const uint16_t* z, const uint16_t* lora_a, const uint16_t* lora_b,
                      float scale, uint16_t* dx, int64_t lddx, uint16_t* dz, uint16_t* da,
                      uint16_t* db, void* workspace, size_t workspace_bytes,
                      void* rank_workspace, size_t rank_workspace_bytes, void* stream);

/* The same two steps with LoRA dropout p in (0, 1) on the LoRA input
 * (reference solution/lora.py:1-40,151-163: PEFT's Dropout on an fp32 copy of
 * X feeding lora_A only).  The mask is a function of (seed, element index of
 * X [t, k]) -- Philox4x32-10, defined in ss_dropout_mask below -- recomputed
 * wherever an element is used, never stored; forward and backward must get
 * the same seed and p.  With Xd = fp16(keep ? fp32(x) * fp32(1 / (1 - p)) : 0):
 * forward:  z = fp16(Xd . lora_a^T); y as ss_qlora_forward;
 * backward: dz, db as ss_qlora_backward; da = fp16(dz^T . Xd);
 *           dx = fp16(fp16(dy . Wdec) + (keep ? fp16(fp32(fp16(dz . lora_a))
 *                * fp32(1 / (1 - p))) : 0)).
 * K % 8 == 0; the backward also needs 16-byte aligned x, dx and lora_a rows
 * (SS_ERR_UNSUPPORTED otherwise). */
int ss_qlora_forward_dropout(const uint16_t* x, int64_t ldx, int64_t t, const uint8_t* packed,
                             const uint8_t* qabs, const float* absmax2, const float* code2,
                             const float* offset, int64_t n, int64_t k, const uint16_t* bias,
                             const uint16_t* lora_a, const uint16_t* lora_b, float scale,
                             uint64_t seed, float p, uint16_t* z, uint16_t* y, int64_t ldy,
                             void* workspace, size_t workspace_bytes, void* rank_workspace,
                             size_t rank_workspace_bytes, void* stream);
int ss_qlora_backward_dropout(const uint16_t* dy, int64_t lddy, int64_t t, const uint8_t* packed,
                              const uint8_t* qabs, const float* absmax2, const float* code2,
                              const float* offset, int64_t n, int64_t k, const uint16_t* x,
                              int64_t ldx, const uint16_t* z, const uint16_t* lora_a,
                              const uint16_t* lora_b, float scale, uint64_t seed, float p,
                              uint16_t* dx, int64_t lddx, uint16_t* dz, uint16_t* da,
                              uint16_t* db, void* workspace, size_t workspace_bytes,
                              void* rank_workspace, size_t rank_workspace_bytes, void* stream);

/* The dropout mask of an X [rows, cols] for (seed, p): out[e] = 1 if element
 * e = row * cols + col is kept, else 0 (uint8 [rows * cols]).  Definition:
 * key = (seed mod 2^32, seed div 2^32), counter = (e div 4 mod 2^32,
 * e div 4 div 2^32, 0, 0), u = word (e mod 4) of Philox4x32-10(counter, key)
 * (Salmon et al., SC'11), keep = u < floor((1 - p) * 2^32).  The fused
 * dropout entry points use exactly these bits.  p in (0, 1). */
int ss_dropout_mask(uint64_t seed, float p, int64_t rows, int64_t cols, uint8_t* out,
                    void* stream);

/* ------------------------------------------------ rank-16 LoRA products ---
 * HBM-bound skinny GEMMs of the LoRA branch (reference solution/lora.py:161,
 * solution/lora_pair.py:52-65), fp32 accumulation, one fp16 rounding.
 * ss_lora_project: out[m, 16] = fp16(A'[m, k] . W) with A' = A or, when
 *   scale_a, fp16(A * a_scale) elementwise (dL = fp16(g * s)); W element
 *   (kk, r) at w[kk*ldw + r] when w_kr (lora_B [N,16]) else w[r*ldw + kk]
 *   (lora_A [16,K]).  Z = X.A^T and dZ = dL.B.
 * ss_lora_grad: C[16, n] = fp16(P[t,16]^T . Q'[t, n]) with Q' = Q or
 *   fp16(Q * q_scale); stored [16][n], or [n][16] when transpose.
 *   dA = dZ^T.X and dB = dL^T.Z.
 * Each op is one launch; the reduction is split over workgroups and the last
 * workgroup of an output block to arrive adds the splits in split order
 * (deterministic).
 * workspace: at least ss_lora_workspace_size(rows, cols) bytes for an output
 * with rows x 16 or 16 x cols elements.  Its first 256 KiB are arrival
 * counters (a fixed area shared by both ops and all shapes) that must be
 * zero when the op starts; the op leaves them zero, so a workspace
 * zero-filled once serves any sequence of calls that do not overlap in time
 * (calls on one stream); overlapping calls need separate workspaces.  With a
 * NULL or smaller workspace the reduction is not split (slower, same
 * contract otherwise). */
size_t ss_lora_workspace_size(int64_t rows, int64_t cols);
int ss_lora_project(const uint16_t* a, int64_t lda, int64_t m, int64_t k, const uint16_t* w,
                    int64_t ldw, int w_kr, int scale_a, float a_scale, uint16_t* out,
                    void* workspace, size_t workspace_bytes, void* stream);
int ss_lora_grad(const uint16_t* p, int64_t ldp, const uint16_t* q, int64_t ldq, int64_t t,
                 int64_t n, int scale_q, float q_scale, int transpose, uint16_t* out,
                 void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------- dense fp16 GEMM ---
 * C[M,N] = alpha * op(A)[M,K] . op(B)[K,N] (+ bias[N]) (+ beta * C), fp16
 * operands, fp32 accumulation.  a_trans = 0: A stored [M,K] (row stride lda);
 * a_trans = 1: A stored [K,M].  b_trans = 0: B stored [K,N]; b_trans = 1: B
 * stored [N,K].  c_dtype SS_F16 or SS_F32; beta must be 0 or 1 (1 reads C).
 * bias (fp16, length N) may be NULL.  Serves the LoRA products
 * (solution/lora.py:161, solution/lora_pair.py:34-65) and the vocabulary-chunk
 * GEMMs of the fused cross-entropy (solution/kernels/cross_entropy.py:149,
 * 195,202), which the reference sends to cuBLAS. */
int ss_gemm_f16(int a_trans, int b_trans, int64_t m, int64_t n, int64_t k, float alpha,
                const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                const uint16_t* bias, float beta, void* c, int c_dtype, int64_t ldc,
                void* stream);

/* Same product with scratch for splitting the reduction over workgroups (the
 * direct-to-LDS kernel: K % 64 == 0, 16-byte aligned operands, M % 8 == 0
 * for a_trans = 1 and N % 8 == 0 for b_trans = 0):
 * ss_gemm_f16_workspace_size(a_trans, b_trans, m, n, k) bytes; a smaller
 * workspace (or none) means no split.  alpha_dev, when not NULL, is a device
 * fp32 scalar that multiplies alpha (a scale computed on the device needs no
 * host round trip).  Serves the vocabulary-chunk products of the fused
 * cross-entropy backward (solution/kernels/cross_entropy.py:195,202), whose
 * output tile count is small. */
size_t ss_gemm_f16_workspace_size(int a_trans, int b_trans, int64_t m, int64_t n, int64_t k);
int ss_gemm_f16_split(int a_trans, int b_trans, int64_t m, int64_t n, int64_t k, float alpha,
                      const float* alpha_dev, const uint16_t* a, int64_t lda, const uint16_t* b,
                      int64_t ldb, const uint16_t* bias, float beta, void* c, int c_dtype,
                      int64_t ldc, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------- LoRA (A11) ---
 * out = round_out(fp32(base) + fp32(scaled)), scaled = round_adapter(adapter*s),
 * rounded again to the base dtype when cast_to_result.  out_dtype is
 * base_dtype if cast_to_result else promote(base_dtype, adapter_dtype).
 * Replaces lora_scale_add_kernel (solution/kernels/lora_epilogue.py:24-34). */
int ss_lora_epilogue_fwd(const void* base, int base_dtype, const void* adapter, int adapter_dtype,
                         void* out, int out_dtype, int64_t count, float scale, int cast_to_result,
                         void* stream);

/* d_adapter = round_adapter(fp32(round_adapter(grad)) * s).  Replaces
 * lora_scale_gradient_kernel (solution/kernels/lora_epilogue.py:37-43). */
int ss_lora_epilogue_bwd(const void* grad, int grad_dtype, void* d_adapter, int adapter_dtype,
                         int64_t count, float scale, void* stream);

/* ---------------------------------------------- NF4 GEMM + SwiGLU (MLP) ---
 * Forward: up = fp16(X . W_up^T) (W_up the NF4 weight [n, k], X [t, k]),
 * act = fp16(silu(gate) * up) with gate [t, n] fp16; `up` may be NULL (not
 * kept, e.g. recomputed in backward).  Backward: dact = fp16(dY . W_down)
 * (W_down [n, k], dY [t, n]), then dgate = fp16((dact up) slope(gate)),
 * dup = fp16(dact silu(gate)) over [t, k].  The activation is applied in the
 * GEMM epilogue where the chosen kernel supports it, else by the SwiGLU
 * kernel in place; results are bit-identical to ss_nf4_gemm_fwd / _dx
 * followed by ss_swiglu_fwd / _bwd.  Workspace as ss_nf4_gemm_workspace_size.
 * Replace the projection + swiglu_fused_forward / swiglu_fused_backward pairs
 * of the frozen MLP node (solution/mlp.py:500-576). */
int ss_nf4_gemm_fwd_swiglu(const uint16_t* x, int64_t ldx, int64_t t, const uint8_t* packed,
                           const uint8_t* qabs, const float* absmax2, const float* code2,
                           const float* offset, int64_t n, int64_t k, const uint16_t* gate,
                           int64_t ldgate, uint16_t* up, int64_t ldup, uint16_t* act,
                           int64_t ldact, void* workspace, size_t workspace_bytes, void* stream);

int ss_nf4_gemm_dx_swiglu(const uint16_t* dy, int64_t lddy, int64_t t, const uint8_t* packed,
                          const uint8_t* qabs, const float* absmax2, const float* code2,
                          const float* offset, int64_t n, int64_t k, const uint16_t* gate,
                          int64_t ldgate, const uint16_t* up, int64_t ldup, uint16_t* dgate,
                          int64_t lddgate, uint16_t* dup, int64_t lddup, void* workspace,
                          size_t workspace_bytes, void* stream);

/* --------------------------------------------------------------- RoPE ---
 * Joint q/k rotary embedding.  q [B, Hq, S, D] and k [B, Hk, S, D] with
 * element strides (batch, head, token; last dimension 1 in the forward, qd /
 * kd for the gradients), cos / sin [c_batches (1 or B), S, D] of one dtype
 * with strides (batch, token) and last stride 1, half = D / 2.  Forward
 * y1 = R(x1 c1) + R(-x2 s1), y2 = R(x2 c2) + R(x1 s2), R = rounding to the
 * output dtype promote(x, cos); backward d1 = R'(g1 c1) + R'(g2 s2),
 * d2 = R'(g2 c2) - R'(g1 s1), R' = rounding to the input dtype.  Forward
 * outputs are contiguous [B, H, S, D]; the backward writes dq / dk with the
 * given element strides (batch, head, token; last dimension 1), e.g. the
 * layout of the forward's input views.  A NULL q (or k) operand is skipped.  Replace
 * rope_pair_forward_kernel / rope_pair_backward_kernel
 * (solution/kernels/rope.py:24-98) as launched by _RoPE (:101-144). */
int ss_rope_fwd(const void* q, int q_dtype, int64_t qb, int64_t qh, int64_t qt, const void* k,
                int k_dtype, int64_t kb, int64_t kh, int64_t kt, const void* cos,
                const void* sin, int cs_dtype, int64_t cb, int64_t ct, int64_t sb, int64_t st,
                int64_t c_batches, void* yq, int yq_dtype, void* yk, int yk_dtype,
                int64_t batches, int64_t qheads, int64_t kheads, int64_t tokens, int64_t half,
                void* stream);

int ss_rope_bwd(const void* gq, int gq_dtype, int64_t qb, int64_t qh, int64_t qt, int64_t qd,
                const void* gk, int gk_dtype, int64_t kb, int64_t kh, int64_t kt, int64_t kd,
                const void* cos, const void* sin, int cs_dtype, int64_t cb, int64_t ct,
                int64_t sb, int64_t st, int64_t c_batches, void* dq, int dq_dtype, int64_t dqb,
                int64_t dqh, int64_t dqt, void* dk, int dk_dtype, int64_t dkb, int64_t dkh,
                int64_t dkt, int64_t batches, int64_t qheads, int64_t kheads, int64_t tokens,
                int64_t half, void* stream);

/* ------------------------------------------------------------ SwiGLU ---
 * Qwen2 MLP activation on rows x cols matrices with independent row/column
 * strides (elements) and dtypes (SS_F16 / SS_F32), fp32 arithmetic:
 * p = 1/(1+exp(-g)), act = g*p; forward out = act*u; backward
 * dgate = (grad*u)*(p + act*(1-p)), dup = grad*act.  Empty extents are a
 * no-op.  Replace swiglu_tile_engine (solution/kernels/swiglu_fused.py:20-46)
 * as called by swiglu_fused_forward (:52-64) and swiglu_fused_backward
 * (:67-78). */
int ss_swiglu_fwd(const void* gate, int gate_dtype, int64_t g_rs, int64_t g_cs, const void* up,
                  int up_dtype, int64_t u_rs, int64_t u_cs, void* out, int out_dtype, int64_t o_rs,
                  int64_t o_cs, int64_t rows, int64_t cols, void* stream);

int ss_swiglu_bwd(const void* gate, int gate_dtype, int64_t g_rs, int64_t g_cs, const void* up,
                  int up_dtype, int64_t u_rs, int64_t u_cs, const void* grad, int grad_dtype,
                  int64_t d_rs, int64_t d_cs, void* dgate, int dgate_dtype, int64_t dg_rs,
                  int64_t dg_cs, void* dup, int dup_dtype, int64_t du_rs, int64_t du_cs,
                  int64_t rows, int64_t cols, void* stream);

/* ------------------------------------------------- add + RMSNorm (A13/14) ---
 * Row-wise over [rows, h] contiguous.  s = cast_s(r + d), rstd[row] =
 * rsqrt(mean(s^2) + eps), y = cast_y(w * cast_s(s * rstd)); s_dtype must be
 * promote(r_dtype, d_dtype); y_dtype is promote(s_dtype, w_dtype) or SS_F16.
 * Replaces add_rmsnorm_forward_kernel (solution/kernels/add_rmsnorm.py:37-51). */
int ss_add_rmsnorm_fwd(const void* r, int r_dtype, const void* d, int d_dtype, const void* w,
                       int w_dtype, int64_t w_stride, void* s, int s_dtype, void* y, int y_dtype,
                       float* rstd, int64_t rows, int64_t h, float eps, void* stream);

/* ds = cast_s(rstd*(u - a*mean(u*a))) + gs, a = s*rstd, u = cast_s(gy*w);
 * written to dr (dr_dtype) and/or dd (dd_dtype) (either may be NULL); gs or gy
 * may be NULL (absent upstream).  Strides are in elements.  Replaces
 * add_rmsnorm_backward_kernel (solution/kernels/add_rmsnorm.py:54-81). */
int ss_add_rmsnorm_bwd(const void* s, int s_dtype, const void* w, int w_dtype, int64_t w_stride,
                       const float* rstd, const void* gs, int gs_dtype, int64_t gs_row,
                       int64_t gs_col, const void* gy, int gy_dtype, int64_t gy_row,
                       int64_t gy_col, void* dr, int dr_dtype, void* dd, int dd_dtype,
                       int64_t rows, int64_t h, void* stream);

/* The backward of ss_add_rmsnorm_bwd and the weight gradient in one pass over
 * s and gy: dr / dd as there (either may be NULL) and
 * dgamma[c] = sum_rows gy * cast_s(s*rstd) (products rounded to fp16 when
 * half_products), summed per group of consecutive rows in fp32 into partial
 * fp32[ss_add_rmsnorm_dgamma_waves(rows), h] (caller-provided scratch, no
 * initialisation needed) and those sums added in group order (deterministic).
 * Replaces add_rmsnorm_backward_kernel followed by the two dgamma kernels
 * (solution/kernels/add_rmsnorm.py:54-81,123-135; rmsnorm.py:73-102). */
int64_t ss_add_rmsnorm_dgamma_waves(int64_t rows);
int ss_add_rmsnorm_bwd_dgamma(const void* s, int s_dtype, const void* w, int w_dtype,
                              int64_t w_stride, const float* rstd, const void* gs, int gs_dtype,
                              int64_t gs_row, int64_t gs_col, const void* gy, int gy_dtype,
                              int64_t gy_row, int64_t gy_col, void* dr, int dr_dtype, void* dd,
                              int dd_dtype, int half_products, float* partial, void* dw,
                              int dw_dtype, int64_t rows, int64_t h, void* stream);

/* Standalone Qwen2 RMSNorm forward (no residual): rstd = rsqrt(mean(fp32(x)^2)
 * + eps), y = w * cast_x(fp32(x) * rstd) in promote(x, w), or rounded to fp16
 * when y_dtype is SS_F16 (the fused output cast).  x rows have stride x_row
 * (elements, >= h), y is contiguous [rows, h], rstd fp32[rows].  The backward
 * is ss_add_rmsnorm_bwd / ss_add_rmsnorm_bwd_dgamma with s = x (contiguous)
 * and no residual gradient.  Replaces rmsnorm_forward_kernel
 * (solution/kernels/rmsnorm.py:42-53,108-125). */
int ss_rmsnorm_fwd(const void* x, int x_dtype, int64_t x_row, const void* w, int w_dtype,
                   int64_t w_stride, void* y, int y_dtype, float* rstd, int64_t rows, int64_t h,
                   float eps, void* stream);

/* dgamma[c] = sum_rows gy * cast_s(s*rstd) (products rounded to fp16 when
 * half_products), two-stage and non-atomic: partial fp32[ceil(rows/32), h]
 * is caller-provided scratch.  Replaces rmsnorm_weight_partials_kernel /
 * rmsnorm_weight_finalize_kernel (solution/kernels/rmsnorm.py:73-102). */
int ss_rmsnorm_dgamma(const void* s, int s_dtype, const float* rstd, const void* gy, int gy_dtype,
                      int64_t gy_row, int64_t gy_col, int half_products, float* partial,
                      void* dw, int dw_dtype, int64_t rows, int64_t h, void* stream);

/* ------------------------------------------------------------ unpad (A16) ---
 * Row copies of row_bytes bytes (any even number), bit-exact.
 * gather:  packed[t] = padded[indices[t]]        (solution/unpad.py:149-150);
 *          an index outside [0, padded_rows) yields a zero row.
 * scatter: padded[r] = 0 <= inverse[r] < tokens ? packed[inverse[r]] : 0
 *                                                 (solution/unpad.py:153-161)
 * inverse: inverse[r] = t where indices[t] == r, else -1 (int32[rows]);
 *          out-of-range indices are ignored. */
int ss_unpad_gather(const void* padded, int64_t padded_rows, void* packed,
                    const int64_t* indices, int64_t tokens, int64_t row_bytes, void* stream);
int ss_unpad_inverse(const int64_t* indices, int64_t tokens, int32_t* inverse, int64_t rows,
                     void* stream);
int ss_unpad_scatter(const void* packed, int64_t tokens, void* padded, const int32_t* inverse,
                     int64_t rows, int64_t row_bytes, void* stream);

/* ----------------------------------------------- fused linear CE (A17-19) ---
 * Vocabulary statistics of fp16 logits z[n, width] (row stride ldz) whose first
 * column is vocabulary index `start`, in pieces of `piece` columns (1..8192;
 * the last may be narrower): piece p of row r writes its partial state to slot
 * slot0 + p of row r of partial fp32[n, slots, 4] = (max m, sum exp(z - m),
 * sum exp(z - m) * z, target logit) and of partial_arg int64[n, slots] (first
 * argmax).  One call may cover any number of vocabulary chunks; the partial
 * row holds every piece of the vocabulary.  partial must be 16-byte aligned.
 * Replaces vocabulary_statistics_kernel (solution/kernels/cross_entropy.py:51-89),
 * whose per-chunk running state becomes one slot per piece, folded by
 * ss_ce_outputs. */
int ss_ce_stats(const uint16_t* z, int64_t ldz, const int64_t* targets, float* partial,
                int64_t* partial_arg, int64_t n, int64_t width, int64_t piece, int64_t start,
                int64_t slot0, int64_t slots, int64_t ignore_index, void* stream);

/* Folds each row's `slots` partial states in slot order (both sums rescaled to
 * the larger max; ties of the max keep the lower index) into max M, sum S, sum
 * T, target logit Z and argmax; then lse = M + log S, entropy = lse - T/S,
 * loss = lse - Z (0 when ignored), best = the first argmax (int64[n]).
 * Replaces vocabulary_outputs_kernel (cross_entropy.py:92-105). */
int ss_ce_outputs(const float* partial, const int64_t* partial_arg, int64_t slots,
                  const int64_t* targets, float* loss, float* entropy, float* lse,
                  int64_t* best, int64_t n, int64_t ignore_index, void* stream);

/* dz[r, c] = fp16((exp(z - lse[r]) - [start + c == target[r]]) * grad[r] / gain[r]),
 * gain[r] = max(|grad[r]|, 1e-30) / 1024 (zero on ignored rows); when dz_global
 * is not NULL it also receives the same derivative scaled by 1/global_gain
 * instead of 1/gain[r] (for the lm_head gradient; global_gain points at one
 * fp32 value > 0 in device memory).  dz is dense [n, width], dz_global dense
 * [global_rows, width] with rows n .. global_rows - 1 written as zeros
 * (global_rows = n without dz_global).  Row r of the logits is z[z_rows[r]]
 * when z_rows (int64 [n]) is not NULL, else z[r] (row stride ldz).  Replaces
 * vocabulary_derivative_kernel
 * (solution/kernels/cross_entropy.py:108-122). */
int ss_ce_derivative(const uint16_t* z, int64_t ldz, const int64_t* z_rows,
                     const int64_t* targets, const float* lse, const float* grad, uint16_t* dz,
                     uint16_t* dz_global, const float* global_gain, int64_t n,
                     int64_t global_rows, int64_t width, int64_t start, int64_t ignore_index,
                     void* stream);

/* Labelled rows of targets[n] and their validation, in one launch: order[0 ..
 * count) holds the rows whose target is not ignore_index, ascending (the
 * reference's row compaction before its backward), order[count .. order_len)
 * is -1 (order_len >= n: an index vector padded for ss_unpad_gather, which
 * writes a zero row for -1); count[0] = count (int64, device); ok[0] = 1 when
 * every target is ignore_index or in [0, vocab), else 0 (the reference's
 * "Target outside vocabulary" check, solution/kernels/cross_entropy.py:235-238,
 * read by a device-side assertion). */
int ss_ce_rows(const int64_t* targets, int64_t n, int64_t vocab, int64_t ignore_index,
               int64_t* order, int64_t order_len, int64_t* count, uint8_t* ok, void* stream);

/* gain[0] = max(max_r |grad[r]|, 1e-30) / 1024 over grad[n] (NaN if a grad is
 * NaN): the global gain of the lm_head gradient's derivative copy.  No
 * counterpart in the reference (its head is frozen); this build's weight_grad
 * extension. */
int ss_ce_head_gain(const float* grad, int64_t n, float* gain, void* stream);

/* out[r, :] = cast(acc[inverse[r], :] * max(|grad[r]|, 1e-30) / 1024) when
 * inverse[r] >= 0 (a valid row, compacted to position inverse[r]), else 0:
 * the dX rescale and scatter of solution/kernels/cross_entropy.py:205-210.
 * acc is fp32[valid_n, h]; grad fp32[n]; out_dtype SS_F16 or SS_F32. */
int ss_ce_finalize_dx(const float* acc, int64_t valid_n, const float* grad,
                      const int32_t* inverse, void* out, int out_dtype, int64_t n, int64_t h,
                      void* stream);

/* ------------------------------------------- causal attention, packed rows ---
 * Rows of the packed token axis are given by cu_seqlens (int32 [rows + 1] on
 * the device, cu[0] = 0, cu[rows] = total, nondecreasing); a query attends to
 * the keys of its own row at positions <= its own, softmax(scale q.k), GQA
 * (kv head = q head / (hq / hk)).  Replaces the per-row SDPA loop over a
 * packed batch (solution/unpad.py:359-410).  q [T, hq, 128], k / v
 * [T, hk, 128], o [T, hq, 128], fp16, each given as (base, token stride, head
 * stride) in elements with a unit last stride; bases 16-byte aligned, strides
 * multiples of 8.  max_len >= the longest row.  lse2 fp32 [hq, T] receives
 * m + log2(sum) of the base-2 scaled scores.  head_dim must be 128. */
int ss_attn_varlen_fwd(const void* q, int64_t q_tok, int64_t q_head, const void* k,
                       int64_t k_tok, int64_t k_head, const void* v, int64_t v_tok,
                       int64_t v_head, const int32_t* cu_seqlens, int rows, int max_len,
                       int64_t total, int hq, int hk, int head_dim, float scale, void* o,
                       int64_t o_tok, int64_t o_head, float* lse2, void* stream);

/* Scratch bytes of ss_attn_varlen_bwd: rowsum(dout . o) per (q head, token)
 * and, with GQA (hq > hk), the q heads' fp32 dK / dV partial planes. */
size_t ss_attn_varlen_bwd_workspace_size(int hq, int hk, int64_t total);

/* Backward of ss_attn_varlen_fwd: dq [T, hq, 128], dk / dv [T, hk, 128] fp16
 * (fully written; same base / stride rules as the inputs), from q, k, v, the
 * forward's o and lse2 and the upstream dout.  workspace: at least
 * ss_attn_varlen_bwd_workspace_size() bytes, 16-byte aligned, fully written
 * before it is read.  Deterministic: the GQA group's partials are added in
 * head order. */
int ss_attn_varlen_bwd(const void* q, int64_t q_tok, int64_t q_head, const void* k,
                       int64_t k_tok, int64_t k_head, const void* v, int64_t v_tok,
                       int64_t v_head, const void* o, int64_t o_tok, int64_t o_head,
                       const void* dout, int64_t do_tok, int64_t do_head, const float* lse2,
                       const int32_t* cu_seqlens, int rows, int max_len, int64_t total, int hq,
                       int hk, int head_dim, float scale, void* dq, int64_t dq_tok,
                       int64_t dq_head, void* dk, int64_t dk_tok, int64_t dk_head, void* dv,
                       int64_t dv_tok, int64_t dv_head, void* workspace, size_t workspace_bytes,
                       void* stream);

/* --------------------------------------- lossless fp16 table storage (f4) ---
 * dst[i] = fp16_rne(src[i]) for i < n, and *flag = 1 if any element does not
 * round-trip exactly ((float)dst[i] != src[i]; NaN never does).  *flag is
 * only ever set, never cleared: the caller zeroes it first and reads it
 * after the stream reaches this call.  Replaces the chunked copy-and-compare
 * of solution/embedding.py:51-64 (_lossless_candidate) with one pass.
 * Any alignment (16-byte aligned src / dst take the vector path). */
int ss_f32_to_f16_exact(const float* src, uint16_t* dst, int64_t n, int* flag, void* stream);

/* ------------------------------------------- HBM read ceiling (measurement) ---
 * No counterpart in the reference: a plain streaming read of `bytes` (a
 * multiple of 16, 16-byte aligned src) by `blocks` workgroups of 256 threads,
 * folded to one word per workgroup in sink[blocks].  bench.py times it on
 * weight-sized buffers to measure what a cold read costs on the board, the
 * yardstick for the weight-streaming NF4 kernels at small T. */
int ss_hbm_read_probe(const void* src, int64_t bytes, int64_t blocks, uint32_t* sink,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SOUPSUCK_AMD_H */
