// Tuning choices of the GEMM dispatch, fixed at build time.
//
// The shipped library reads no environment variables: every path choice is a
// function of the call's shapes and alignment and of the constants below,
// whose defaults are the measured best on MI355X.  An experiment build may
// override one with -DSS_TUNE_<NAME>=<value>; the default build never does.
#pragma once

// XCD-aware workgroup -> tile remap of the register-staged GEMM (1 on, 0 off).
#ifndef SS_TUNE_GEMM_REMAP
#define SS_TUNE_GEMM_REMAP 1
#endif
// Tile of the register-staged GEMM: 0 automatic, 1..4 = 64x64, 128x128,
// 256x128, 128x256.
#ifndef SS_TUNE_GEMM_TILE
#define SS_TUNE_GEMM_TILE 0
#endif
// Dense K-contiguous products on the direct-to-LDS NT kernel (1) or the
// register-staged kernel (0).
#ifndef SS_TUNE_GEMM_NT
#define SS_TUNE_GEMM_NT 1
#endif
// T from which the NF4 GEMM decodes W once into the workspace (decode-first).
#ifndef SS_TUNE_NF4_DECODE_FIRST_T
#define SS_TUNE_NF4_DECODE_FIRST_T 256
#endif
// Streaming small-T NF4 kernels (1 on, 0 off).
#ifndef SS_TUNE_NF4_STREAM
#define SS_TUNE_NF4_STREAM 1
#endif
// Fused NF4 GEMM: 0 off, 1 where measured faster, 2 wherever it applies.
#ifndef SS_TUNE_NF4_FUSED
#define SS_TUNE_NF4_FUSED 1
#endif
// Fused NF4 dX for 16 < T <= 256 (1 on, 0 off: decode-first there).
#ifndef SS_TUNE_NF4_DX_FUSED
#define SS_TUNE_NF4_DX_FUSED 1
#endif
// NT kernel configuration (0 automatic, 1..10) and split count (0 automatic).
#ifndef SS_TUNE_NT_TILE
#define SS_TUNE_NT_TILE 0
#endif
#ifndef SS_TUNE_NT_SPLITS
#define SS_TUNE_NT_SPLITS 0
#endif
// Ping-pong main loop of the 8-wave NT configurations (1 on, 0 lockstep).
#ifndef SS_TUNE_NT_PINGPONG
#define SS_TUNE_NT_PINGPONG 1
#endif
// fp16 epilogues staged through LDS with 16-byte row stores (1 on, 0 off).
#ifndef SS_TUNE_NT_STAGED
#define SS_TUNE_NT_STAGED 1
#endif
