// Internal launcher interface between the C-ABI layer (fgm_api.hip) and the
// kernels.  All pointers are device pointers; shapes are validated by the
// caller before any launch.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

struct GemmArgs {
  int M, N, K;
  const int8_t* A;        // packed A [ceil(M/16)][K/64][16][64]
  const float* a_scale;   // [M]
  const void* B;          // int8 tiles, or packed int4 tiles
  const void* b_scale;    // f32 [N] (q8c) or f16 bits [K/group][N] (q4g)
  int group;              // q4g only
  float* C;
  int ldc;
  int n0;                 // first n-block; blockIdx enumerates [n0, n1)
  int32_t* acc_out;       // raw int32 accumulators instead of C when non-null
  int ldacc;
};

hipError_t fgm_launch_prep_rows(const float* src, int lda, float* rot, int8_t* qa, float* qs,
                                int8_t* pa, int m, int k, int hsz, int r0, int r1,
                                float fwht_scale, hipStream_t st);
hipError_t fgm_launch_pack_a(int M, int K, const int8_t* A, int8_t* Ap, hipStream_t st);
hipError_t fgm_launch_fwht(float* x, int n, int hsz, float scale, hipStream_t st);

// Skinny path, M <= 64.  nblocks = n1 - n0 workgroups.
hipError_t fgm_launch_decode(int bits, const GemmArgs& a, int nblocks, hipStream_t st);
size_t fgm_decode_lds_bytes(int bits, int M, int K, int group);

// Dense MFMA path (any M).
hipError_t fgm_launch_gemm(int bits, const GemmArgs& a, int nblocks, hipStream_t st);
