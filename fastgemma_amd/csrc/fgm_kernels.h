// Internal launcher interface between the C-ABI layer (fgm_api.hip) and the
// kernels.  All pointers are device pointers; shapes are validated by the
// caller before any launch.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

// Independent problems served by one launch.
constexpr int FGM_MAX_BATCH = 4;

struct GemmProb {
  const int8_t* A;        // packed A [ceil(M/16)][K/64][16][64]
  const float* a_scale;   // [M]
  const void* B;          // int8 tiles, or packed int4 tiles
  const void* b_scale;    // f32 [N] (q8c) or f16 bits [K/group][N] (q4g)
  float* C;
  int32_t* acc_out;       // raw int32 accumulators instead of C when non-null
  int M, N, K, group, ldc, ldacc;
  int n0, nblocks;        // n-block range [n0, n0 + nblocks)
  int wg0;                // first workgroup of this problem (set by the launcher)
  int tw, ks, nbw;        // skinny path: k-blocks per wave, waves per n-block,
                          // n-blocks per workgroup (set by the launcher)
};

struct GemmBatch {
  GemmProb p[FGM_MAX_BATCH];
  int count;
};

struct PrepProb {
  const float* src;
  float* rot;      // may be null (device API only)
  int8_t* qa;      // may be null (device API only)
  float* qs;
  int8_t* pa;      // null for quant_act
  int lda, m, k, hsz, r0, r1;
  float fwht_scale;
  int wg0;         // first workgroup (set by the launcher)
};

struct PrepBatch {
  PrepProb p[FGM_MAX_BATCH];
  int count;
};

hipError_t fgm_launch_prep(const PrepBatch& b, hipStream_t st);
hipError_t fgm_launch_pack_a(int M, int K, const int8_t* A, int8_t* Ap, hipStream_t st);
hipError_t fgm_launch_fwht(float* x, int n, int hsz, float scale, hipStream_t st);

// Skinny weight-stream path, M <= 64 (all problems of a batch share the
// weight type and are served by one launch).
bool fgm_decode_fits(int bits, int M, int K, int group);
size_t fgm_decode_lds_bytes(int bits, int M, int K, int group);
hipError_t fgm_launch_decode(int bits, const GemmBatch& b, hipStream_t st);

// Dense MFMA path (any M).
hipError_t fgm_launch_gemm(int bits, const GemmBatch& b, hipStream_t st);

// f32 elementwise primitives (fgm_elem.hip).  rows x n contiguous rows for
// rmsnorm (w NULL: no scale); gelu: up NULL for in-place gelu (out may be
// gate); rope: cs [rows][head_dim / 2][2] (cos, sin); binop: 0 add, 1 mul,
// 2 scale by s.
hipError_t fgm_launch_rmsnorm(float* out, const float* x, const float* w, int rows, int n, float eps,
                              hipStream_t st);
hipError_t fgm_launch_gelu(float* out, const float* gate, const float* up, int n, hipStream_t st);
hipError_t fgm_launch_softcap(float* x, int n, float cap, hipStream_t st);
hipError_t fgm_launch_rope(float* x, int rows, int n_heads, int head_dim, const float* cs, hipStream_t st);
hipError_t fgm_launch_binop(float* a, const float* b, int n, int op, float s, hipStream_t st);
