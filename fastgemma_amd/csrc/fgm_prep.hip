// GEMM activation preamble on gfx950: copy, optional FWHT, per-row int8
// quantisation and A tile-packing -- the device side of fgm_prep_rows,
// fgm_quant_act, fgm_fwht and fgm_pack_a (ops.c:153-204, 279-314).
//
// One workgroup owns one activation row.  The row is staged in LDS, rotated
// there (every FWHT stage is one add or one subtract per element, so the
// parallel schedule gives the reference's bytes), reduced to its absolute
// maximum (order-free for non-NaN rows), then quantised and written to the
// row-major int8 copy and to its slots in the packed tiles.
#include "fgm_common.h"
#include "fgm_kernels.h"

namespace {

constexpr int PREP_THREADS = 256;

// Block-wide max of non-negative floats.
__device__ float block_max(float v, float* red) {
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float m = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); w++) m = fmaxf(m, red[w]);
  __syncthreads();
  return m;
}

// In-place normalised FWHT of the `k` floats in LDS, blocks of `hsz`
// (ops.c:153-175).  `scale` = 1/sqrtf(hsz) computed on the host; it is only
// applied for hsz >= 16, matching the reference's 16-wide scale loop.
__device__ void fwht_lds(float* buf, int k, int hsz, float scale) {
  const int half = k >> 1;
  for (int len = 1; len < hsz; len <<= 1) {
    for (int p = threadIdx.x; p < half; p += blockDim.x) {
      const int i = (p / len) * (len << 1) + (p % len);  // pairs never straddle a block
      const float u = buf[i], v = buf[i + len];
      buf[i] = u + v;
      buf[i + len] = u - v;
    }
    __syncthreads();
  }
  if (hsz >= 16) {
    for (int i = threadIdx.x; i < k; i += blockDim.x) buf[i] = buf[i] * scale;
    __syncthreads();
  }
}

// Packed-A byte offset of (row, col): [row/16][col/64][row%16][col%64].
__device__ __forceinline__ size_t pa_off(int row, int col, int KB) {
  return (((size_t)(row >> 4) * KB + (col >> 6)) * 16 + (row & 15)) * 64 + (col & 63);
}

// The problem a workgroup belongs to, chosen with uniform selects so the
// kernel-argument array is never indexed dynamically.
__device__ __forceinline__ PrepProb pick(const PrepBatch& bt) {
  const int b = blockIdx.x;
  PrepProb p = bt.p[0];
  if (bt.count > 1 && b >= bt.p[1].wg0) p = bt.p[1];
  if (bt.count > 2 && b >= bt.p[2].wg0) p = bt.p[2];
  if (bt.count > 3 && b >= bt.p[3].wg0) p = bt.p[3];
  return p;
}

__global__ __launch_bounds__(PREP_THREADS) void prep_rows_kernel(PrepBatch bt) {
  extern __shared__ float buf[];
  __shared__ float red[PREP_THREADS / 64];
  const PrepProb a = pick(bt);
  const int row = a.r0 + (blockIdx.x - a.wg0);
  const int k = a.k, KB = k >> 6;

  if (row >= a.r1) {
    // Rows of the last covered tile block beyond r1: zero padding when past m,
    // otherwise whatever the caller's qa row holds (ops.c:308-311).
    if (!a.pa) return;
    for (int c = threadIdx.x * 4; c < k; c += blockDim.x * 4) {
      int32_t v = 0;
      if (row < a.m) {
        const int8_t* q = a.qa + (size_t)row * k + c;
        v = (int32_t)((uint32_t)(uint8_t)q[0] | (uint32_t)(uint8_t)q[1] << 8 |
                      (uint32_t)(uint8_t)q[2] << 16 | (uint32_t)(uint8_t)q[3] << 24);
      }
      *(int32_t*)(a.pa + pa_off(row, c, KB)) = v;
    }
    return;
  }

  // Stage the row in LDS: eight loads in flight per thread before any store.
  // Lanes past the row's end read 0 through the buffer range check.
  const float* src = a.src + (size_t)row * a.lda;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(src, (uint32_t)k * 4);
  if ((((uintptr_t)src) & 15) == 0 && (k & 3) == 0) {
    const int k4 = k >> 2;
    for (int base = 0; base < k4; base += PREP_THREADS * 8) {
      v4i v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int c = base + (int)threadIdx.x + u * PREP_THREADS;
        v[u] = buf_load_b128(rs, c < k4 ? (uint32_t)c * 16 : FGM_OOB, 0);
      }
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int c = base + (int)threadIdx.x + u * PREP_THREADS;
        if (c < k4) *(v4i*)(buf + 4 * c) = v[u];
      }
    }
  } else {
    for (int base = 0; base < k; base += PREP_THREADS * 8) {
      int32_t v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int c = base + (int)threadIdx.x + u * PREP_THREADS;
        v[u] = buf_load_b32(rs, c < k ? (uint32_t)c * 4 : FGM_OOB, 0);
      }
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int c = base + (int)threadIdx.x + u * PREP_THREADS;
        if (c < k) buf[c] = __int_as_float(v[u]);
      }
    }
  }
  __syncthreads();
  if (a.hsz > 0) fwht_lds(buf, k, a.hsz, a.fwht_scale);

  float mx = 0.0f;
  for (int i = threadIdx.x; i < k; i += blockDim.x) mx = fmaxf(mx, __builtin_fabsf(buf[i]));
  mx = block_max(mx, red);
  const float s = (mx == 0.0f) ? 1.0f : mx / 127.0f;
  const float inv = 1.0f / s;
  if (threadIdx.x == 0) a.qs[row] = s;

  const int kv = k & ~15;
  float* rot = a.rot ? a.rot + (size_t)row * k : nullptr;
  int8_t* qa = a.qa ? a.qa + (size_t)row * k : nullptr;
  // four consecutive columns per thread: one dword store to qa and to pa
  for (int c = threadIdx.x * 4; c < k; c += blockDim.x * 4) {
    uint32_t packed = 0;
    for (int e = 0; e < 4 && c + e < k; e++) {
      const float x = buf[c + e];
      if (rot) rot[c + e] = x;
      const float v = x * inv;
      const int8_t q = (c + e < kv) ? quant_vec(v) : quant_tail(v);
      packed |= (uint32_t)(uint8_t)q << (8 * e);
      if (qa) qa[c + e] = q;
    }
    if (a.pa) *(uint32_t*)(a.pa + pa_off(row, c, KB)) = packed;
  }
}

// fgm_pack_a (ops.c:279-290), 16 bytes per thread.
__global__ void pack_a_kernel(int M, int K, const int8_t* __restrict__ A, int8_t* __restrict__ Ap,
                              size_t n16) {
  const size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= n16) return;
  const int KB = K >> 6;
  const size_t tile_row = o >> 2;  // 64-byte row of a tile
  const int c16 = (int)(o & 3);
  const int r = (int)(tile_row & 15);
  const size_t t = tile_row >> 4;  // (mb * KB + kb)
  const int kb = (int)(t % KB);
  const int mb = (int)(t / KB);
  const int m = mb * 16 + r;
  uint4 v = make_uint4(0, 0, 0, 0);
  if (m < M) {
    const int8_t* s = A + (size_t)m * K + kb * 64 + c16 * 16;
    uint32_t w[4];
    for (int q = 0; q < 4; q++)
      w[q] = (uint32_t)(uint8_t)s[4 * q] | (uint32_t)(uint8_t)s[4 * q + 1] << 8 |
             (uint32_t)(uint8_t)s[4 * q + 2] << 16 | (uint32_t)(uint8_t)s[4 * q + 3] << 24;
    v = make_uint4(w[0], w[1], w[2], w[3]);
  }
  *(uint4*)(Ap + o * 16) = v;
}

// fgm_fwht on a flat array: one workgroup per `chunk` floats (whole blocks).
__global__ __launch_bounds__(PREP_THREADS) void fwht_kernel(float* x, int chunk, int hsz,
                                                            float scale) {
  extern __shared__ float buf[];
  float* p = x + (size_t)blockIdx.x * chunk;
  for (int i = threadIdx.x; i < chunk; i += blockDim.x) buf[i] = p[i];
  __syncthreads();
  fwht_lds(buf, chunk, hsz, scale);
  for (int i = threadIdx.x; i < chunk; i += blockDim.x) p[i] = buf[i];
}

}  // namespace

// ---------------------------------------------------------------- launchers
// Shapes are validated by the caller (fgm_api.hip).

// Rows are staged whole in LDS; allow the kernels the full 160 KB.
template <typename K>
static hipError_t allow_big_lds(K kernel) {
  return hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                             160 * 1024 - 1024);
}

hipError_t fgm_launch_prep(const PrepBatch& in, hipStream_t st) {
  static hipError_t attr = allow_big_lds(prep_rows_kernel);
  if (attr != hipSuccess) return attr;
  PrepBatch b = in;
  int nwg = 0, kmax = 0;
  for (int i = 0; i < b.count; i++) {
    PrepProb& p = b.p[i];
    p.wg0 = nwg;
    if (p.r0 < p.r1) {
      // rows [r0, r1) compute; rows [r1, end of r1's tile block) only pack
      const int end = p.pa ? ((p.r1 + 15) / 16) * 16 : p.r1;
      nwg += end - p.r0;
    }
    if (p.k > kmax) kmax = p.k;
  }
  if (nwg == 0) return hipSuccess;
  hipLaunchKernelGGL(prep_rows_kernel, dim3(nwg), dim3(PREP_THREADS), (size_t)kmax * sizeof(float),
                     st, b);
  return hipGetLastError();
}

hipError_t fgm_launch_pack_a(int M, int K, const int8_t* A, int8_t* Ap, hipStream_t st) {
  const size_t n16 = (size_t)((M + 15) / 16) * 16 * K / 16;
  if (!n16) return hipSuccess;
  hipLaunchKernelGGL(pack_a_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, st, M, K,
                     A, Ap, n16);
  return hipGetLastError();
}

hipError_t fgm_launch_fwht(float* x, int n, int hsz, float scale, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  static hipError_t attr = allow_big_lds(fwht_kernel);
  if (attr != hipSuccess) return attr;
  int chunk = hsz;
  while (chunk < 2048 && n % (chunk * 2) == 0) chunk *= 2;
  hipLaunchKernelGGL(fwht_kernel, dim3(n / chunk), dim3(PREP_THREADS),
                     (size_t)chunk * sizeof(float), st, x, chunk, hsz, scale);
  return hipGetLastError();
}
