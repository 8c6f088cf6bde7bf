// Ceiling probes for the measurements: the floors the roofline fractions and
// the traffic calibration are read against, measured on the box that runs the
// benchmark.  Built into libfgm_ceil.so, apart from the product library.
//
//   fgm_ceil_empty  a launch that does nothing: the back-to-back launch floor
//   fgm_ceil_read   a pure read of `bytes`: 16-byte non-temporal loads, one
//                   contiguous chunk per workgroup, the words xor-folded so
//                   no load is dead
//   fgm_ceil_read_lds  the same read on the skinny GEMM's path: 1 KB
//                   LDS-DMA units, up to 16 waves per workgroup
//   fgm_ceil_copy   a plain copy of `bytes`, 16 bytes per lane and load: the
//                   kernel whose FETCH_SIZE / WRITE_SIZE counters calibrate the
//                   traffic figures (its algorithmic bytes are known exactly)
//   fgm_ceil_mfma   independent int8 MFMA chains on every SIMD: the dense int8
//                   peak (v_mfma_i32_32x32x32_i8 or v_mfma_i32_16x16x64_i8)
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fgm_common.h"

namespace {

__global__ __launch_bounds__(1024) void empty_kernel(int* sink) {
  if (sink && threadIdx.x == 0 && blockIdx.x == 0x7FFFFFFF) sink[0] = 1;
}

// Workgroup b reads chunk b: 256 threads x 16 bytes x U contiguous bytes, all
// U loads of a thread in flight at once (one chunk per workgroup, so every
// workgroup does the same work).  The loaded words only feed a store that
// (practically) never happens, so the measured path has no reduction tail.
template <int U>
__global__ __launch_bounds__(256) void read_kernel(const char* p, uint32_t* sink) {
  constexpr uint32_t chunk = 256u * 16u * U;
  const __amdgpu_buffer_rsrc_t r = make_rsrc(p + (size_t)blockIdx.x * chunk, chunk);
  v4i v[U];
#pragma unroll
  for (int u = 0; u < U; u++)
    v[u] = __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)(u * 4096 + threadIdx.x * 16), 0, 2);
  v4i x = v[0];
#pragma unroll
  for (int u = 1; u < U; u++) x ^= v[u];
  // a store that depends on every load and (practically) never happens: no
  // reduction tail on the measured path
  const uint32_t f = (uint32_t)(x[0] ^ x[1] ^ x[2] ^ x[3]);
  if (f == 0x9E3779B9u) sink[blockIdx.x] = f;
}

// The decode kernel's access path without its arithmetic: NW waves per
// workgroup, each moving U 1 KB units straight into LDS with 16-byte
// non-temporal buffer loads (buffer_load_dwordx4 ... lds), all in flight at
// once; workgroup b reads bytes [b NW U KB, (b + 1) NW U KB).  One LDS word
// per lane and unit feeds a store that (practically) never happens, so no
// load is dead and there is no reduction tail.
template <int U>
__global__ __launch_bounds__(1024) void read_lds_kernel(const char* p, uint32_t* sink) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int w = wave_id(), l = threadIdx.x & 63, nw = blockDim.x >> 6;
  const size_t wg_bytes = (size_t)nw * U * 1024;
  const v4i rs = rsrc_words(p + (size_t)blockIdx.x * wg_bytes, (uint32_t)wg_bytes);
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem + (uint32_t)w * U * 1024;
#pragma unroll
  for (int u = 0; u < U; u++) dma16<true>(rs, lds0 + u * 1024, 16u * l, (uint32_t)(w * U + u) * 1024u);
  wait_vm<0>();
  uint32_t x = 0;
#pragma unroll
  for (int u = 0; u < U; u++) x ^= *(const uint32_t*)(smem + (size_t)(w * U + u) * 1024 + 16 * l);
  if (x == 0x9E3779B9u) sink[blockIdx.x] = x;
}

__global__ __launch_bounds__(256) void copy_kernel(const char* src, char* dst, size_t bytes) {
  const size_t n16 = bytes / 16;
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride)
    ((v4i*)dst)[i] = ((const v4i*)src)[i];
}

typedef int v16i __attribute__((ext_vector_type(16)));

// CH independent accumulator chains per wave, `iters` rounds; the operands
// are loop-invariant registers, so the loop is MFMA issue only.
template <bool BIG>
__global__ __launch_bounds__(256) void mfma_kernel(int iters, int* sink) {
  constexpr int CH = 4;
  const v4i a = v4i{(int)threadIdx.x, 3, 5, 7}, b = v4i{11, (int)blockIdx.x, 13, 17};
  if constexpr (BIG) {
    v16i acc[CH];
#pragma unroll
    for (int c = 0; c < CH; c++) acc[c] = v16i{};
    for (int i = 0; i < iters; i++)
#pragma unroll
      for (int c = 0; c < CH; c++) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[c], 0, 0, 0);
    int s = 0;
#pragma unroll
    for (int c = 0; c < CH; c++)
#pragma unroll
      for (int r = 0; r < 16; r++) s ^= acc[c][r];
    if (s == 0x13572468) sink[blockIdx.x] = s;
  } else {
    v4i acc[CH];
#pragma unroll
    for (int c = 0; c < CH; c++) acc[c] = v4i{};
    for (int i = 0; i < iters; i++)
#pragma unroll
      for (int c = 0; c < CH; c++) acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[c], 0, 0, 0);
    int s = 0;
#pragma unroll
    for (int c = 0; c < CH; c++)
#pragma unroll
      for (int r = 0; r < 4; r++) s ^= acc[c][r];
    if (s == 0x13572468) sink[blockIdx.x] = s;
  }
}

}  // namespace

extern "C" {

int fgm_ceil_empty(int nwg, int threads, void* stream) {
  if (nwg < 1 || threads < 64 || threads > 1024 || threads % 64) return 1;
  hipLaunchKernelGGL(empty_kernel, dim3(nwg), dim3(threads), 0, (hipStream_t)stream, nullptr);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// u in {1, 2, 4, 8}: chunks of 4 KiB x u, one workgroup each; bytes a
// multiple of the chunk; sink: one word per workgroup
int fgm_ceil_read(const void* p, size_t bytes, int u, uint32_t* sink, void* stream) {
  const size_t chunk = (size_t)4096 * u;
  if (!p || !sink || (u != 1 && u != 2 && u != 4 && u != 8) || bytes % chunk || bytes / chunk > 0x7FFFFFFF) return 1;
  const dim3 g((unsigned)(bytes / chunk));
  hipStream_t st = (hipStream_t)stream;
  switch (u) {
    case 1: hipLaunchKernelGGL(read_kernel<1>, g, dim3(256), 0, st, (const char*)p, sink); break;
    case 2: hipLaunchKernelGGL(read_kernel<2>, g, dim3(256), 0, st, (const char*)p, sink); break;
    case 4: hipLaunchKernelGGL(read_kernel<4>, g, dim3(256), 0, st, (const char*)p, sink); break;
    default: hipLaunchKernelGGL(read_kernel<8>, g, dim3(256), 0, st, (const char*)p, sink); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// nw waves x u KB per workgroup (u in {1, 2, 4, 8}, nw <= 16), one
// workgroup per nw u KB of `bytes` (a multiple of it); sink: one word per
// workgroup
int fgm_ceil_read_lds(const void* p, size_t bytes, int nw, int u, uint32_t* sink, void* stream) {
  const size_t wg = (size_t)nw * u * 1024;
  if (!p || !sink || nw < 1 || nw > 16 || (u != 1 && u != 2 && u != 4 && u != 8) || bytes % wg ||
      bytes / wg > 0x7FFFFFFF)
    return 1;
  const dim3 g((unsigned)(bytes / wg)), b((unsigned)nw * 64);
  hipStream_t st = (hipStream_t)stream;
  static const hipError_t attr[4] = {
      hipFuncSetAttribute((const void*)read_lds_kernel<1>, hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024),
      hipFuncSetAttribute((const void*)read_lds_kernel<2>, hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024),
      hipFuncSetAttribute((const void*)read_lds_kernel<4>, hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024),
      hipFuncSetAttribute((const void*)read_lds_kernel<8>, hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024)};
  for (hipError_t e : attr)
    if (e != hipSuccess) return 2;
  switch (u) {
    case 1: hipLaunchKernelGGL(read_lds_kernel<1>, g, b, wg, st, (const char*)p, sink); break;
    case 2: hipLaunchKernelGGL(read_lds_kernel<2>, g, b, wg, st, (const char*)p, sink); break;
    case 4: hipLaunchKernelGGL(read_lds_kernel<4>, g, b, wg, st, (const char*)p, sink); break;
    default: hipLaunchKernelGGL(read_lds_kernel<8>, g, b, wg, st, (const char*)p, sink); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// bytes: a multiple of 16
int fgm_ceil_copy(const void* src, void* dst, size_t bytes, int nwg, void* stream) {
  if (!src || !dst || nwg < 1 || bytes % 16) return 1;
  hipLaunchKernelGGL(copy_kernel, dim3(nwg), dim3(256), 0, (hipStream_t)stream, (const char*)src, (char*)dst,
                     bytes);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// shape 32: v_mfma_i32_32x32x32_i8 (65,536 ops each); 16: v_mfma_i32_16x16x64_i8
// (32,768 ops).  Ops of one launch: nwg x 4 waves x iters x 4 chains x ops.
int fgm_ceil_mfma(int shape, int nwg, int iters, int* sink, void* stream) {
  if ((shape != 32 && shape != 16) || nwg < 1 || iters < 1 || !sink) return 1;
  if (shape == 32)
    hipLaunchKernelGGL(mfma_kernel<true>, dim3(nwg), dim3(256), 0, (hipStream_t)stream, iters, sink);
  else
    hipLaunchKernelGGL(mfma_kernel<false>, dim3(nwg), dim3(256), 0, (hipStream_t)stream, iters, sink);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
