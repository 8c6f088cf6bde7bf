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
//   fgm_ceil_gridbar  a device-wide barrier between dependent steps inside one
//                   cooperative launch (what a persistent decode kernel would
//                   pay per dependent GEMM instead of a kernel boundary), with
//                   the 2 KB per workgroup a decode GEMM hands on
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

// Device-wide barrier variants (one wave per workgroup arrives; the others
// wait at the workgroup barrier).  Each iteration every workgroup writes 2 KB
// (512 floats, as a decode GEMM's 8 x 64 output slice), crosses the barrier
// and reads the 2 KB another workgroup wrote, counting stale values.
//   0: agent-scope release fence, acq_rel arrival, every poll an agent-scope
//      acquire load
//   1: agent-scope release fence, relaxed arrival, relaxed polls, one
//      agent-scope acquire fence after the poll
//   2: as 1, the 2 KB stored non-temporally (streamed past the L2)
//   3: relaxed arrival and polls, no fences (the atomic round trip alone;
//      the data may be stale, which the count shows)
//   4: hierarchical: workgroup b arrives at group counter b % 8 (the XCD it
//      is dispatched to when workgroups go round-robin over the eight XCDs),
//      the group's last arriver takes one agent-scope release fence for the
//      group and arrives at the top counter; relaxed polls, one agent-scope
//      acquire fence per workgroup after them
//   5: as 4 without fences (the hierarchical atomics alone)
// Spins are bounded: past the limit the workgroup raises bar[2] and every
// later barrier is skipped, so the grid always drains.
struct GridBar {
  uint32_t count, gen, err, pad[29];
  uint32_t grp[8][32];  // variants 4-5: group counters, one 128-byte line each
};

template <int V>
FGM_DEV void grid_barrier(GridBar* b, uint32_t nwg, uint32_t spin_limit) {
  if constexpr (V >= 4) {
    __syncthreads();
    if (threadIdx.x == 0 && !__hip_atomic_load(&b->err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
      const uint32_t grp = blockIdx.x & 7, ngrp = nwg < 8 ? nwg : 8;
      const uint32_t members = nwg / 8 + (grp < nwg % 8 ? 1u : 0u);
      const uint32_t g = __hip_atomic_load(&b->gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t a = __hip_atomic_fetch_add(&b->grp[grp][0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      bool last = false;
      if (a == members - 1) {
        __hip_atomic_store(&b->grp[grp][0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (V == 4) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        last = __hip_atomic_fetch_add(&b->count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ngrp - 1;
      }
      if (last) {
        __hip_atomic_store(&b->count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&b->gen, g + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        uint32_t spins = 0;
        while (__hip_atomic_load(&b->gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == g) {
          if (++spins > spin_limit) {
            __hip_atomic_store(&b->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
          }
        }
      }
      if (V == 4) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    return;
  }
  __syncthreads();
  if (threadIdx.x == 0 && !__hip_atomic_load(&b->err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
    if (V != 3) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    const uint32_t g = __hip_atomic_load(&b->gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t arrived = V == 0 ? __hip_atomic_fetch_add(&b->count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT)
                                    : __hip_atomic_fetch_add(&b->count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (arrived == nwg - 1) {
      __hip_atomic_store(&b->count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&b->gen, g + 1, V == 0 ? __ATOMIC_RELEASE : __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      uint32_t spins = 0;
      while ((V == 0 ? __hip_atomic_load(&b->gen, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT)
                     : __hip_atomic_load(&b->gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) == g) {
        if (++spins > spin_limit) {
          __hip_atomic_store(&b->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
      }
    }
    if (V == 1 || V == 2) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
}

template <int V>
__global__ __launch_bounds__(256) void gridbar_kernel(GridBar* b, float* buf, int iters, uint32_t spin_limit,
                                                      uint32_t* stale) {
  const uint32_t nwg = gridDim.x, wg = blockIdx.x, t = threadIdx.x;
  uint32_t bad = 0;
  for (int i = 0; i < iters; i++) {
    float* mine = buf + ((size_t)(i & 1) * nwg + wg) * 512;
    const float v = (float)(i * 4096 + (int)wg);
    if (V == 2) {
      __builtin_nontemporal_store(v, mine + t);
      __builtin_nontemporal_store(v, mine + 256 + t);
    } else {
      mine[t] = v;
      mine[256 + t] = v;
    }
    grid_barrier<V>(b, nwg, spin_limit);
    const uint32_t o = (wg + 1) % nwg;
    const float* other = buf + ((size_t)(i & 1) * nwg + o) * 512;
    const float want = (float)(i * 4096 + (int)o);
    bad += (other[t] != want) + (other[256 + t] != want);
  }
  if (bad) atomicAdd(stale, bad);
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

// Cooperative launch of nwg workgroups (256 threads) running `iters`
// barriers of variant v (0 .. 5).  bar: fgm_ceil_gridbar_bytes() bytes, zeroed
// by the caller before each launch (word 2 is set when a spin limit was hit);
// buf: 2 x nwg x 512 floats; stale: one word (stale reads are added).
// Returns 0, 1 for bad arguments, 2 for a failed launch.
size_t fgm_ceil_gridbar_bytes(void) { return sizeof(GridBar); }

int fgm_ceil_gridbar(int v, int nwg, int iters, void* bar, float* buf, uint32_t* stale, void* stream) {
  if (v < 0 || v > 5 || nwg < 1 || iters < 1 || !bar || !buf || !stale) return 1;
  const uint32_t spin_limit = 1u << 20;
  GridBar* b = (GridBar*)bar;
  void* args[] = {&b, &buf, &iters, (void*)&spin_limit, &stale};
  const void* k = v == 0 ? (const void*)gridbar_kernel<0>
                : v == 1 ? (const void*)gridbar_kernel<1>
                : v == 2 ? (const void*)gridbar_kernel<2>
                : v == 3 ? (const void*)gridbar_kernel<3>
                : v == 4 ? (const void*)gridbar_kernel<4>
                         : (const void*)gridbar_kernel<5>;
  hipError_t e = hipLaunchCooperativeKernel(k, dim3(nwg), dim3(256), args, 0, (hipStream_t)stream);
  return e == hipSuccess ? 0 : 2;
}

}  // extern "C"
