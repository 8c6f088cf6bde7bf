// The forward pass's f32 elementwise primitives on gfx950: rmsnorm (with and
// without scale), gelu / gelu_mul, rope, add / mul / scale and softcap -- the
// device side of ops.c:15-147, 316-351, keeping activations on the GPU
// between GEMMs.
//
// Every function reproduces the reference's floating-point operations in the
// reference's order, element for element:
//   * the reference processes 16 floats per AVX-512 vector and a scalar tail;
//     the vector part's exp (exp512_ps, ops.c:21-39) is a Cephes polynomial of
//     IEEE operations and is restated exactly (exp16 below);
//   * rmsnorm's sum of squares is 16 lane accumulators (lane j takes
//     x[16 t + j] by fma in ascending t), reduced by GCC's
//     _mm512_reduce_add_ps tree, then the tail by fma (GCC fuses it);
//     division and square root are correctly rounded here as on the CPU;
//   * rope takes its (cos, sin) pairs from the host, computed with the host's
//     libm exactly as ops.c:138-139 does (fgm_hip_rope_table);
//   * the scalar tails of gelu and softcap call libm's tanhf on the CPU (not
//     correctly rounded in glibc 2.35); here tanh is evaluated in double and
//     rounded once, so the tails agree to libm's own error (a few ulp of
//     tanh; these tails only exist when n % 16 != 0, which no model
//     dimension is).
#include <algorithm>

#include "fgm_common.h"
#include "fgm_kernels.h"

namespace {

// --------------------------------------------------------------- rmsnorm
// One workgroup per row; the row's latency is the whole cost at the forward
// pass's sizes, so the steps are arranged to overlap:
//  * every thread loads its share of x and w into registers at the start
//    (w does not wait for the norm);
//  * x is staged in LDS transposed, x[16 t + j] at lds[j * S + t] with
//    S = 4 (mod 64) and S >= n / 16 + 16: accumulator j's operands are contiguous (128-bit reads)
//    and the 16 chains read 64 distinct banks, the staging writes too;
//  * lanes 0..15 of wave 0 run the reference's 16 accumulators, reading four
//    128-bit words ahead of the fmas; GCC's reduce tree runs on DPP row
//    rotations (a + b == b + a exactly, so the tree's pairing is all that
//    matters); lane 0 adds the tail by fma and finishes;
//  * every thread writes (x * inv) * w (or x * inv) from its registers.
// The variant for n % 4 != 0 or unaligned rows keeps nothing in registers:
// x goes straight to LDS and w is read at the end.
constexpr int RMS_MAXV = 8;  // float4 slots per thread (n <= 32 T)

template <bool VEC>
__global__ __launch_bounds__(1024) void rmsnorm_kernel(float* out, const float* x, const float* w, int n, int S,
                                                       float eps) {
  extern __shared__ float lds[];  // [16][S] transposed row, then inv
  const int tid = threadIdx.x, T = blockDim.x;
  const float* xr = x + (size_t)blockIdx.x * n;
  float* orow = out + (size_t)blockIdx.x * n;
  // register slot 4 v + e holds element idx(v, e) (VEC variant)
  auto idx = [&](int v, int e) { return 4 * (tid + T * v) + e; };
  float xv[4 * RMS_MAXV], wv[4 * RMS_MAXV];
#pragma unroll
  for (int v = 0; v < RMS_MAXV; v++) {
    if (VEC) {
      const int i = idx(v, 0);
      if (i < n) {
        const float4 a = *(const float4*)(xr + i);
        xv[4 * v] = a.x, xv[4 * v + 1] = a.y, xv[4 * v + 2] = a.z, xv[4 * v + 3] = a.w;
        if (w) {
          const float4 b = *(const float4*)(w + i);
          wv[4 * v] = b.x, wv[4 * v + 1] = b.y, wv[4 * v + 2] = b.z, wv[4 * v + 3] = b.w;
        }
      }
    }
  }
  if (!VEC) {  // x goes straight to LDS, w is read at the end
#pragma unroll 1
    for (int i = tid; i < n; i += T) lds[(i & 15) * S + (i >> 4)] = xr[i];
  }
  if (VEC) {
#pragma unroll
    for (int v = 0; v < RMS_MAXV; v++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int i = idx(v, e);
        if (i < n) lds[(i & 15) * S + (i >> 4)] = xv[4 * v + e];
      }
  }
  __syncthreads();
  if (tid < 16) {
    float ss = rms_sumsq16(lds + tid * S, n >> 4);
    if (tid == 0) {
      for (int i = n & ~15; i < n; i++) {
        const float v = lds[(i & 15) * S + (i >> 4)];
        ss = __builtin_fmaf(v, v, ss);
      }
      lds[16 * S] = 1.0f / __builtin_sqrtf(ss / (float)n + eps);
    }
  }
  __syncthreads();
  const float inv = lds[16 * S];
#pragma unroll
  for (int v = 0; v < RMS_MAXV; v++) {
    if (VEC) {
      const int i = idx(v, 0);
      if (i < n) {
        float4 o;
        if (w) {
          o = float4{(xv[4 * v] * inv) * wv[4 * v], (xv[4 * v + 1] * inv) * wv[4 * v + 1],
                     (xv[4 * v + 2] * inv) * wv[4 * v + 2], (xv[4 * v + 3] * inv) * wv[4 * v + 3]};
        } else {
          o = float4{xv[4 * v] * inv, xv[4 * v + 1] * inv, xv[4 * v + 2] * inv, xv[4 * v + 3] * inv};
        }
        *(float4*)(orow + i) = o;
      }
    }
  }
  if (!VEC) {
#pragma unroll 1
    for (int i = tid; i < n; i += T) {
      const float xi = lds[(i & 15) * S + (i >> 4)];
      orow[i] = w ? (xi * inv) * w[i] : xi * inv;
    }
  }
}

// ------------------------------------------------------- gelu, softcap
// One element per thread; elements below n & ~15 take the vector form.
__global__ __launch_bounds__(256) void gelu_kernel(float* out, const float* gate, const float* up, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float g = gate[i];
  const float y = i < (n & ~15) ? gelu_vec(g) : gelu_tail(g);
  out[i] = up ? y * up[i] : y;
}

__global__ __launch_bounds__(256) void softcap_kernel(float* x, int n, float cap) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  if (i < (n & ~15)) {
    const float u = v * (1.0f / cap);
    const float e = exp16(u + u);
    x[i] = cap * (1.0f - 2.0f / (e + 1.0f));
  } else {
    x[i] = cap * tanh_rn(v / cap);
  }
}

// ------------------------------------------------------------------ rope
// x [rows][n_heads][head_dim], cs [rows][head_dim / 2][2] = (cos, sin); one
// thread per (row, head, j < head_dim / 2).
__global__ __launch_bounds__(256) void rope_kernel(float* x, int rows, int n_heads, int head_dim,
                                                   const float* cs) {
  const int h = head_dim >> 1;
  const long t = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (long)rows * n_heads * h) return;
  const int j = (int)(t % h);
  const long rh = t / h;  // row * n_heads + head
  const int r = (int)(rh / n_heads);
  const float c = cs[((size_t)r * h + j) * 2], s = cs[((size_t)r * h + j) * 2 + 1];
  float* p = x + (size_t)rh * head_dim;
  const float lo = p[j], hi = p[j + h];
  p[j] = __builtin_fmaf(lo, c, -(hi * s));
  p[j + h] = __builtin_fmaf(hi, c, lo * s);
}

// -------------------------------------------------------- add, mul, scale
__global__ __launch_bounds__(256) void binop_kernel(float* a, const float* b, int n, int op, float s) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  if (op == 0) a[i] = a[i] + b[i];
  else if (op == 1) a[i] = a[i] * b[i];
  else a[i] = a[i] * s;
}

// zeros into rows x cols floats, rows ld apart (an empty contraction's C)
__global__ __launch_bounds__(256) void fill_zero_kernel(float* p, int ld, int cols) {
  float* row = p + (size_t)blockIdx.y * ld;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < cols; i += gridDim.x * blockDim.x) row[i] = 0.0f;
}

unsigned blocks(long n) { return (unsigned)((n + 255) / 256); }

}  // namespace

hipError_t fgm_launch_fill_zero(float* p, int ld, int rows, int cols, hipStream_t st) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  const unsigned gx = std::min(blocks(cols), 64u);
  hipLaunchKernelGGL(fill_zero_kernel, dim3(gx, rows), dim3(256), 0, st, p, ld, cols);
  return hipGetLastError();
}

hipError_t fgm_launch_rmsnorm(float* out, const float* x, const float* w, int rows, int n, float eps,
                              hipStream_t st) {
  if (rows <= 0 || n <= 0) return hipSuccess;
  static hipError_t attr[2] = {
      hipFuncSetAttribute((const void*)rmsnorm_kernel<false>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024),
      hipFuncSetAttribute((const void*)rmsnorm_kernel<true>, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024)};
  if (attr[0] != hipSuccess) return attr[0];
  if (attr[1] != hipSuccess) return attr[1];
  // about two float4 slots per thread; at most RMS_MAXV (n <= 32 T, T <= 1024)
  const int T = std::min(1024, std::max(64, ((n + 7) / 8 + 63) / 64 * 64));
  if (n > 32 * T) return hipErrorInvalidValue;
  const int S = fgm_rms_stride(n);
  const size_t lds = ((size_t)16 * S + 4) * 4;
  const bool vec = n % 4 == 0 && (((uintptr_t)out | (uintptr_t)x | (uintptr_t)w) & 15) == 0;
  if (vec)
    hipLaunchKernelGGL(rmsnorm_kernel<true>, dim3(rows), dim3(T), lds, st, out, x, w, n, S, eps);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<false>, dim3(rows), dim3(T), lds, st, out, x, w, n, S, eps);
  return hipGetLastError();
}

hipError_t fgm_launch_gelu(float* out, const float* gate, const float* up, int n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(gelu_kernel, dim3(blocks(n)), dim3(256), 0, st, out, gate, up, n);
  return hipGetLastError();
}

hipError_t fgm_launch_softcap(float* x, int n, float cap, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(softcap_kernel, dim3(blocks(n)), dim3(256), 0, st, x, n, cap);
  return hipGetLastError();
}

hipError_t fgm_launch_rope(float* x, int rows, int n_heads, int head_dim, const float* cs, hipStream_t st) {
  const long t = (long)rows * n_heads * (head_dim / 2);
  if (t <= 0) return hipSuccess;
  hipLaunchKernelGGL(rope_kernel, dim3(blocks(t)), dim3(256), 0, st, x, rows, n_heads, head_dim, cs);
  return hipGetLastError();
}

hipError_t fgm_launch_binop(float* a, const float* b, int n, int op, float s, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(binop_kernel, dim3(blocks(n)), dim3(256), 0, st, a, b, n, op, s);
  return hipGetLastError();
}
