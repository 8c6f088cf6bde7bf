// GEMM activation preamble on gfx950: copy, optional FWHT, per-row int8
// quantisation and A tile-packing -- the device side of fgm_prep_rows,
// fgm_quant_act, fgm_fwht and fgm_pack_a (ops.c:153-204, 279-314).
// Optionally the row's producer runs first in the same workgroup: rmsnorm
// (ops.c:59-91, before the q/k/v and gate/up GEMMs, forward.rs:477-481,
// 614-618) or gelu_mul (ops.c:119-128, before down, forward.rs:621-622),
// with the reference's operations in its order, so the bytes equal the two
// separate calls'.
//
// One workgroup owns one activation row; each thread holds NV <= VMAX
// float4s of it (vector i = thread + v * blockDim covers columns 4i..4i+3)
// in registers from load to store, with the body compiled once per NV so
// that no loop carries a bound check.  A rotation runs its stages of
// distance 1 .. 128 in registers and across lanes and only longer ones
// through LDS (every FWHT stage is one add or one subtract per element, so
// the parallel schedule gives the reference's bytes).  The absolute maximum
// is a wave reduction plus one LDS exchange (order-free for non-NaN rows);
// then each float4 becomes one dword of the row-major int8 copy and one
// dword of its packed tile.
#include <algorithm>

#include "fgm_common.h"
#include "fgm_kernels.h"

namespace {

constexpr int PREP_MAX_THREADS = 1024;
constexpr int VMAX = 8;  // float4s per thread: rows up to 8 * 4 * 1024 = 32768 floats

// The butterfly stages of distance 2^lg0 .. hsz / 2 of the FWHT of the `k`
// floats in LDS, blocks of `hsz` (a power of two; ops.c:153-175).
__device__ void fwht_lds_stages(float* buf, int k, int hsz, int lg0) {
  const int half = k >> 1;
  for (int lg = lg0; (1 << lg) < hsz; lg++) {
    const int len = 1 << lg;
    for (int p = threadIdx.x; p < half; p += blockDim.x) {
      const int i = ((p >> lg) << (lg + 1)) | (p & (len - 1));  // pairs never straddle a block
      const float u = buf[i], v = buf[i + len];
      buf[i] = u + v;
      buf[i + len] = u - v;
    }
    __syncthreads();
  }
}

// In-place normalised FWHT in LDS.  `scale` = 1/sqrtf(hsz) computed on the
// host; it is only applied for hsz >= 16, matching the reference's 16-wide
// scale loop.
__device__ void fwht_lds(float* buf, int k, int hsz, float scale) {
  fwht_lds_stages(buf, k, hsz, 0);
  if (hsz >= 16) {
    for (int i = threadIdx.x; i < k; i += blockDim.x) buf[i] = buf[i] * scale;
    __syncthreads();
  }
}

// One butterfly across lane distance L (< 64): the lane without bit L keeps
// x + y, its partner (lane ^ L) keeps y - x, with y the other lane's value;
// both are y + (+-x), the same single rounding.  A row of k = 8192 puts two
// waves on each SIMD, so the stages are VALU-issue-bound and each costs two
// VALU ops per value: the sign select and an add that reads y itself.  For 1,
// 2 and 8 the exchange is a full-mask DPP pattern (quad permutes, a row
// rotation) that folds into the add as v_add_f32_dpp; 4 and 16 use
// ds_swizzle's xor mode (within 32 lanes) and 32 ds_bpermute, which run on
// the LDS pipe.  (v_permlane16/32_swap need a register copy first and cost
// one more VALU op than the LDS forms.)
template <int L>
__device__ __forceinline__ float butterfly(float x, bool upper) {
  const float s = upper ? -x : x;
  const int b = __float_as_int(x);
  int p;
  if constexpr (L == 1) p = __builtin_amdgcn_update_dpp(0, b, 0xB1, 0xF, 0xF, true);
  else if constexpr (L == 2) p = __builtin_amdgcn_update_dpp(0, b, 0x4E, 0xF, 0xF, true);
  else if constexpr (L == 8) p = __builtin_amdgcn_update_dpp(0, b, 0x128, 0xF, 0xF, true);
  else if constexpr (L < 32) p = __builtin_amdgcn_ds_swizzle(b, (L << 10) | 0x1F);
  else p = __float_as_int(__shfl_xor(x, L, 64));
  return __int_as_float(p) + s;
}

// Maximum over the 64 lanes of a wave: DPP within each 16-lane row, then the
// four row results read back as scalars.
template <int CTRL>
__device__ __forceinline__ float dpp_max(float v) {
  return fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false)));
}
__device__ __forceinline__ float wave_max(float v) {
  v = dpp_max<0xB1>(v);   // quad_perm 1,0,3,2
  v = dpp_max<0x4E>(v);   // quad_perm 2,3,0,1
  v = dpp_max<0x124>(v);  // row_ror 4
  v = dpp_max<0x128>(v);  // row_ror 8
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Packed-A byte offset of (row, col): [row/16][col/64][row%16][col%64].
__device__ __forceinline__ size_t pa_off(int row, int col, int KB) {
  return (((size_t)(row >> 4) * KB + (col >> 6)) * 16 + (row & 15)) * 64 + (col & 63);
}

// The computing part of prep_rows_kernel for a row whose float4s fit NV per
// thread (4 T NV >= k).  Every per-float4 loop is fully unrolled with no
// bound checks: float4s past the row read 0 through the buffer range check,
// stay 0 through every stage (the rotation's blocks past k hold only them),
// do not move the maximum, and their stores fall outside the store ranges.
template <int PRE, int NV, bool ROT, bool FAST>
__device__ __forceinline__ void prep_row(const PrepProb& a, int row, float* buf, float* red) {
  const int k = a.k, KB = k >> 6;
  const int T = blockDim.x, tid = threadIdx.x;

  // 1. the row into registers
  const float* src = a.src + (size_t)row * a.lda;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(src, (uint32_t)k * 4);
  const bool vec = FAST || (((((uintptr_t)a.src) & 15) == 0) && (a.lda & 3) == 0 && (k & 3) == 0);
  float x[NV][4];
  if (vec) {
#pragma unroll
    for (int v = 0; v < NV; v++) {
      const int c = 4 * (tid + v * T);
      const v4i q = buf_load_b128(rs, c < k ? (uint32_t)c * 4 : FGM_OOB, 0);
#pragma unroll
      for (int e = 0; e < 4; e++) x[v][e] = __int_as_float(q[e]);
    }
  } else {
#pragma unroll
    for (int v = 0; v < NV; v++) {
      const int c = 4 * (tid + v * T);
#pragma unroll
      for (int e = 0; e < 4; e++)
        x[v][e] = __int_as_float(buf_load_b32(rs, c + e < k ? (uint32_t)(c + e) * 4 : FGM_OOB, 0));
    }
  }

  // 1b. the fused producer (k % 64 == 0 here: the reference's vector forms
  //     cover the whole row, no scalar tails)
  if constexpr (PRE == PREP_RMSNORM) {
    // w is loaded before the reduction so its latency hides behind it
    float w[NV][4];
    if (a.aux) {
      const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.aux, (uint32_t)k * 4);
      const bool wvec = FAST || (((uintptr_t)a.aux) & 15) == 0;
#pragma unroll
      for (int v = 0; v < NV; v++) {
        const int c = 4 * (tid + v * T);
        if (wvec) {
          const v4i q = buf_load_b128(rw, c < k ? (uint32_t)c * 4 : FGM_OOB, 0);
#pragma unroll
          for (int e = 0; e < 4; e++) w[v][e] = __int_as_float(q[e]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; e++)
            w[v][e] = __int_as_float(buf_load_b32(rw, c + e < k ? (uint32_t)(c + e) * 4 : FGM_OOB, 0));
        }
      }
    }
    // the row transposed, x[16 t + j] at buf[j * S + t], for the 16 chains:
    // float4 i4 (columns 4 i4 .. 4 i4 + 3) goes to rows 4 (i4 % 4) + e,
    // column i4 / 4 (k % 4 == 0, so a float4 is wholly in or out of the row)
    const int S = fgm_rms_stride(k);
    auto tpos = [&](int i4) { return buf + 4 * (i4 & 3) * S + (i4 >> 2); };
#pragma unroll
    for (int v = 0; v < NV; v++) {
      const int i4 = tid + v * T;
      if (4 * i4 < k) {
        float* p = tpos(i4);
#pragma unroll
        for (int e = 0; e < 4; e++) p[e * S] = x[v][e];
      }
    }
    __syncthreads();
    if (tid < 16) {
      const float ss = rms_sumsq16(buf + tid * S, k >> 4);
      if (tid == 0) buf[16 * S] = 1.0f / __builtin_sqrtf(ss / (float)k + a.eps);
    }
    __syncthreads();
    // buf[16 * S] lies beyond the k floats a rotation stages below.  x is
    // read back from LDS so that it is not live in registers across the
    // reduction (w and the chains' read-ahead already need them).
    const float rinv = buf[16 * S];
#pragma unroll
    for (int v = 0; v < NV; v++) {
      const int i4 = tid + v * T;
      const float* p = tpos(i4);
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float xi = 4 * i4 < k ? p[e * S] : 0.0f;
        x[v][e] = a.aux ? (xi * rinv) * w[v][e] : xi * rinv;
      }
    }
  }
  if constexpr (PRE == PREP_GELU_MUL) {
    const __amdgpu_buffer_rsrc_t ru = make_rsrc(a.aux + (size_t)row * a.lda, (uint32_t)k * 4);
    const bool uvec = FAST || (((((uintptr_t)a.aux) & 15) == 0) && (a.lda & 3) == 0);
#pragma unroll
    for (int v = 0; v < NV; v++) {
      const int c = 4 * (tid + v * T);
      float u[4];
      if (uvec) {
        const v4i q = buf_load_b128(ru, c < k ? (uint32_t)c * 4 : FGM_OOB, 0);
#pragma unroll
        for (int e = 0; e < 4; e++) u[e] = __int_as_float(q[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; e++)
          u[e] = __int_as_float(buf_load_b32(ru, c + e < k ? (uint32_t)(c + e) * 4 : FGM_OOB, 0));
      }
#pragma unroll
      for (int e = 0; e < 4; e++) x[v][e] = gelu_vec(x[v][e]) * u[e];  // 0 past k
    }
  }
  if constexpr (PRE != PREP_COPY) {
    if (a.pre) {
      const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.pre + (size_t)row * k, (uint32_t)k * 4);
      const bool ovec = FAST || (((uintptr_t)a.pre) & 15) == 0;
#pragma unroll
      for (int v = 0; v < NV; v++) {
        const int c = 4 * (tid + v * T);
        const uint32_t off = c < k ? (uint32_t)c * 4 : FGM_OOB;
        if (ovec) {
          const v4i q = {__float_as_int(x[v][0]), __float_as_int(x[v][1]), __float_as_int(x[v][2]),
                         __float_as_int(x[v][3])};
          __builtin_amdgcn_raw_buffer_store_b128(q, ro, off, 0, 0);
        } else {
#pragma unroll
          for (int e = 0; e < 4; e++)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(x[v][e]), ro,
                                                  c < k ? off + 4 * e : FGM_OOB, 0, 0);
        }
      }
    }
  }

  // 2. optional rotation.  Element c = 4 i4 + e sits in lane i4 % 64 of its
  //    wave (T is a multiple of 64, so a wave holds 64 consecutive float4s):
  //    stages of distance 1 and 2 stay in the thread, 4 .. 128 pair lanes of
  //    one wave, 256 and up go through LDS.  Each stage is one add (lower
  //    element) or one subtract (upper element) of the same two values in
  //    every schedule, so the bytes are the reference's.
  if (ROT && a.hsz > 0) {
    const int hsz = a.hsz;
    const int lane = tid & 63;
    if (hsz > 1) {
#pragma unroll
      for (int v = 0; v < NV; v++) {
        const float u0 = x[v][0], u1 = x[v][1], u2 = x[v][2], u3 = x[v][3];
        x[v][0] = u0 + u1, x[v][1] = u0 - u1, x[v][2] = u2 + u3, x[v][3] = u2 - u3;
      }
    }
    if (hsz > 2) {
#pragma unroll
      for (int v = 0; v < NV; v++) {
        const float u0 = x[v][0], u1 = x[v][1], u2 = x[v][2], u3 = x[v][3];
        x[v][0] = u0 + u2, x[v][1] = u1 + u3, x[v][2] = u0 - u2, x[v][3] = u1 - u3;
      }
    }
    sfor<0, 6>([&](auto J) {
      constexpr int L = 1 << J;  // partner lane distance; element distance 4 L
      if (hsz > 4 * L) {
        const bool upper = lane & L;
#pragma unroll
        for (int v = 0; v < NV; v++)
#pragma unroll
          for (int e = 0; e < 4; e++) x[v][e] = butterfly<L>(x[v][e], upper);
      }
    });
    if (hsz > 256) {
      if constexpr (PRE == PREP_RMSNORM) __syncthreads();  // x was re-read from buf
#pragma unroll
      for (int v = 0; v < NV; v++) {
        const int c = 4 * (tid + v * T);
#pragma unroll
        for (int e = 0; e < 4; e++)
          if (c + e < k) buf[c + e] = x[v][e];
      }
      __syncthreads();
      fwht_lds_stages(buf, k, hsz, 8);
#pragma unroll
      for (int v = 0; v < NV; v++) {
        const int c = 4 * (tid + v * T);
#pragma unroll
        for (int e = 0; e < 4; e++) x[v][e] = (c + e < k) ? buf[c + e] : 0.0f;
      }
    }
    if (hsz >= 16) {
#pragma unroll
      for (int v = 0; v < NV; v++)
#pragma unroll
        for (int e = 0; e < 4; e++) x[v][e] = x[v][e] * a.fwht_scale;
    }
  }

  // 3. absolute maximum of the row
  float mx = 0.0f;
#pragma unroll
  for (int v = 0; v < NV; v++)
#pragma unroll
    for (int e = 0; e < 4; e++) mx = fmaxf(mx, __builtin_fabsf(x[v][e]));
  mx = wave_max(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  {
    // every wave's maximum in four 16-byte reads (one LDS round trip), the
    // slots past the workgroup's waves masked; every maximum is >= 0
    const int nw = T >> 6;
    mx = 0.0f;
#pragma unroll
    for (int q = 0; q < PREP_MAX_THREADS / 256; q++) {
      const float4 r = *(const float4*)(red + 4 * q);
      mx = fmaxf(mx, 4 * q + 0 < nw ? r.x : 0.0f);
      mx = fmaxf(mx, 4 * q + 1 < nw ? r.y : 0.0f);
      mx = fmaxf(mx, 4 * q + 2 < nw ? r.z : 0.0f);
      mx = fmaxf(mx, 4 * q + 3 < nw ? r.w : 0.0f);
    }
  }
  const float s = (mx == 0.0f) ? 1.0f : mx / 127.0f;
  const float inv = 1.0f / s;
  if (tid == 0) a.qs[row] = s;

  // 4. quantise and store: vector part [0, k & ~15) as _mm512_cvtps_epi32 +
  //    saturation, the scalar tail as lrintf + clamp (ops.c:194-203)
  if (FAST || (k & 15) == 0) {
    // the whole row in vector form: one dword of int8 per float4, stores
    // past the row dropped by the range check.  The packed tile row of
    // `row` is 64 bytes every 1024: [row/16][k/64][row%16][k%64].
    const __amdgpu_buffer_rsrc_t rr =
        make_rsrc(a.rot ? a.rot + (size_t)row * k : nullptr, a.rot ? (uint32_t)k * 4 : 0);
    const __amdgpu_buffer_rsrc_t rq =
        make_rsrc(a.qa ? a.qa + (size_t)row * k : nullptr, a.qa ? (uint32_t)k : 0);
    const __amdgpu_buffer_rsrc_t rp =
        make_rsrc(a.pa ? a.pa + ((size_t)(row >> 4) * KB * 16 + (row & 15)) * 64 : nullptr,
                  a.pa ? (uint32_t)KB * 1024 : 0);
#pragma unroll
    for (int v = 0; v < NV; v++) {
      const int c = 4 * (tid + v * T);
      const bool in = c < k;
      const uint32_t packed =
          pack4_i8(quant_vec_i(x[v][0] * inv), quant_vec_i(x[v][1] * inv),
                   quant_vec_i(x[v][2] * inv), quant_vec_i(x[v][3] * inv));
      if (a.rot) {
        const v4i q = {__float_as_int(x[v][0]), __float_as_int(x[v][1]), __float_as_int(x[v][2]),
                       __float_as_int(x[v][3])};
        __builtin_amdgcn_raw_buffer_store_b128(q, rr, in ? (uint32_t)c * 4 : FGM_OOB, 0, 0);
      }
      if (a.qa)
        __builtin_amdgcn_raw_buffer_store_b32((int)packed, rq, in ? (uint32_t)c : FGM_OOB, 0, 0);
      if (a.pa)
        __builtin_amdgcn_raw_buffer_store_b32(
            (int)packed, rp, in ? (uint32_t)((c >> 6) * 1024 + (c & 63)) : FGM_OOB, 0, 0);
    }
    return;
  }
  const int kv = k & ~15;
  float* rot = a.rot ? a.rot + (size_t)row * k : nullptr;
  int8_t* qa = a.qa ? a.qa + (size_t)row * k : nullptr;
  const bool dw = (k & 3) == 0;  // rows of qa / rot start 4-byte aligned
#pragma unroll
  for (int v = 0; v < NV; v++) {
    const int c = 4 * (tid + v * T);
    if (c >= k) break;
    uint32_t packed;
    if (c + 4 <= kv) {
      packed = pack4_i8(quant_vec_i(x[v][0] * inv), quant_vec_i(x[v][1] * inv),
                        quant_vec_i(x[v][2] * inv), quant_vec_i(x[v][3] * inv));
    } else {
      packed = 0;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float y = x[v][e] * inv;
        const int8_t q = (c + e < kv) ? quant_vec(y) : quant_tail(y);
        packed |= (uint32_t)(uint8_t)q << (8 * e);
      }
    }
    if (dw && c + 4 <= kv) {
      if (rot) *(float4*)(rot + c) = make_float4(x[v][0], x[v][1], x[v][2], x[v][3]);
      if (qa) *(uint32_t*)(qa + c) = packed;
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        if (c + e >= k) break;
        if (rot) rot[c + e] = x[v][e];
        if (qa) qa[c + e] = (int8_t)(packed >> (8 * e));
      }
    }
    if (a.pa) *(uint32_t*)(a.pa + pa_off(row, c, KB)) = packed;
  }
}

template <int PRE, bool ROT, bool FAST, int NVK>
__global__ __launch_bounds__(PREP_MAX_THREADS) void prep_rows_kernel(PrepBatch bt) {
  extern __shared__ float buf[];
  __shared__ __attribute__((aligned(16))) float red[PREP_MAX_THREADS / 64];
  const PrepProb a = pick_problem(bt);
  fetch_all(a);
  if ((int)blockIdx.x >= a.nwg) return;  // past this problem's rows
  const int row = a.r0 + (int)blockIdx.x;
  const int k = a.k, KB = k >> 6;
  const int T = blockDim.x, tid = threadIdx.x;

  if (row >= a.r1) {
    // Rows of the last covered tile block beyond r1: zero padding when past m,
    // otherwise whatever the caller's qa row holds (ops.c:308-311).
    if (!a.pa) return;
    for (int c = tid * 4; c < k; c += T * 4) {
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
  if constexpr (NVK > 0) {
    // one body for every row of the batch, NVK float4s per thread: those past
    // a shorter row read 0 and store nothing
    prep_row<PRE, NVK, ROT, FAST>(a, row, buf, red);
  } else {
    // float4s per thread that reach into the row (uniform; the launcher keeps
    // it within 1 .. VMAX)
    const int nv = ((k + 3) / 4 + T - 1) / T;
    sfor<1, VMAX + 1>([&](auto N) {
      if (nv == N) prep_row<PRE, N, ROT, FAST>(a, row, buf, red);
    });
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
__global__ __launch_bounds__(256) void fwht_kernel(float* x, int chunk, int hsz,
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

// One kernel per (producer, rotation compiled in, every operand aligned for
// 16-byte access with k % 16 == 0, float4s per thread): a batch that needs
// neither the rotation nor the unaligned and scalar-tail paths runs a single
// straight-line row body.  At this kernel's sizes the code on the executed
// path matters: it is fetched cold at every launch (a copy prep of 8 rows,
// k = 8192: 3.57 us with every path in one kernel, 3.33 us without the
// rotation, the unaligned loads and the scalar tail).
template <int PRE, bool ROT, bool FAST, int NVK>
static hipError_t launch_prep_kernel(const PrepBatch& b, int nwg, int threads, size_t lds, hipStream_t st) {
  static hipError_t attr = allow_big_lds(prep_rows_kernel<PRE, ROT, FAST, NVK>);
  if (attr != hipSuccess) return attr;
  // one grid row per problem, as wide as the problem with the most rows
  hipLaunchKernelGGL((prep_rows_kernel<PRE, ROT, FAST, NVK>), dim3(nwg, b.count), dim3(threads), lds, st, b);
  return hipGetLastError();
}

template <int PRE, bool ROT>
static hipError_t launch_prep_rot(const PrepBatch& b, bool fast, int nvk, int nwg, int threads, size_t lds,
                                  hipStream_t st) {
  if (!fast) return launch_prep_kernel<PRE, ROT, false, 0>(b, nwg, threads, lds, st);
  switch (nvk) {
    case 1: return launch_prep_kernel<PRE, ROT, true, 1>(b, nwg, threads, lds, st);
    case 2: return launch_prep_kernel<PRE, ROT, true, 2>(b, nwg, threads, lds, st);
    case 4: return launch_prep_kernel<PRE, ROT, true, 4>(b, nwg, threads, lds, st);
    default: return launch_prep_kernel<PRE, ROT, true, 8>(b, nwg, threads, lds, st);
  }
}

template <int PRE>
static hipError_t launch_prep_pre(const PrepBatch& b, bool rot, bool fast, int nvk, int nwg, int threads,
                                  size_t lds, hipStream_t st) {
  return rot ? launch_prep_rot<PRE, true>(b, fast, nvk, nwg, threads, lds, st)
             : launch_prep_rot<PRE, false>(b, fast, nvk, nwg, threads, lds, st);
}

hipError_t fgm_launch_prep(const PrepBatch& in, hipStream_t st) {
  PrepBatch b = in;
  const int pre = b.count ? b.p[0].preop : PREP_COPY;
  if (pre < PREP_COPY || pre > PREP_GELU_MUL) return hipErrorInvalidValue;
  int nwg = 0, kmax = 0, lds_floats = 0;
  for (int i = 0; i < b.count; i++) {
    PrepProb& p = b.p[i];
    if (p.preop != pre || (pre != PREP_COPY && p.k % 64)) return hipErrorInvalidValue;
    p.nwg = 0;
    if (p.r0 < p.r1) {
      // rows [r0, r1) compute; rows [r1, end of r1's tile block) only pack
      const int end = p.pa ? ((p.r1 + 15) / 16) * 16 : p.r1;
      p.nwg = end - p.r0;
      nwg = std::max(nwg, p.nwg);
      if (p.k > kmax) kmax = p.k;
      if (p.hsz > 0 && p.k > lds_floats) lds_floats = p.k;
      // the transposed row plus 1/rms (16 S + 1 > k floats)
      if (pre == PREP_RMSNORM) lds_floats = std::max(lds_floats, 16 * fgm_rms_stride(p.k) + 4);
    }
  }
  if (nwg == 0) return hipSuccess;
  // One float4 per thread up to 512 threads (gelu_mul, heavier per element:
  // 1024), more float4s per thread beyond, at most VMAX: a row's work is
  // latency-bound at the decode sizes, so more waves per row pay until the
  // cross-wave reduction costs more than they save (measured: 512 threads
  // for k = 2048 .. 8192).  Whole waves.
  const int cap = pre == PREP_GELU_MUL ? PREP_MAX_THREADS : 512;
  int threads = std::min(cap, ((kmax + 3) / 4 + 63) / 64 * 64);
  threads = std::max(threads, ((kmax + 4 * VMAX - 1) / (4 * VMAX) + 63) / 64 * 64);
  threads = std::max(64, std::min(threads, PREP_MAX_THREADS));
  // the kernel has a row body for 1 .. VMAX float4s per thread only
  if (((kmax + 3) / 4 + threads - 1) / threads > VMAX) return hipErrorInvalidValue;
  const size_t lds = (size_t)lds_floats * sizeof(float);
  bool rot = false, fast = true;
  for (int i = 0; i < b.count; i++) {
    const PrepProb& p = b.p[i];
    if (p.r0 >= p.r1) continue;
    rot = rot || p.hsz > 0;
    fast = fast && ((uintptr_t)p.src & 15) == 0 && (p.lda & 3) == 0 && (p.k & 15) == 0 &&
           ((uintptr_t)p.aux & 15) == 0 && ((uintptr_t)p.pre & 15) == 0;
  }
  // the fast kernels' body: the widest row's float4s per thread, rounded up
  // to a power of two
  const int nvmax = ((kmax + 3) / 4 + threads - 1) / threads;
  const int nvk = nvmax <= 1 ? 1 : nvmax <= 2 ? 2 : nvmax <= 4 ? 4 : 8;
  if (pre == PREP_RMSNORM) return launch_prep_pre<PREP_RMSNORM>(b, rot, fast, nvk, nwg, threads, lds, st);
  if (pre == PREP_GELU_MUL) return launch_prep_pre<PREP_GELU_MUL>(b, rot, fast, nvk, nwg, threads, lds, st);
  return launch_prep_pre<PREP_COPY>(b, rot, fast, nvk, nwg, threads, lds, st);
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
  hipLaunchKernelGGL(fwht_kernel, dim3(n / chunk), dim3(256),
                     (size_t)chunk * sizeof(float), st, x, chunk, hsz, scale);
  return hipGetLastError();
}
