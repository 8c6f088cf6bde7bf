// Shared device helpers for the gfx950 kernels of the fgm quantized-matmul path.
//
// Operand layouts (unchanged from the .fgm file, see include/fgm_hip.h):
//   packed A   [MB][KB][16 rows][64 bytes]            (ops.c:279-290)
//   int8 B     [N/16][K/64] tiles of 1024 bytes, each (K=64,N=16) as
//              [k/4][n][k%4]                          (quant.py:96-107)
//   int4 B     the int8 stream nibble-packed per 64-byte block:
//              packed[i] = q[i] | q[i+32] << 4        (quant.py:76-82)
//
// MFMA mapping used by every GEMM kernel here (v_mfma_i32_16x16x64_i8):
//   lane l = 16*g + j (g = l/16 in 0..3, j = l%16)
//   A operand: row j, B operand: column j; operand byte 4*t + e (t, e in
//   0..3) carries k = 16*t + 4*g + e of the 64-wide k-block.  The hardware
//   pairs A and B bytes by (lane group, byte), so this k-permutation leaves
//   the int32 sum exact.  With it, lane l's B bytes for t are the dword at
//   byte 256*t + 4*l of a 1024-byte int8 tile -- each of the four loads of a
//   wave reads 256 contiguous bytes.
//   Output: lane l, register r holds D[4*g + r][j].
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

typedef int v4i __attribute__((ext_vector_type(4)));

#define FGM_DEV static __device__ __forceinline__

// Signed int4 -> int8 for four nibbles at once: `x` holds four raw nibbles in
// the low half of each byte.  ((u ^ 8) + 120) ^ 128 == (u ^ 8) - 8 per byte,
// with no carry across bytes (the sum stays in 120..135).  Two's-complement
// nibbles, as amx_gemm.c:80-89 and vnni_test.c:52-69 define them.
FGM_DEV uint32_t nib4_to_i8x4(uint32_t u) {
  return ((u ^ 0x08080808u) + 0x78787878u) ^ 0x80808080u;
}

// Exact IEEE half -> float (v_cvt_f32_f16 is exact for every half).
FGM_DEV float f16_bits_to_f32(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return (float)v;
}

FGM_DEV v4i mfma16(v4i a, v4i b, v4i c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Quantisation of one activation value, reproducing fgm_quant_act
// (ops.c:195-203) bit for bit:
//   vector part (index < k & ~15): _mm512_cvtps_epi32 (round to nearest even;
//   NaN or |v| >= 2^31 gives 0x80000000) then _mm512_cvtsepi32_epi8
//   (saturate to [-128, 127]);
//   scalar tail: (int)lrintf(v) -- cvtss2si with a 64-bit result, NaN or
//   |v| >= 2^63 gives INT64_MIN, (int) keeps the low 32 bits -- clamped to
//   [-127, 127].
FGM_DEV int8_t quant_vec(float v) {
  if (!(__builtin_fabsf(v) < 2147483648.0f)) return (int8_t)-128;
  float r = __builtin_rintf(v);
  r = r > 127.0f ? 127.0f : (r < -128.0f ? -128.0f : r);
  return (int8_t)(int)r;
}

// quant_vec without branches, as an int in [-128, 127].
FGM_DEV int quant_vec_i(float v) {
  const int q = (int)__builtin_amdgcn_fmed3f(__builtin_rintf(v), -128.0f, 127.0f);
  return __builtin_fabsf(v) < 2147483648.0f ? q : -128;
}

// the low bytes of four ints, q0 in bits 7..0
FGM_DEV uint32_t pack4_i8(int q0, int q1, int q2, int q3) {
  const uint32_t lo = __builtin_amdgcn_perm((uint32_t)q1, (uint32_t)q0, 0x0C0C0400u);
  const uint32_t hi = __builtin_amdgcn_perm((uint32_t)q3, (uint32_t)q2, 0x04000C0Cu);
  return lo | hi;
}

FGM_DEV int8_t quant_tail(float v) {
  int64_t l;
  if (!(__builtin_fabsf(v) < 9223372036854775808.0f)) l = INT64_MIN;
  else l = (int64_t)__builtin_rintf(v);
  int32_t iv = (int32_t)(uint32_t)(uint64_t)l;
  return (int8_t)(iv > 127 ? 127 : (iv < -127 ? -127 : iv));
}

// Raw buffer access (gfx9 buffer descriptor, no stride).  A lane whose byte
// offset lies at or beyond `bytes` reads 0 without touching memory, which is
// how the kernels mask rows and columns without branches.
constexpr int FGM_BUF_FLAGS = 0x00020000;  // gfx9 family descriptor word 3
constexpr uint32_t FGM_OOB = 0x80000000u;  // an offset no buffer here reaches
// Cache-policy operand of the buffer load / store builtins on gfx950: nt
// (non-temporal, streamed past the caches' normal allocation).
constexpr int FGM_CPOL_NT = 2;

FGM_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           FGM_BUF_FLAGS);
}

FGM_DEV int32_t buf_load_b32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}

FGM_DEV v4i buf_load_b128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
}

FGM_DEV uint16_t buf_load_u16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}

// threadIdx.x / 64 as a scalar: lets the compiler keep per-wave loop bounds
// and tile indices in SGPRs and branch uniformly.
FGM_DEV int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// A raw buffer descriptor as four scalars (gfx9 layout: base, stride 0,
// num_records, the same flags as make_rsrc).
FGM_DEV v4i rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)base;
  return v4i{__builtin_amdgcn_readfirstlane((int)(uint32_t)p),
             __builtin_amdgcn_readfirstlane((int)((uint32_t)(p >> 32) & 0xFFFF)),
             __builtin_amdgcn_readfirstlane((int)bytes), FGM_BUF_FLAGS};
}

// One 16-byte chunk per lane from buffer offset voff + soff to LDS byte
// address lds + 16 * lane (buffer_load_dwordx4 ... lds).  Out-of-range lanes
// read zeros.  The compiler does not see these loads: the caller waits for
// them with wait_vm.
// NT: non-temporal (streamed data that is read once).
template <bool NT = false>
FGM_DEV void dma16(v4i rs, uint32_t lds, uint32_t voff, uint32_t soff) {
  // lds and soff are wave-uniform: keep them in scalar registers
  const int l0 = __builtin_amdgcn_readfirstlane((int)lds);
  const int s0 = __builtin_amdgcn_readfirstlane((int)soff);
  if constexpr (NT)
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds"
                 :
                 : "s"(l0), "v"(voff), "s"(rs), "s"(s0)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(l0), "v"(voff), "s"(rs), "s"(s0)
                 : "memory", "m0");
}

// One dword per lane to LDS byte address lds + 4 * lane (buffer_load_dword ...
// lds); like dma16, waited for with wait_vm.
FGM_DEV void dma4(v4i rs, uint32_t lds, uint32_t voff, uint32_t soff) {
  const int l0 = __builtin_amdgcn_readfirstlane((int)lds);
  const int s0 = __builtin_amdgcn_readfirstlane((int)soff);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               :
               : "s"(l0), "v"(voff), "s"(rs), "s"(s0)
               : "memory", "m0");
}

template <int N>
FGM_DEV void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// Compile-time loop: f(integral_constant<I>) for I = B .. E - 1.
template <int B, int E, class F>
FGM_DEV void sfor(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    sfor<B + 1, E>(f);
  }
}

// ------------------------------------------------- forward-pass f32 math
// Shared by the elementwise kernels and the fused prep pre-ops; each
// reproduces the reference's IEEE operations in the reference's order.

// exp512_ps (ops.c:21-39) on one lane: Cephes range reduction and polynomial.
FGM_DEV float exp16(float x) {
  x = __builtin_fminf(__builtin_fmaxf(x, -88.0f), 88.0f);
  const float fx = __builtin_rintf(x * 1.44269504088896341f);
  float z = __builtin_fmaf(-fx, 0.693359375f, x);
  z = __builtin_fmaf(-fx, -2.12194440e-4f, z);
  float y = 1.9875691500E-4f;
  y = __builtin_fmaf(y, z, 1.3981999507E-3f);
  y = __builtin_fmaf(y, z, 8.3334519073E-3f);
  y = __builtin_fmaf(y, z, 4.1665795894E-2f);
  y = __builtin_fmaf(y, z, 1.6666665459E-1f);
  y = __builtin_fmaf(y, z, 5.0000001201E-1f);
  y = __builtin_fmaf(y, z * z, z);
  y = y + 1.0f;
  return y * __int_as_float(((int)fx + 127) << 23);
}

// gelu_tanh_v (ops.c:96-107) on one lane, and the scalar tail's form
// (ops.c:114, 126; GCC fuses v + 0.044715 v^3 into one fma).  The tail's
// tanhf is evaluated in double and rounded once.
FGM_DEV float gelu_vec(float x) {
  const float x3 = (x * x) * x;
  const float u = 0.7978845608028654f * __builtin_fmaf(0.044715f, x3, x);
  const float e = exp16(u + u);
  const float t = 1.0f - 2.0f / (e + 1.0f);
  return (0.5f * x) * (1.0f + t);
}
FGM_DEV float tanh_rn(float a) { return (float)tanh((double)a); }
FGM_DEV float gelu_tail(float v) {
  return (0.5f * v) * (1.0f + tanh_rn(0.7978845608028654f * __builtin_fmaf((0.044715f * v) * v, v, v)));
}

template <int R>
FGM_DEV float row_ror(float v) {  // lane j of a 16-lane row reads lane (j + R) % 16
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + R, 0xF, 0xF, false));
}

// rmsnorm's sum of squares (ops.c:59-91) over a row staged transposed in LDS:
// x[16 t + j] at lds[j * S + t].  S = 4 (mod 64) puts the 16 accumulator rows
// in distinct banks, and S >= n / 16 + 16 lets every read-ahead stay in
// bounds unconditionally.
__host__ __device__ inline int fgm_rms_stride(int n) { return ((n + 15) / 16 + 16 + 63) / 64 * 64 + 4; }

// Called by lanes 0..15 of one wave (lane j = accumulator j, c = lds + j * S)
// with nt = n / 16: the reference's 16 fma chains in ascending t, then
// _mm512_reduce_add_ps as GCC emits it -- t3[j] = p[j + 8] + p[j];
// t6[j] = t3[j + 4] + t3[j]; (t6[0] + t6[2]) + (t6[1] + t6[3]) -- on DPP row
// rotations (a + b == b + a exactly, so the pairing is all that matters).
// Lane 0 returns the vector part's sum.
FGM_DEV float rms_sumsq16(const float* c, int nt) {
  float acc = 0.0f;
  // ping-pong over two sets of four 128-bit reads
  float4 A[4], B[4];
  auto rd = [&](float4* r, int t0) {
#pragma unroll
    for (int q = 0; q < 4; q++) r[q] = *(const float4*)(c + t0 + 4 * q);
  };
  auto chain = [&](const float4* r) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      acc = __builtin_fmaf(r[q].x, r[q].x, acc);
      acc = __builtin_fmaf(r[q].y, r[q].y, acc);
      acc = __builtin_fmaf(r[q].z, r[q].z, acc);
      acc = __builtin_fmaf(r[q].w, r[q].w, acc);
    }
  };
  int t = 0;
  rd(A, 0);
  for (; t + 32 <= nt; t += 32) {  // the barriers keep each read group ahead of the other's fmas
    rd(B, t + 16);
    __builtin_amdgcn_sched_barrier(0);
    chain(A);
    __builtin_amdgcn_sched_barrier(0);
    rd(A, t + 32);
    __builtin_amdgcn_sched_barrier(0);
    chain(B);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (t + 16 <= nt) {
    chain(A);
    t += 16;
  }
  for (; t < nt; t++) acc = __builtin_fmaf(c[t], c[t], acc);
  acc = acc + row_ror<8>(acc);
  acc = acc + row_ror<4>(acc);
  acc = acc + row_ror<2>(acc);
  return acc + row_ror<1>(acc);
}
