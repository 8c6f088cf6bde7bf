/*
 * fgm_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain scalar C restatement of fastgemma's fgm-kernels quantized-matmul
 * path, written from the reference's algorithm so that the HIP kernels in
 * fastgemma_amd/csrc can be checked against it.  Nothing in the product
 * library links, loads or calls this file; only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may use it, and only as the checker.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the fastgemma repository root).  The floating-point operations are written
 * in exactly the reference's order, so the oracle is bit-exact with the
 * reference's VNNI / AMX kernels on finite inputs:
 *
 *   quant_act  : s = (amax == 0) ? 1 : amax / 127;  inv = 1 / s;
 *                q = sat_i8(cvt_rne(x * inv))                 ops.c:181-204
 *   gemm_q8c   : C = (float)acc * (b_scale[n] * a_scale[m])   vnni_gemm.c:208-219
 *   gemm_q4g   : C = 0; per group g ascending:
 *                C = fmaf((float)acc_g, f16(b_scale[g][n]), C);
 *                then C *= a_scale[m]                         vnni_gemm.c:258-285,316-321
 *   fwht       : butterflies len = 1, 2, 4 ... then x *= 1/sqrt(hsz)
 *                (the final scale is skipped when hsz < 16)   ops.c:153-175
 *
 * Pinning (what checks each function beyond "same formula twice"): see
 * tests/test_oracle.py -- the reference's own known-answer nibble table,
 * closed forms, brute-force int64 sums through an independent layout decode,
 * M-invariance / n-range invariance, and byte-for-byte comparison against the
 * reference's own C compiled from its sources into oracle/_ref.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off; no fast-math).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------- fault injection
 * Negative controls for the parity checks (tests/test_negative_controls.py):
 * a non-zero orc_fault makes the oracle compute one plausible WRONG variant,
 * so the tests can show that the golden / reference byte comparisons reject
 * it.  Each variant is a neighbouring convention the reference itself
 * contains or once contained:
 *   1  q8c epilogue (float)acc * as * bs           (vnni_test.c:72-85's ref_q8c)
 *   2  q8c per-64-k-tile float sums, then *= as*bs (amx_gemm.c:500-522)
 *   3  int4 nibble as offset binary, v - 8         (JOURNAL.md:1908-1937)
 *   4  q4g unfused C = (float)acc * s + C          (amx_gemm.c:478-498)
 *   5  q4g groups summed in descending order
 *   6  quant_act truncating instead of rounding to nearest even
 *   10 attention softmax sum as one serial chain instead of 16 lane sums
 *   11 attention P.V counting a slot shared by two ring spans once
 * 0 (the default) is the reference's behaviour; nothing else reads it. */
int orc_fault = 0;

/* ------------------------------------------------------------ f16 helpers */

/* Exact IEEE binary16 -> binary32 widening (every half value is exactly
 * representable in single precision).  The reference widens with
 * _mm512_cvtph_ps / _cvtsh_ss (vnni_gemm.c:272-275, vnni_test.c:112). */
float orc_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) << 31;
  uint32_t exp = (h >> 10) & 0x1F;
  uint32_t man = h & 0x3FF;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal half: normalise */
      int e = -1;
      do { man <<= 1; e++; } while (!(man & 0x400));
      man &= 0x3FF;
      bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
    }
  } else if (exp == 0x1F) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* binary32 -> binary16, round to nearest even (what numpy's astype(float16)
 * and _cvtss_sh(x, 0) do).  Used only to make synthetic f16 group scales,
 * the way the converter stores them (quant.py:165). */
uint16_t orc_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000;
  uint32_t exp = (x >> 23) & 0xFF;
  uint32_t man = x & 0x7FFFFF;
  if (exp == 0xFF) return (uint16_t)(sign | 0x7C00 | (man ? 0x200 | (man >> 13) : 0));
  int e = (int)exp - 127 + 15;
  if (e >= 0x1F) return (uint16_t)(sign | 0x7C00);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000;
    int shift = 14 - e;
    uint32_t half = man >> shift;
    uint32_t rem = man & ((1u << shift) - 1);
    uint32_t mid = 1u << (shift - 1);
    if (rem > mid || (rem == mid && (half & 1))) half++;
    return (uint16_t)(sign | half);
  }
  uint32_t half = ((uint32_t)e << 10) | (man >> 13);
  uint32_t rem = man & 0x1FFF;
  if (rem > 0x1000 || (rem == 0x1000 && (half & 1))) half++;
  return (uint16_t)(sign | half);
}

/* ------------------------------------------------ activation quantisation */

/* _mm512_cvtps_epi32 under the default MXCSR (round to nearest even): a NaN or
 * an out-of-range value gives the "integer indefinite" 0x80000000. */
static int32_t cvt_ps_epi32_rne(float v) {
  if (!(fabsf(v) < 2147483648.0f)) return INT32_MIN;
  return orc_fault == 6 ? (int32_t)v : (int32_t)rintf(v);
}

/* _mm512_cvtsepi32_epi8: signed saturation to [-128, 127]. */
static int8_t sat_i8(int32_t v) {
  return (int8_t)(v > 127 ? 127 : (v < -128 ? -128 : v));
}

/* The scalar tail of fgm_quant_act (ops.c:199-202): (int)lrintf(v) clamped to
 * [-127, 127].  On x86-64 lrintf is cvtss2si with a 64-bit destination (NaN or
 * |v| >= 2^63 gives INT64_MIN), and the (int) cast keeps the low 32 bits. */
static int8_t tail_q(float v) {
  int64_t l;
  if (!(fabsf(v) < 9223372036854775808.0f)) l = INT64_MIN;
  else l = (int64_t)rintf(v);
  int32_t iv = (int32_t)(uint32_t)(uint64_t)l;
  return (int8_t)(iv > 127 ? 127 : (iv < -127 ? -127 : iv));
}

/* fgm_quant_act, ops.c:181-204.  Per-row symmetric int8.
 * The reference reduces |x| with 16-lane _mm512_max_ps and a final tree; for
 * rows without NaN the maximum is order-free, which is what this restates.
 * (Rows containing NaN are outside the parity contract: the reference's
 * answer then depends on which SIMD lane the NaN lands in.) */
void orc_quant_act(const float *x, int rows, int k, int8_t *q, float *scale) {
  const int kv = k & ~15; /* elements handled by the 16-wide vector loop */
  for (int r = 0; r < rows; r++) {
    const float *src = x + (size_t)r * k;
    float m = 0.0f;
    for (int i = 0; i < k; i++) {
      float a = fabsf(src[i]);
      if (a > m) m = a;
    }
    float s = (m == 0.0f) ? 1.0f : m / 127.0f;
    float inv = 1.0f / s;
    scale[r] = s;
    int8_t *dst = q + (size_t)r * k;
    for (int i = 0; i < kv; i++) dst[i] = sat_i8(cvt_ps_epi32_rne(src[i] * inv));
    for (int i = kv; i < k; i++) dst[i] = tail_q(src[i] * inv);
  }
}

/* ------------------------------------------------------------- A packing */

/* packed_a_len, lib.rs:155-157. */
size_t orc_packed_a_len(int m, int k) { return (size_t)((m + 15) / 16) * 16 * (size_t)k; }

/* fgm_pack_a, ops.c:279-290: [MB][KB][16 rows][64 bytes]; rows >= M zero. */
void orc_pack_a(int M, int K, const int8_t *A, int8_t *Ap) {
  const int KB = K / 64, MB = (M + 15) / 16;
  for (int mb = 0; mb < MB; mb++)
    for (int kb = 0; kb < KB; kb++)
      for (int r = 0; r < 16; r++) {
        int m = mb * 16 + r;
        int8_t *d = Ap + (((size_t)mb * KB + kb) * 16 + r) * 64;
        for (int j = 0; j < 64; j++) d[j] = (m < M) ? A[(size_t)m * K + kb * 64 + j] : 0;
      }
}

/* Inverse of the packing: A[m][k] out of the packed tiles. */
static inline int8_t apk(const int8_t *Ap, int K, int m, int k) {
  const int KB = K / 64;
  return Ap[(((size_t)(m / 16) * KB + k / 64) * 16 + (m % 16)) * 64 + (k % 64)];
}

/* ------------------------------------------------------------------- FWHT */

/* fgm_fwht, ops.c:153-175.  In place on contiguous blocks of hsz (power of 2);
 * butterfly stages len = 1, 2, 4, ...; each stage writes (u + v, u - v).
 * scale = 1 / sqrtf(hsz), applied 16 at a time, so hsz < 16 is not scaled. */
void orc_fwht(float *x, int n, int hsz) {
  const float scale = 1.0f / sqrtf((float)hsz);
  for (int b = 0; b < n; b += hsz) {
    float *p = x + b;
    for (int len = 1; len < hsz; len <<= 1)
      for (int i = 0; i < hsz; i += len << 1)
        for (int j = i; j < i + len; j++) {
          float u = p[j], v = p[j + len];
          p[j] = u + v;
          p[j + len] = u - v;
        }
    for (int i = 0; i < hsz / 16 * 16; i++) p[i] = p[i] * scale;
  }
}

/* fgm_prep_rows, ops.c:293-314: rows [r0, r1) -- strided copy into rot, FWHT
 * when hsz > 0, quantise, then tile-pack the 16-row blocks the range covers
 * (rows >= m of those blocks are zero-filled). */
void orc_prep_rows(const float *src, int lda, float *rot, int8_t *qa, float *qs,
                   int8_t *pa, int m, int k, int hsz, int r0, int r1) {
  if (r0 >= r1) return;
  const int n = r1 - r0;
  for (int r = r0; r < r1; r++)
    memcpy(rot + (size_t)r * k, src + (size_t)r * lda, (size_t)k * sizeof(float));
  if (hsz > 0) orc_fwht(rot + (size_t)r0 * k, n * k, hsz);
  orc_quant_act(rot + (size_t)r0 * k, n, k, qa + (size_t)r0 * k, qs + r0);
  const int KB = k / 64;
  for (int mb = r0 / 16; mb * 16 < r1; mb++)
    for (int kb = 0; kb < KB; kb++)
      for (int rr = 0; rr < 16; rr++) {
        int row = mb * 16 + rr;
        int8_t *d = pa + (((size_t)mb * KB + kb) * 16 + rr) * 64;
        for (int j = 0; j < 64; j++) d[j] = (row < m) ? qa[(size_t)row * k + kb * 64 + j] : 0;
      }
}

/* ---------------------------------------------------------- weight layout */

/* Byte offset of B[k][n] in the int8 VNNI tile stream (quant.py:96-107,
 * vnni_test.c:49-50): tiles [N/16][K/64] of 1024 bytes, each holding
 * (K=64, N=16) as [k/4][n][k%4]. */
static inline size_t b8_off(int K, int k, int n) {
  const int KB = K / 64;
  return ((size_t)(n / 16) * KB + k / 64) * 1024 + ((k % 64) / 4) * 64 + (n % 16) * 4 + k % 4;
}

/* Signed int4 B[k][n] out of the packed stream: the int8 stream above, each
 * 64-byte block nibble-packed as packed[i] = q[i] | q[i+32] << 4
 * (quant.py:76-82), two's-complement nibbles (vnni_test.c:52-69). */
static inline int b4_val(const uint8_t *Bq, int K, int k, int n) {
  size_t p = b8_off(K, k, n);
  size_t blk = p / 64, off = p % 64;
  uint8_t byte = Bq[blk * 32 + off % 32];
  int v = (off < 32) ? (byte & 0xF) : (byte >> 4);
  return orc_fault == 3 ? v - 8 : (v ^ 8) - 8;
}

/* pack_b_tiles, quant.py:96-107: q[N][K] row-major (out, in) -> tile stream. */
void orc_pack_b_tiles(const int8_t *q, int N, int K, int8_t *blob) {
  for (int n = 0; n < N; n++)
    for (int k = 0; k < K; k++) blob[b8_off(K, k, n)] = q[(size_t)n * K + k];
}

/* pack_nibbles, quant.py:76-82: per 64-byte block, low nibble = value i,
 * high nibble = value i + 32. */
void orc_pack_nibbles(const int8_t *flat, size_t nbytes, uint8_t *packed) {
  for (size_t b = 0; b < nbytes / 64; b++)
    for (int i = 0; i < 32; i++)
      packed[b * 32 + i] =
          (uint8_t)((flat[b * 64 + i] & 0xF) | ((flat[b * 64 + 32 + i] & 0xF) << 4));
}

/* unpack_nibbles, quant.py:85-92. */
void orc_unpack_nibbles(const uint8_t *packed, size_t nbytes_out, int8_t *flat) {
  for (size_t b = 0; b < nbytes_out / 64; b++)
    for (int i = 0; i < 32; i++) {
      int lo = packed[b * 32 + i] & 0xF, hi = packed[b * 32 + i] >> 4;
      flat[b * 64 + i] = (int8_t)((lo ^ 8) - 8);
      flat[b * 64 + 32 + i] = (int8_t)((hi ^ 8) - 8);
    }
}

/* ------------------------------------------------------------------ GEMMs */

/* Exact integer dot products, int32 wrap-around semantics (vpdpbusd does not
 * saturate, so the reference's biased sum minus 128*asum equals the true sum
 * modulo 2^32). */

/* Raw int32 accumulators of the q8c GEMM: acc[m][n] = sum_k A[m][k] * B[k][n]
 * for m < M, n in [16*n0, 16*n1), stored at acc[m * ldacc + n]. */
void orc_acc_q8c(int M, int K, const int8_t *Ap, const int8_t *B, int32_t *acc, int ldacc,
                 int n0, int n1) {
  for (int m = 0; m < M; m++)
    for (int n = n0 * 16; n < n1 * 16; n++) {
      uint32_t s = 0;
      for (int k = 0; k < K; k++)
        s += (uint32_t)((int32_t)apk(Ap, K, m, k) * (int32_t)B[b8_off(K, k, n)]);
      acc[(size_t)m * ldacc + n] = (int32_t)s;
    }
}

/* The q8c epilogue on given accumulators, vnni_gemm.c:206-219:
 * C[m][n] = (float)acc * (b_scale[n] * a_scale[m]) -- the scale product is
 * rounded first, the int32 -> float conversion rounds to nearest even. */
void orc_epilogue_q8c(int M, const int32_t *acc, int ldacc, const float *a_scale,
                      const float *b_scale, float *C, int ldc, int n0, int n1) {
  for (int m = 0; m < M; m++)
    for (int n = n0 * 16; n < n1 * 16; n++) {
      float f = (float)acc[(size_t)m * ldacc + n];
      float sc = b_scale[n] * a_scale[m];
      C[(size_t)m * ldc + n] = orc_fault == 1 ? f * a_scale[m] * b_scale[n] : f * sc;
    }
}

/* fgm_gemm_q8c_vnni, vnni_gemm.c:224-245 (+ q8c_block :190-222).
 * Writes C[m][n] for m < M, n in [16*n0, 16*n1); nothing else is touched. */
void orc_gemm_q8c(int M, int N, int K, const int8_t *Ap, const float *a_scale,
                  const int8_t *B, const float *b_scale, float *C, int ldc, int n0, int n1) {
  if (M <= 0 || n1 <= n0) return;
  if (orc_fault == 2) {
    for (int m = 0; m < M; m++)
      for (int n = n0 * 16; n < n1 * 16; n++) {
        float c = 0.0f;
        for (int kb = 0; kb < K / 64; kb++) {
          int32_t t = 0;
          for (int k = 64 * kb; k < 64 * kb + 64; k++) t += (int32_t)apk(Ap, K, m, k) * (int32_t)B[b8_off(K, k, n)];
          c += (float)t;
        }
        C[(size_t)m * ldc + n] = c * (a_scale[m] * b_scale[n]);
      }
    return;
  }
  int32_t *acc = (int32_t *)malloc((size_t)M * N * sizeof(int32_t));
  orc_acc_q8c(M, K, Ap, B, acc, N, n0, n1);
  orc_epilogue_q8c(M, acc, N, a_scale, b_scale, C, ldc, n0, n1);
  free(acc);
}

/* Raw per-group int32 accumulators of the q4g GEMM:
 * acc[(g * M + m) * ldacc + n] = sum_{k in group g} A[m][k] * B[k][n]. */
void orc_acc_q4g(int M, int K, const int8_t *Ap, const uint8_t *Bq, int group, int32_t *acc,
                 int ldacc, int n0, int n1) {
  const int NG = K / group;
  for (int g = 0; g < NG; g++)
    for (int m = 0; m < M; m++)
      for (int n = n0 * 16; n < n1 * 16; n++) {
        uint32_t s = 0;
        for (int k = g * group; k < (g + 1) * group; k++)
          s += (uint32_t)((int32_t)apk(Ap, K, m, k) * b4_val(Bq, K, k, n));
        acc[((size_t)g * M + m) * ldacc + n] = (int32_t)s;
      }
}

/* The q4g epilogue on given per-group accumulators (acc laid out as
 * orc_acc_q4g writes it), vnni_gemm.c:258-285 and 316-321: C = 0, then per
 * group g in ascending order C = fmaf((float)acc_g, f16(b_scale[g][n]), C),
 * finally C *= a_scale[m]. */
void orc_epilogue_q4g(int M, int N, int NG, const int32_t *acc, int ldacc, const float *a_scale,
                      const uint16_t *b_scale, float *C, int ldc, int n0, int n1) {
  for (int m = 0; m < M; m++)
    for (int n = n0 * 16; n < n1 * 16; n++) {
      float c = 0.0f;
      for (int i = 0; i < NG; i++) {
        const int g = orc_fault == 5 ? NG - 1 - i : i;
        const float a = (float)acc[((size_t)g * M + m) * ldacc + n];
        const float sc = orc_f16_to_f32(b_scale[(size_t)g * N + n]);
        if (orc_fault == 4) {
          const float p = a * sc;
          c = p + c;
        } else {
          c = fmaf(a, sc, c);
        }
      }
      C[(size_t)m * ldc + n] = c;
    }
  for (int m = 0; m < M; m++)
    for (int n = n0 * 16; n < n1 * 16; n++)
      C[(size_t)m * ldc + n] = C[(size_t)m * ldc + n] * a_scale[m];
}

/* fgm_gemm_q4g_vnni, vnni_gemm.c:291-322 (+ q4g_block :252-289).
 * b_scale is f16 [K/group][N]. */
void orc_gemm_q4g(int M, int N, int K, const int8_t *Ap, const float *a_scale,
                  const uint8_t *Bq, const uint16_t *b_scale, int group, float *C, int ldc,
                  int n0, int n1) {
  if (M <= 0 || n1 <= n0) return;
  const int NG = K / group;
  int32_t *acc = (int32_t *)malloc((size_t)(NG ? NG : 1) * M * N * sizeof(int32_t));
  orc_acc_q4g(M, K, Ap, Bq, group, acc, N, n0, n1);
  orc_epilogue_q4g(M, N, NG, acc, N, a_scale, b_scale, C, ldc, n0, n1);
  free(acc);
}

/* ------------------------------------------------------------ generators */

/* The reference tests' own generators, so their case lists can be replayed
 * with identical inputs.
 * vnni_test.c:39-43: xorshift64 (13, 7, 17), rnd(lo, hi) = lo + s % (hi-lo+1).
 * Returns the advanced state (the reference keeps it in one static). */
uint64_t orc_xorshift_fill(uint64_t s, size_t n, int lo, int hi, int32_t *out) {
  uint64_t span = (uint64_t)(hi - lo + 1);
  for (size_t i = 0; i < n; i++) {
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    out[i] = lo + (int)(s % span);
  }
  return s;
}

/* gemm_test.c:30-31 and dbg.c:33-34: 32-bit LCG, value = lo + (s >> 16) % span. */
uint32_t orc_lcg_fill(uint32_t s, size_t n, int lo, int hi, int32_t *out) {
  uint32_t span = (uint32_t)(hi - lo + 1);
  for (size_t i = 0; i < n; i++) {
    s = s * 1103515245u + 12345u;
    out[i] = lo + (int)((s >> 16) % span);
  }
  return s;
}

/* SplitMix64 (Steele, Lea, Flood 2014): the synthetic-input generator shared
 * by tests and bench so both sides see identical inputs for a seed. */
static inline uint64_t splitmix64(uint64_t *s) {
  uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* Uniform integers in [lo, hi] as int8 (Lemire-free modulo: the bias is
 * below 2^-56 for these ranges). */
void orc_gen_i8(uint64_t seed, size_t n, int lo, int hi, int8_t *out) {
  uint64_t s = seed;
  uint64_t span = (uint64_t)(hi - lo + 1);
  for (size_t i = 0; i < n; i++) out[i] = (int8_t)(lo + (int)(splitmix64(&s) % span));
}

/* Uniform bytes -- a packed int4 stream of iid uniform [-8, 7] nibbles. */
void orc_gen_u8(uint64_t seed, size_t n, uint8_t *out) {
  uint64_t s = seed;
  for (size_t i = 0; i < n; i++) out[i] = (uint8_t)(splitmix64(&s) >> 56);
}

static inline double u01(uint64_t *s) { return (double)(splitmix64(s) >> 11) * 0x1.0p-53; }

/* Uniform floats in [lo, hi). */
void orc_gen_uniform(uint64_t seed, size_t n, float lo, float hi, float *out) {
  uint64_t s = seed;
  for (size_t i = 0; i < n; i++) out[i] = (float)(lo + (hi - lo) * u01(&s));
}

/* Standard normals (Box-Muller). */
void orc_gen_normal(uint64_t seed, size_t n, float *out) {
  uint64_t s = seed;
  for (size_t i = 0; i < n; i += 2) {
    double u1 = u01(&s), u2 = u01(&s);
    if (u1 < 1e-300) u1 = 1e-300;
    double r = sqrt(-2.0 * log(u1)), t = 6.283185307179586 * u2;
    out[i] = (float)(r * cos(t));
    if (i + 1 < n) out[i + 1] = (float)(r * sin(t));
  }
}

/* Student-t with nu degrees of freedom: Z / sqrt(chi2_nu / nu), chi2 as a sum
 * of nu squared normals (nu is a small integer here). */
void orc_gen_student_t(uint64_t seed, size_t n, int nu, float *out) {
  uint64_t s = seed;
  if (nu < 1) nu = 1;
  if (nu > 7) nu = 7;
  for (size_t i = 0; i < n; i++) {
    double z[8];
    int need = nu + 1;
    for (int j = 0; j < need; j += 2) {
      double u1 = u01(&s), u2 = u01(&s);
      if (u1 < 1e-300) u1 = 1e-300;
      double r = sqrt(-2.0 * log(u1)), t = 6.283185307179586 * u2;
      z[j] = r * cos(t);
      if (j + 1 < 8) z[j + 1] = r * sin(t);
    }
    double chi = 0;
    for (int j = 1; j <= nu; j++) chi += z[j] * z[j];
    out[i] = (float)(z[0] / sqrt(chi / nu));
  }
}

/* ======================================================= elementwise ops
 * The forward pass's f32 elementwise primitives, ops.c:15-39 (exp512_ps),
 * :55-88 (rmsnorm), :90-124 (gelu), :126-142 (rope), :316-350 (add, mul,
 * scale, softcap).  The reference processes 16 floats per AVX-512 vector and
 * finishes with a scalar tail; both parts are restated element by element in
 * the reference's operation order.  The reference is built by GCC, whose
 * default for GNU C is -ffp-contract=fast: it fuses some scalar-tail
 * expressions into one fma.  Where it does (determined against the compiled
 * reference, tests/test_elem.py), this restatement writes fmaf explicitly. */

/* exp512_ps (ops.c:21-39) on one lane: Cephes range reduction. */
float orc_exp16(float x) {
  x = fminf(fmaxf(x, -88.0f), 88.0f);
  const float fx = rintf(x * 1.44269504088896341f); /* _mm512_roundscale_ps, RNE */
  float z = fmaf(-fx, 0.693359375f, x);              /* _mm512_fnmadd_ps */
  z = fmaf(-fx, -2.12194440e-4f, z);
  float y = 1.9875691500E-4f;
  y = fmaf(y, z, 1.3981999507E-3f);
  y = fmaf(y, z, 8.3334519073E-3f);
  y = fmaf(y, z, 4.1665795894E-2f);
  y = fmaf(y, z, 1.6666665459E-1f);
  y = fmaf(y, z, 5.0000001201E-1f);
  y = fmaf(y, z * z, z);
  y = y + 1.0f;
  const int32_t n = (int32_t)fx; /* _mm512_cvtps_epi32 of an integral value */
  const uint32_t bits = (uint32_t)(n + 127) << 23;
  float p2;
  memcpy(&p2, &bits, 4);
  return y * p2;
}

/* _mm512_reduce_add_ps as GCC's avx512fintrin.h defines it: the upper eight
 * lanes onto the lower eight, then four, then lanes {0,1} + {2,3}, then the
 * last pair. */
static float gcc_reduce_add16(const float *a) {
  float t3[8], t6[4];
  for (int j = 0; j < 8; j++) t3[j] = a[j + 8] + a[j];
  for (int j = 0; j < 4; j++) t6[j] = t3[j + 4] + t3[j];
  return (t6[0] + t6[2]) + (t6[1] + t6[3]);
}

/* sum of squares and 1/rms of one row (ops.c:60-67, 78-85): 16 lane
 * accumulators, lane j takes x[16t + j] in ascending t by fma; GCC's tree;
 * the tail fused as fmaf(x, x, ss); then 1 / sqrtf(ss / n + eps). */
static float rms_inv(const float *x, int n, float eps) {
  float acc[16] = {0};
  int i = 0;
  for (; i + 16 <= n; i += 16)
    for (int j = 0; j < 16; j++) acc[j] = fmaf(x[i + j], x[i + j], acc[j]);
  float ss = gcc_reduce_add16(acc);
  for (; i < n; i++) ss = fmaf(x[i], x[i], ss);
  return 1.0f / sqrtf(ss / (float)n + eps);
}

/* fgm_rmsnorm (ops.c:59-74): out = (x * inv) * w */
void orc_rmsnorm(float *out, const float *x, const float *w, int n, float eps) {
  const float inv = rms_inv(x, n, eps);
  for (int i = 0; i < n; i++) out[i] = (x[i] * inv) * w[i];
}

/* fgm_rmsnorm_noscale (ops.c:77-91): out = x * inv */
void orc_rmsnorm_noscale(float *out, const float *x, int n, float eps) {
  const float inv = rms_inv(x, n, eps);
  for (int i = 0; i < n; i++) out[i] = x[i] * inv;
}

/* gelu_tanh_v (ops.c:96-107) on one lane */
static float gelu_vec(float x) {
  const float x3 = (x * x) * x;
  const float u = 0.7978845608028654f * fmaf(0.044715f, x3, x);
  const float e = orc_exp16(u + u);
  const float t = 1.0f - 2.0f / (e + 1.0f);
  return (0.5f * x) * (1.0f + t);
}

/* the scalar tail's gelu (ops.c:114, 126): libm tanhf; GCC fuses
 * v + 0.044715f * v * v * v into fmaf((0.044715f * v) * v, v, v) */
static float gelu_tail(float v) {
  return (0.5f * v) * (1.0f + tanhf(0.7978845608028654f * fmaf((0.044715f * v) * v, v, v)));
}

/* fgm_gelu_mul (ops.c:119-128): out = gelu(gate) * up */
void orc_gelu_mul(float *out, const float *gate, const float *up, int n) {
  const int nv = n & ~15;
  for (int i = 0; i < n; i++) out[i] = (i < nv ? gelu_vec(gate[i]) : gelu_tail(gate[i])) * up[i];
}

/* fgm_gelu (ops.c:109-116), in place */
void orc_gelu(float *x, int n) {
  const int nv = n & ~15;
  for (int i = 0; i < n; i++) x[i] = i < nv ? gelu_vec(x[i]) : gelu_tail(x[i]);
}

/* fgm_rope (ops.c:135-147): a = pos * inv_freq[j], c = cosf(a), s = sinf(a)
 * (libm); GCC fuses the rotation into fmaf(lo, c, -(hi * s)) and
 * fmaf(hi, c, lo * s). */
void orc_rope(float *x, int n_heads, int head_dim, const float *inv_freq, int pos) {
  const int h = head_dim / 2;
  for (int j = 0; j < h; j++) {
    const float a = (float)pos * inv_freq[j];
    const float c = cosf(a), s = sinf(a);
    for (int hh = 0; hh < n_heads; hh++) {
      float *p = x + (size_t)hh * head_dim;
      const float lo = p[j], hi = p[j + h];
      p[j] = fmaf(lo, c, -(hi * s));
      p[j + h] = fmaf(hi, c, lo * s);
    }
  }
}

/* fgm_add / fgm_mul / fgm_scale (ops.c:317-337) */
void orc_add(float *a, const float *b, int n) { for (int i = 0; i < n; i++) a[i] += b[i]; }
void orc_mul(float *a, const float *b, int n) { for (int i = 0; i < n; i++) a[i] *= b[i]; }
void orc_scale(float *a, float s, int n) { for (int i = 0; i < n; i++) a[i] *= s; }

/* fgm_softcap (ops.c:340-351): vector part cap * (1 - 2 / (exp(2u) + 1)) with
 * u = x * (1 / cap); tail cap * tanhf(x / cap) */
void orc_softcap(float *x, int n, float cap) {
  const float ci = 1.0f / cap;
  const int nv = n & ~15;
  for (int i = 0; i < n; i++) {
    if (i < nv) {
      const float u = x[i] * ci;
      const float e = orc_exp16(u + u);
      x[i] = cap * (1.0f - 2.0f / (e + 1.0f));
    } else {
      x[i] = cap * tanhf(x[i] / cap);
    }
  }
}

/* ------------------------------------------------------ int8-KV attention
 * fgm_attend_q8_heads / fgm_attend_q8_row / fgm_store_v_t (ops.c:353-877).
 * Caches: K [cap][kv_heads * head_dim] int8 with one f32 scale per slot; V
 * transposed in groups of four slots, vt[((slot/4) * kvd + j) * 4 + slot%4]
 * (ops.c:645-657, kv.rs:20-31); slot = ring ? t % ring : t.
 *
 * The integer parts (Q.K dot products, P.V accumulators) are exact, so any
 * summation order gives the reference's values; the float parts follow the
 * reference's order: score = ((float)dot * qscale) * kscale; exp of the
 * 16-wide chunks by exp512_ps with 16 lane sums (plain adds, chunk order) and
 * GCC's reduce tree, the n % 16 tail by libm expf added in order; weights
 * ((e * inv) * vs) with a 16-bit quantisation iw = (int)(w * wq_inv + 0.5f)
 * (GCC contracts the multiply-add into one fma at -O2 -march=cascadelake);
 * out = (float)(sum iw * v) * wq_scale.
 *
 * orc_attn_tail_noncr counts tail expf values that differ from the correctly
 * rounded exp (the GPU evaluates the tail correctly rounded); tests read it to
 * know when the tail can be compared bit for bit. */
int orc_attn_tail_noncr = 0;

static void orc_attn_head(float *oh, const float *qh, const int8_t *kc, const float *ks,
                          const int8_t *vc, const float *vs, int kvd, int kv_off, int head_dim,
                          int start, int end, int ring) {
  /* per-head int8 query (ops.c:417-433) */
  int8_t qq[512];
  float qamax = 0.0f;
  for (int i = 0; i < head_dim; i++) {
    const float a = fabsf(qh[i]);
    if (a > qamax) qamax = a;
  }
  const float qscale = qamax / 127.0f;
  const float qinv = qamax > 0.0f ? 127.0f / qamax : 0.0f;
  for (int i = 0; i < head_dim; i++) {
    int v = (int)lrintf(qh[i] * qinv);
    v = v > 127 ? 127 : (v < -127 ? -127 : v);
    qq[i] = (int8_t)v;
  }
  const int n = end - start;
  float *sc = (float *)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
  float mx = -INFINITY;
  /* scores (ops.c:441-488): sum (k + 128) q - 128 sum q == sum k q exactly */
  for (int t = start; t < end; t++) {
    const int slot = ring ? t % ring : t;
    const int8_t *kp = kc + (size_t)slot * kvd + kv_off;
    int32_t d = 0;
    for (int i = 0; i < head_dim; i++) d += (int32_t)kp[i] * (int32_t)qq[i];
    const float s = (float)d * qscale * ks[slot];
    sc[t - start] = s;
    if (s > mx) mx = s;
  }
  /* softmax (ops.c:493-505) */
  float lanes[16] = {0};
  int u = 0;
  for (; u + 16 <= n; u += 16)
    for (int j = 0; j < 16; j++) {
      const float e = orc_exp16(sc[u + j] - mx);
      sc[u + j] = e;
      lanes[j] = lanes[j] + e;
    }
  float sum = gcc_reduce_add16(lanes);
  if (orc_fault == 10) {
    sum = 0.0f;
    for (int i = 0; i < (n & ~15); i++) sum += sc[i];
  }
  for (; u < n; u++) {
    const float x = sc[u] - mx;
    sc[u] = expf(x);
    if (sc[u] != (float)exp((double)x)) orc_attn_tail_noncr++;
    sum += sc[u];
  }
  const float inv = 1.0f / sum;
  /* weight range (ops.c:546-550) */
  float wmax = 0.0f;
  for (int t = start; t < end; t++) {
    const float w = sc[t - start] * inv * vs[ring ? t % ring : t];
    if (w > wmax) wmax = w;
  }
  if (!(wmax > 0.0f)) {
    for (int i = 0; i < head_dim; i++) oh[i] = 0.0f;
    free(sc);
    return;
  }
  const float wq_scale = wmax / 65535.0f, wq_inv = 65535.0f / wmax;
  /* slot runs and their four-slot-aligned spans (ops.c:560-584) */
  int run_lo[2], run_hi[2], nrun;
  if (!ring) {
    run_lo[0] = start; run_hi[0] = end; nrun = 1;
  } else if (n >= ring) {
    run_lo[0] = 0; run_hi[0] = ring; nrun = 1;
  } else {
    const int s0 = start % ring;
    if (s0 + n <= ring) {
      run_lo[0] = s0; run_hi[0] = s0 + n; nrun = 1;
    } else {
      run_lo[0] = s0; run_hi[0] = ring; run_lo[1] = 0; run_hi[1] = s0 + n - ring; nrun = 2;
    }
  }
  int span_hi = 0;
  for (int r = 0; r < nrun; r++) {
    const int hi = (run_hi[r] + 3) & ~3;
    if (hi > span_hi) span_hi = hi;
  }
  /* u16 weights by slot (ops.c:591-598): zero over the spans, the later t wins */
  int32_t *iw = (int32_t *)calloc((size_t)span_hi + 4, sizeof(int32_t));
  for (int t = start; t < end; t++) {
    const int sl = ring ? t % ring : t;
    const float w = sc[t - start] * inv * vs[sl];
    int q = (int)fmaf(w, wq_inv, 0.5f);
    if (q > 65535) q = 65535;
    if (q < 0) q = 0;
    iw[sl] = q;
  }
  /* P.V over each run's span (ops.c:605-631); a slot inside two spans counts
   * twice, as there.  (acc_hi << 8) + acc_lo == sum iw * v modulo 2^32. */
  uint32_t acc[512];
  for (int i = 0; i < head_dim; i++) acc[i] = 0;
  for (int r = 0; r < nrun; r++) {
    const int glo = run_lo[r] & ~3, ghi = (run_hi[r] + 3) & ~3;
    for (int s = glo; s < ghi; s++) {
      if (!iw[s]) continue;
      if (orc_fault == 11 && r == 1 && s >= (run_lo[0] & ~3) && s < ((run_hi[0] + 3) & ~3)) continue;
      const int8_t *vp = vc + ((size_t)(s >> 2) * kvd + kv_off) * 4 + (s & 3);
      for (int i = 0; i < head_dim; i++) acc[i] += (uint32_t)(iw[s] * (int32_t)vp[(size_t)i * 4]);
    }
  }
  for (int i = 0; i < head_dim; i++) oh[i] = (float)(int32_t)acc[i] * wq_scale;
  free(iw);
  free(sc);
}

/* fgm_attend_q8_heads (ops.c:378-637): heads [h0, h1); kv head h / (n_heads /
 * kv_heads) */
void orc_attend_q8_heads(float *out, const float *q, const int8_t *kc, const float *ks,
                         const int8_t *vc, const float *vs, int n_heads, int kv_heads,
                         int head_dim, int start, int end, int h0, int h1, int ring, int cap) {
  (void)cap;
  const int kvd = kv_heads * head_dim, grp = n_heads / kv_heads;
  for (int h = h0; h < h1; h++)
    orc_attn_head(out + (size_t)h * head_dim, q + (size_t)h * head_dim, kc, ks, vc, vs, kvd,
                  (h / grp) * head_dim, head_dim, start, end, ring);
}

/* fgm_attend_q8 (ops.c:363-368) */
void orc_attend_q8(float *out, const float *q, const int8_t *kc, const float *ks,
                   const int8_t *vc, const float *vs, int n_heads, int kv_heads, int head_dim,
                   int start, int end) {
  orc_attend_q8_heads(out, q, kc, ks, vc, vs, n_heads, kv_heads, head_dim, start, end, 0,
                      n_heads, 0, end);
}

/* fgm_attend_q8_row (ops.c:729-872): n <= 0 zeroes every head; kv_heads != 1
 * takes the per-head path; otherwise at most 8 heads are computed (heads past
 * the eighth are left untouched), with the per-head numerics. */
void orc_attend_q8_row(float *out, const float *q, const int8_t *kc, const float *ks,
                       const int8_t *vc, const float *vs, int n_heads, int kv_heads,
                       int head_dim, int start, int end, int ring, int cap) {
  if (end - start <= 0) {
    for (int i = 0; i < n_heads * head_dim; i++) out[i] = 0.0f;
    return;
  }
  if (kv_heads != 1) {
    orc_attend_q8_heads(out, q, kc, ks, vc, vs, n_heads, kv_heads, head_dim, start, end, 0,
                        n_heads, ring, cap);
    return;
  }
  orc_attend_q8_heads(out, q, kc, ks, vc, vs, n_heads, 1, head_dim, start, end, 0,
                      n_heads > 8 ? 8 : n_heads, ring, cap);
}

/* fgm_store_v_t (ops.c:653-657) */
void orc_store_v_t(int8_t *vt, const int8_t *src, int n, int slot) {
  int8_t *dst = vt + (size_t)(slot >> 2) * n * 4 + (slot & 3);
  for (int j = 0; j < n; j++) dst[(size_t)j * 4] = src[j];
}

/* fgm_rowbatch_scratch (ops.c:875-877) */
int orc_rowbatch_scratch(int n_heads, int cap, int head_dim) {
  return n_heads * cap + (cap + 3) / 2 + 2 * head_dim + 64;
}

/* fgm_gather_q8r (ops.c:208-217): out = (float)q * sc[row] */
void orc_gather_q8r(float *out, const int8_t *tbl, const float *sc, int row, int k) {
  const int8_t *p = tbl + (size_t)row * k;
  for (int i = 0; i < k; i++) out[i] = (float)p[i] * sc[row];
}

/* fgm_gather_q4r (ops.c:228-251): per 64-block, 32 packed bytes; element j <
 * 32 is the low nibble of byte j, element j >= 32 the high nibble of byte
 * j - 32 (two's complement); scale f16 [row][k/64] widened exactly. */
void orc_gather_q4r(float *out, const uint8_t *tbl, const uint16_t *sc, int row, int k) {
  const int g = k / 64;
  const uint8_t *p = tbl + (size_t)row * (k / 2);
  for (int b = 0; b < g; b++) {
    const float s = orc_f16_to_f32(sc[(size_t)row * g + b]);
    for (int j = 0; j < 64; j++) {
      const uint8_t byte = p[b * 32 + (j & 31)];
      const int nib = j < 32 ? (byte & 15) : (byte >> 4);
      out[b * 64 + j] = (float)((nib ^ 8) - 8) * s;
    }
  }
}
