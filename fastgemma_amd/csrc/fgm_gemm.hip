// Dense prefill GEMM on gfx950 MFMA: the M >= 65 replacement for
// fgm_gemm_q8c / fgm_gemm_q4g (amx_gemm.c:333-372, 444-475) and their VNNI
// twins (vnni_gemm.c:224-322).
//
// Workgroup tile 128 rows x 128 columns (8 n-blocks), 4 waves in a 2x2 grid,
// each wave 64x64 = 4x4 v_mfma_i32_16x16x64_i8 per 64-wide k-block.  Both
// operands are staged through LDS, double-buffered, one barrier per k-block:
//   A: packed A rows copied as they are, 80-byte row pitch;
//   B: int8 tiles re-laid column-major (one 64-byte k-run per column, 80-byte
//      pitch); int4 tiles are sign-extended to int8 on the way in.
// With the 16-byte pad both fragment reads are single conflict-free
// ds_read_b128s.  This kernel's MFMA k-permutation is the identity: operand
// byte b of lane 16*g + j is k = 16*g + b.
//
// Epilogues are the reference's (see fgm_decode.hip); int4 drains its int32
// accumulators into an fp32 fma chain at the end of every scale group.
#include "fgm_common.h"
#include "fgm_kernels.h"

namespace {

constexpr int BM = 128;            // rows per workgroup tile
constexpr int BNB = 8;             // n-blocks per workgroup tile (128 columns)
constexpr int PITCH = 80;          // LDS bytes per row / column (64 + 16 pad)
constexpr int BLK = 16 * PITCH;    // one 16x64 operand block in LDS
constexpr int STAGE = (BM / 16 + BNB) * BLK;

template <int BITS>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs a, int MT, int NT, int nblocks) {
  __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];
  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, g = l >> 4, j = l & 15;
  const int wm = w & 1, wn = w >> 1;

  // XCD-aware tile order: consecutive workgroup ids land on different XCDs,
  // so give each XCD a contiguous run of tiles (m fastest) to share B in L2.
  int bid = blockIdx.x;
  const int ntiles = MT * NT;
  if ((ntiles & 7) == 0) bid = (bid & 7) * (ntiles >> 3) + (bid >> 3);
  const int mt = bid % MT, nt = bid / MT;

  const int M = a.M, N = a.N, KB = a.K >> 6;
  const int MBtot = (M + 15) >> 4;
  const int mb0 = mt * (BM / 16);
  const int nb0 = a.n0 + nt * BNB;
  const int nbend = a.n0 + nblocks;
  const int gk = (BITS == 4) ? (a.group >> 6) : 1;

  // ---- global -> register staging for one k-block
  v4i ra[2], rb[2];
  auto gload = [&](int kb) {
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int c = tid + 256 * u;
      const int mbl = c >> 6, i = (c & 63) >> 2, h = c & 3;
      const int mb = mb0 + mbl;
      ra[u] = v4i{0, 0, 0, 0};
      if (mb < MBtot)
        ra[u] = *(const v4i*)(a.A + (((size_t)mb * KB + kb) * 16 + i) * 64 + 16 * h);
    }
    if (BITS == 8) {
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int c = tid + 256 * u;
        const int nbl = c >> 6, r = (c & 63) >> 2, h = c & 3;
        const int nb = nb0 + nbl;
        rb[u] = v4i{0, 0, 0, 0};
        if (nb < nbend)
          rb[u] = __builtin_nontemporal_load(
              (const v4i*)((const int8_t*)a.B + ((size_t)nb * KB + kb) * 1024 + r * 64 + 16 * h));
      }
    } else {
      const int nbl = tid >> 5, r = (tid & 31) >> 1, h = tid & 1;
      const int nb = nb0 + nbl;
      rb[0] = v4i{0, 0, 0, 0};
      if (nb < nbend)
        rb[0] = __builtin_nontemporal_load(
            (const v4i*)((const uint8_t*)a.B + ((size_t)nb * KB + kb) * 512 + r * 32 + 16 * h));
    }
  };
  auto swrite = [&](char* st) {
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int c = tid + 256 * u;
      const int mbl = c >> 6, i = (c & 63) >> 2, h = c & 3;
      *(v4i*)(st + mbl * BLK + i * PITCH + 16 * h) = ra[u];
    }
    char* bs = st + (BM / 16) * BLK;
    if (BITS == 8) {
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int c = tid + 256 * u;
        const int nbl = c >> 6, r = (c & 63) >> 2, h = c & 3;
        char* base = bs + nbl * BLK + 4 * r;
        const uint32_t v[4] = {(uint32_t)rb[u][0], (uint32_t)rb[u][1], (uint32_t)rb[u][2],
                               (uint32_t)rb[u][3]};
#pragma unroll
        for (int e = 0; e < 4; e++) *(uint32_t*)(base + (4 * h + e) * PITCH) = v[e];
      }
    } else {
      const int nbl = tid >> 5, r = (tid & 31) >> 1, h = tid & 1;
      char* base = bs + nbl * BLK + 4 * r;
      const uint32_t v[4] = {(uint32_t)rb[0][0], (uint32_t)rb[0][1], (uint32_t)rb[0][2],
                             (uint32_t)rb[0][3]};
#pragma unroll
      for (int d = 0; d < 4; d++) {
        *(uint32_t*)(base + (4 * h + d) * PITCH) = nib4_to_i8x4(v[d] & 0x0F0F0F0Fu);
        *(uint32_t*)(base + (8 + 4 * h + d) * PITCH) = nib4_to_i8x4((v[d] >> 4) & 0x0F0F0F0Fu);
      }
    }
  };

  v4i acc[4][4];
  float cf[4][4][4];
#pragma unroll
  for (int x = 0; x < 4; x++)
#pragma unroll
    for (int y = 0; y < 4; y++) {
      acc[x][y] = v4i{0, 0, 0, 0};
      if (BITS == 4)
#pragma unroll
        for (int r = 0; r < 4; r++) cf[x][y][r] = 0.0f;
    }
  float sc[4] = {0.f, 0.f, 0.f, 0.f};

  gload(0);
  swrite(smem);
  __syncthreads();

  for (int kb = 0; kb < KB; kb++) {
    if (kb + 1 < KB) gload(kb + 1);
    if (BITS == 4 && !a.acc_out && (kb % gk) == 0) {
      // this group's scales, one per owned column, consumed at its last k-block
      const uint16_t* bsp = (const uint16_t*)a.b_scale + (size_t)(kb / gk) * N;
#pragma unroll
      for (int ns = 0; ns < 4; ns++) {
        const int nb = nb0 + wn * 4 + ns;
        sc[ns] = nb < nbend ? f16_bits_to_f32(bsp[nb * 16 + j]) : 0.0f;
      }
    }
    const char* st = smem + (kb & 1) * STAGE;
    v4i af[4], bf[4];
#pragma unroll
    for (int ms = 0; ms < 4; ms++)
      af[ms] = *(const v4i*)(st + (wm * 4 + ms) * BLK + j * PITCH + 16 * g);
#pragma unroll
    for (int ns = 0; ns < 4; ns++)
      bf[ns] = *(const v4i*)(st + (BM / 16 + wn * 4 + ns) * BLK + j * PITCH + 16 * g);
#pragma unroll
    for (int ms = 0; ms < 4; ms++)
#pragma unroll
      for (int ns = 0; ns < 4; ns++) acc[ms][ns] = mfma16(af[ms], bf[ns], acc[ms][ns]);

    if (BITS == 4 && ((kb + 1) % gk) == 0) {
      const int gi = kb / gk;
#pragma unroll
      for (int ms = 0; ms < 4; ms++)
#pragma unroll
        for (int ns = 0; ns < 4; ns++) {
          if (a.acc_out) {
            const int nb = nb0 + wn * 4 + ns;
#pragma unroll
            for (int r = 0; r < 4; r++) {
              const int m = (mb0 + wm * 4 + ms) * 16 + 4 * g + r;
              if (m < M && nb < nbend)
                a.acc_out[((size_t)gi * M + m) * a.ldacc + nb * 16 + j] = acc[ms][ns][r];
            }
          } else {
#pragma unroll
            for (int r = 0; r < 4; r++)
              cf[ms][ns][r] = __builtin_fmaf((float)acc[ms][ns][r], sc[ns], cf[ms][ns][r]);
          }
          acc[ms][ns] = v4i{0, 0, 0, 0};
        }
    }

    if (kb + 1 < KB) swrite(smem + ((kb + 1) & 1) * STAGE);
    __syncthreads();
  }

  // ---- epilogue
#pragma unroll
  for (int ns = 0; ns < 4; ns++) {
    const int nb = nb0 + wn * 4 + ns;
    if (nb >= nbend) continue;
    const int n = nb * 16 + j;
    // raw-accumulator mode passes no scales
    const float bsn = (BITS == 8 && !a.acc_out) ? ((const float*)a.b_scale)[n] : 0.0f;
#pragma unroll
    for (int ms = 0; ms < 4; ms++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = (mb0 + wm * 4 + ms) * 16 + 4 * g + r;
        if (m >= M) continue;
        if (BITS == 8) {
          if (a.acc_out) a.acc_out[(size_t)m * a.ldacc + n] = acc[ms][ns][r];
          else a.C[(size_t)m * a.ldc + n] = (float)acc[ms][ns][r] * (bsn * a.a_scale[m]);
        } else if (!a.acc_out) {
          a.C[(size_t)m * a.ldc + n] = cf[ms][ns][r] * a.a_scale[m];
        }
      }
  }
}

}  // namespace

hipError_t fgm_launch_gemm(int bits, const GemmArgs& a, int nblocks, hipStream_t st) {
  const int MT = (a.M + BM - 1) / BM;
  const int NT = (nblocks + BNB - 1) / BNB;
  const dim3 grid(MT * NT), block(256);
  if (bits == 8) hipLaunchKernelGGL(gemm_kernel<8>, grid, block, 0, st, a, MT, NT, nblocks);
  else hipLaunchKernelGGL(gemm_kernel<4>, grid, block, 0, st, a, MT, NT, nblocks);
  return hipGetLastError();
}
