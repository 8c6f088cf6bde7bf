// Dense prefill GEMM on gfx950 MFMA: the M > 64 replacement for
// fgm_gemm_q8c / fgm_gemm_q4g (amx_gemm.c:333-372, 444-475) and their VNNI
// twins (vnni_gemm.c:224-322).
//
// Workgroup tile BM x BN (BN/16 n-blocks), 4 waves in a 2x2 grid, each wave
// (BM/2) x (BN/2) built from v_mfma_i32_16x16x64_i8, one 64-wide k-block per
// pipeline stage.  Operands move global -> registers -> LDS:
//   * a ring of D register stages keeps D k-blocks of loads in flight, so the
//     L2 / HBM latency is covered by D stages of matrix work;
//   * LDS is double-buffered, one barrier per k-block;
//   * A rows are stored as they are, B tiles re-laid column-major (one 64-byte
//     k-run per column); both with an 80-byte pitch, so every fragment read is
//     one conflict-free ds_read_b128;
//   * int4 tiles are sign-extended to int8 on their way into LDS.
// MFMA k-permutation: operand byte b of lane 16*g + j is k = 16*g + b.
//
// Epilogues are the reference's (see fgm_decode.hip): int8 is exact int32
// over all of K then (float)acc * (b_scale * a_scale); int4 drains its int32
// accumulators into an fp32 fma chain at the end of every scale group, in
// ascending group order, then multiplies by a_scale.
#include "fgm_common.h"
#include "fgm_kernels.h"

namespace {

constexpr int PITCH = 80;        // LDS bytes per row / column (64 + 16 pad)
constexpr int BLK = 16 * PITCH;  // one 16x64 operand block in LDS

FGM_DEV GemmProb pick(const GemmBatch& bt) {
  const int b = blockIdx.x;
  GemmProb p = bt.p[0];
  if (bt.count > 1 && b >= bt.p[1].wg0) p = bt.p[1];
  if (bt.count > 2 && b >= bt.p[2].wg0) p = bt.p[2];
  if (bt.count > 3 && b >= bt.p[3].wg0) p = bt.p[3];
  return p;
}

template <int BITS, int BM, int BN, int D>
__global__ __launch_bounds__(256) void gemm_kernel(GemmBatch bt) {
  constexpr int MBL = BM / 16, NBL = BN / 16;    // operand blocks per stage
  constexpr int MS = BM / 32, NS = BN / 32;      // 16x16 subtiles per wave
  constexpr int STAGE = (MBL + NBL) * BLK;
  constexpr int ACH = BM * 4 / 256;              // 16-byte A chunks per thread
  constexpr int BCH_TOT = (BITS == 8) ? BN * 4 : BN * 2;
  constexpr int BCH = (BCH_TOT + 255) / 256;     // 16-byte B chunks per thread
  static_assert(ACH >= 1 && MS >= 1 && NS >= 1, "tile too small");
  __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];

  const GemmProb a = pick(bt);
  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, g = l >> 4, j = l & 15;
  const int wm = w & 1, wn = w >> 1;

  const int M = a.M, N = a.N, KB = a.K >> 6;
  const int MT = (M + BM - 1) / BM;
  const int NT = (a.nblocks + NBL - 1) / NBL;
  int bid = blockIdx.x - a.wg0;
  const int ntiles = MT * NT;
  // XCD-aware order (workgroup ids go round-robin over the 8 XCDs): give each
  // XCD a contiguous run of tiles, m fastest, so tiles sharing B share an L2.
  if ((ntiles & 7) == 0 && (a.wg0 & 7) == 0) bid = (bid & 7) * (ntiles >> 3) + (bid >> 3);
  const int mt = bid % MT, nt = bid / MT;
  const int MBtot = (M + 15) >> 4;
  const int mb0 = mt * MBL;
  const int nb0 = a.n0 + nt * NBL;
  const int nbend = a.n0 + a.nblocks;
  const int gk = (BITS == 4) ? (a.group >> 6) : 1;
  const bool want_scales = BITS == 4 && a.acc_out == nullptr;

  v4i ra[D][ACH], rb[D][BCH];
  float sreg[D][NS];

  auto gload = [&](int kb, v4i* rA, v4i* rB, float* sc) {
#pragma unroll
    for (int u = 0; u < ACH; u++) {
      const int c = tid + 256 * u;
      const int mbl = c >> 6, i = (c & 63) >> 2, h = c & 3;
      const int mb = mb0 + mbl;
      rA[u] = v4i{0, 0, 0, 0};
      if (mb < MBtot) rA[u] = *(const v4i*)(a.A + (((size_t)mb * KB + kb) * 16 + i) * 64 + 16 * h);
    }
#pragma unroll
    for (int u = 0; u < BCH; u++) {
      const int c = tid + 256 * u;
      rB[u] = v4i{0, 0, 0, 0};
      if (c < BCH_TOT) {
        if (BITS == 8) {
          const int nbl = c >> 6, r = (c & 63) >> 2, h = c & 3, nb = nb0 + nbl;
          if (nb < nbend)
            rB[u] = __builtin_nontemporal_load((const v4i*)((const int8_t*)a.B +
                                               ((size_t)nb * KB + kb) * 1024 + r * 64 + 16 * h));
        } else {
          const int nbl = c >> 5, r = (c & 31) >> 1, h = c & 1, nb = nb0 + nbl;
          if (nb < nbend)
            rB[u] = __builtin_nontemporal_load((const v4i*)((const uint8_t*)a.B +
                                               ((size_t)nb * KB + kb) * 512 + r * 32 + 16 * h));
        }
      }
    }
    if (want_scales) {
      const uint16_t* bsp = (const uint16_t*)a.b_scale + (size_t)(kb / gk) * N;
#pragma unroll
      for (int ns = 0; ns < NS; ns++) {
        const int nb = nb0 + wn * NS + ns;
        sc[ns] = nb < nbend ? f16_bits_to_f32(bsp[nb * 16 + j]) : 0.0f;
      }
    }
  };
  auto swrite = [&](char* st, const v4i* rA, const v4i* rB) {
#pragma unroll
    for (int u = 0; u < ACH; u++) {
      const int c = tid + 256 * u;
      const int mbl = c >> 6, i = (c & 63) >> 2, h = c & 3;
      *(v4i*)(st + mbl * BLK + i * PITCH + 16 * h) = rA[u];
    }
    char* bs = st + MBL * BLK;
#pragma unroll
    for (int u = 0; u < BCH; u++) {
      const int c = tid + 256 * u;
      if (c < BCH_TOT) {
        if (BITS == 8) {
          const int nbl = c >> 6, r = (c & 63) >> 2, h = c & 3;
          char* base = bs + nbl * BLK + 4 * r;
#pragma unroll
          for (int e = 0; e < 4; e++) *(int32_t*)(base + (4 * h + e) * PITCH) = rB[u][e];
        } else {
          const int nbl = c >> 5, r = (c & 31) >> 1, h = c & 1;
          char* base = bs + nbl * BLK + 4 * r;
#pragma unroll
          for (int d = 0; d < 4; d++) {
            const uint32_t v = (uint32_t)rB[u][d];
            *(uint32_t*)(base + (4 * h + d) * PITCH) = nib4_to_i8x4(v & 0x0F0F0F0Fu);
            *(uint32_t*)(base + (8 + 4 * h + d) * PITCH) = nib4_to_i8x4((v >> 4) & 0x0F0F0F0Fu);
          }
        }
      }
    }
  };

  v4i acc[MS][NS];
  float cf[MS][NS][4];
#pragma unroll
  for (int x = 0; x < MS; x++)
#pragma unroll
    for (int y = 0; y < NS; y++) {
      acc[x][y] = v4i{0, 0, 0, 0};
#pragma unroll
      for (int r = 0; r < 4; r++) cf[x][y][r] = 0.0f;
    }

  // prologue: D stages in flight, stage 0 in LDS
#pragma unroll
  for (int s = 0; s < D; s++)
    if (s < KB) gload(s, ra[s], rb[s], sreg[s]);
  swrite(smem, ra[0], rb[0]);
  float scur[NS];  // int4: the scales of the stage being multiplied
#pragma unroll
  for (int ns = 0; ns < NS; ns++) scur[ns] = sreg[0][ns];
  // slot s % D holds stage s: slot 0 moves on to stage D
  if (D < KB) gload(D, ra[0], rb[0], sreg[0]);
  __syncthreads();

  for (int kb0 = 0; kb0 < KB; kb0 += D) {
#pragma unroll
    for (int u = 0; u < D; u++) {
      const int kb = kb0 + u;
      if (kb < KB) {
        // ring slot of stage kb + 1: move it to LDS, keep its scales, then
        // refill the slot with stage kb + 1 + D
        const int nx = (u + 1) % D;
        float snext[NS];
#pragma unroll
        for (int ns = 0; ns < NS; ns++) snext[ns] = sreg[nx][ns];
        if (kb + 1 < KB) swrite(smem + ((kb + 1) & 1) * STAGE, ra[nx], rb[nx]);
        if (kb + 1 + D < KB) gload(kb + 1 + D, ra[nx], rb[nx], sreg[nx]);

        const char* st = smem + (kb & 1) * STAGE;
        v4i af[MS], bf[NS];
#pragma unroll
        for (int ms = 0; ms < MS; ms++)
          af[ms] = *(const v4i*)(st + (wm * MS + ms) * BLK + j * PITCH + 16 * g);
#pragma unroll
        for (int ns = 0; ns < NS; ns++)
          bf[ns] = *(const v4i*)(st + (MBL + wn * NS + ns) * BLK + j * PITCH + 16 * g);
#pragma unroll
        for (int ms = 0; ms < MS; ms++)
#pragma unroll
          for (int ns = 0; ns < NS; ns++) acc[ms][ns] = mfma16(af[ms], bf[ns], acc[ms][ns]);

        if (BITS == 4 && ((kb + 1) % gk) == 0) {
          const int gi = kb / gk;
#pragma unroll
          for (int ms = 0; ms < MS; ms++)
#pragma unroll
            for (int ns = 0; ns < NS; ns++) {
              if (a.acc_out) {
                const int nb = nb0 + wn * NS + ns;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                  const int m = (mb0 + wm * MS + ms) * 16 + 4 * g + r;
                  if (m < M && nb < nbend)
                    a.acc_out[((size_t)gi * M + m) * a.ldacc + nb * 16 + j] = acc[ms][ns][r];
                }
              } else {
#pragma unroll
                for (int r = 0; r < 4; r++)
                  cf[ms][ns][r] = __builtin_fmaf((float)acc[ms][ns][r], scur[ns], cf[ms][ns][r]);
              }
              acc[ms][ns] = v4i{0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int ns = 0; ns < NS; ns++) scur[ns] = snext[ns];
        __syncthreads();
      }
    }
  }

  // ---- epilogue
#pragma unroll
  for (int ns = 0; ns < NS; ns++) {
    const int nb = nb0 + wn * NS + ns;
    if (nb >= nbend) continue;
    const int n = nb * 16 + j;
    const float bsn = (BITS == 8 && !a.acc_out) ? ((const float*)a.b_scale)[n] : 0.0f;
#pragma unroll
    for (int ms = 0; ms < MS; ms++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = (mb0 + wm * MS + ms) * 16 + 4 * g + r;
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

template <int BITS, int BM, int BN, int D>
hipError_t launch(const GemmBatch& in, hipStream_t st) {
  GemmBatch b = in;
  int nwg = 0;
  for (int i = 0; i < b.count; i++) {
    GemmProb& p = b.p[i];
    p.wg0 = nwg;
    nwg += ((p.M + BM - 1) / BM) * ((p.nblocks + BN / 16 - 1) / (BN / 16));
  }
  if (nwg == 0) return hipSuccess;
  hipLaunchKernelGGL((gemm_kernel<BITS, BM, BN, D>), dim3(nwg), dim3(256), 0, st, b);
  return hipGetLastError();
}

// Tile shape: the largest tile that still gives about one tile per CU.
int pick_tile(int bits, const GemmBatch& b) {
  long t128 = 0, t256 = 0, t64 = 0;
  int mmax = 0;
  for (int i = 0; i < b.count; i++) {
    const GemmProb& p = b.p[i];
    t256 += (long)((p.M + 255) / 256) * ((p.nblocks + 7) / 8);
    t128 += (long)((p.M + 127) / 128) * ((p.nblocks + 7) / 8);
    t64 += (long)((p.M + 127) / 128) * ((p.nblocks + 3) / 4);
    if (p.M > mmax) mmax = p.M;
  }
  if (bits == 8 && mmax > 128 && t256 >= 256) return 2;  // 256 x 128
  if (t128 >= 192) return 1;                            // 128 x 128
  (void)t64;
  return 0;                                             // 128 x 64
}

}  // namespace

hipError_t fgm_launch_gemm(int bits, const GemmBatch& b, hipStream_t st) {
  const int t = pick_tile(bits, b);
  if (bits == 8) {
    if (t == 2) return launch<8, 256, 128, 4>(b, st);
    if (t == 1) return launch<8, 128, 128, 4>(b, st);
    return launch<8, 128, 64, 4>(b, st);
  }
  if (t >= 1) return launch<4, 128, 128, 4>(b, st);
  return launch<4, 128, 64, 4>(b, st);
}
