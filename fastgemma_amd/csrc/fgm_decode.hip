// Decode / skinny GEMM (M <= 64) on gfx950: a weight stream.
//
// Replaces fgm_gemm_q8c_vnni / fgm_gemm_q4g_vnni (vnni_gemm.c:224-245,
// 291-322) for the row counts where the GEMM is bound by reading B.
//
// One workgroup owns one 16-column n-block and all of K.  Its W waves split K
// into contiguous ranges (whole scale groups for int4), so N=2048 shapes still
// put 16 waves on a CU.  Every wave issues the loads for a whole chunk of KT
// 64-wide k-blocks before it multiplies: four dword loads per lane per tile,
// each covering 256 contiguous bytes of the tile per wave (int8), or 128
// unique bytes of the 512-byte packed tile (int4; lanes j and j+8 share a
// dword and take its low / high nibbles).  Nibbles are sign-extended in
// registers and the tile goes through one v_mfma_i32_16x16x64_i8 per 16-row
// m-block -- the matrix core does the MACs, VALU only unpacks.
//
// Epilogues, in the reference's operation order:
//   q8c: int32 partials of the waves are summed exactly in LDS, then
//        C = (float)acc * (b_scale[n] * a_scale[m])          vnni_gemm.c:208-219
//   q4g: each wave stores its per-group int32 sums in LDS; after one barrier
//        one lane per output runs the chain in ascending g from C = 0:
//        C = fmaf((float)acc_g, f16(b_scale[g][n]), C), then C *= a_scale[m]
//                                                             vnni_gemm.c:258-285, 316-321
#include "fgm_common.h"
#include "fgm_kernels.h"

namespace {

template <int BITS, int MB, int KT>
__global__ __launch_bounds__(1024) void decode_kernel(GemmArgs a) {
  extern __shared__ int32_t lds[];
  const int W = blockDim.x >> 6;
  const int w = threadIdx.x >> 6;
  const int l = threadIdx.x & 63;
  const int g = l >> 4, j = l & 15;
  const int nb = a.n0 + blockIdx.x;
  const int M = a.M, N = a.N, KB = a.K >> 6;
  const int gk = (BITS == 4) ? (a.group >> 6) : 1;
  const int NG = (BITS == 4) ? KB / gk : 1;

  // contiguous k-block range of this wave (whole groups for int4)
  int tb, te;
  if (BITS == 4) {
    tb = (int)((long)w * NG / W) * gk;
    te = (int)((long)(w + 1) * NG / W) * gk;
  } else {
    tb = (int)((long)w * KB / W);
    te = (int)((long)(w + 1) * KB / W);
  }

  // int4: stage this n-block's group scales in LDS while B is in flight
  uint16_t* S = nullptr;
  if (BITS == 4 && a.b_scale) {
    S = (uint16_t*)(lds + (size_t)NG * M * 16);
    const uint16_t* bs = (const uint16_t*)a.b_scale;
    for (int i = threadIdx.x; i < NG * 16; i += blockDim.x)
      S[i] = bs[(size_t)(i >> 4) * N + nb * 16 + (i & 15)];
  }

  v4i acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; mb++) acc[mb] = v4i{0, 0, 0, 0};

  const int32_t* A32 = (const int32_t*)a.A;
  const int nib_shift = (j >= 8) ? 4 : 0;

  for (int t0 = tb; t0 < te; t0 += KT) {
    int32_t braw[KT][4];
    v4i af[KT][MB];
    // issue every load of the chunk first
#pragma unroll
    for (int u = 0; u < KT; u++) {
      const int kb = t0 + u;
      if (kb < te) {
        if (BITS == 8) {
          const int32_t* bp = (const int32_t*)a.B + ((size_t)nb * KB + kb) * 256;
#pragma unroll
          for (int t = 0; t < 4; t++) braw[u][t] = __builtin_nontemporal_load(bp + 64 * t + l);
        } else {
          const int32_t* bp = (const int32_t*)a.B + ((size_t)nb * KB + kb) * 128;
#pragma unroll
          for (int t = 0; t < 4; t++)
            braw[u][t] = __builtin_nontemporal_load(bp + (4 * t + g) * 8 + (j & 7));
        }
#pragma unroll
        for (int mb = 0; mb < MB; mb++) {
          const int row = mb * 16 + j;
          if (row < M) {
            const int32_t* ap = A32 + (((size_t)mb * KB + kb) * 16 + j) * 16 + g;
            af[u][mb] = v4i{ap[0], ap[4], ap[8], ap[12]};
          } else {
            af[u][mb] = v4i{0, 0, 0, 0};
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < KT; u++) {
      const int kb = t0 + u;
      if (kb < te) {
        v4i bv;
        if (BITS == 8) {
          bv = v4i{braw[u][0], braw[u][1], braw[u][2], braw[u][3]};
        } else {
#pragma unroll
          for (int t = 0; t < 4; t++)
            bv[t] = (int)nib4_to_i8x4(((uint32_t)braw[u][t] >> nib_shift) & 0x0F0F0F0Fu);
        }
#pragma unroll
        for (int mb = 0; mb < MB; mb++) acc[mb] = mfma16(af[u][mb], bv, acc[mb]);
        if (BITS == 4 && ((kb + 1) % gk) == 0) {
          // group complete: park its int32 sums (rows < M) and restart
          int32_t* P = lds + (size_t)(kb / gk) * M * 16;
#pragma unroll
          for (int mb = 0; mb < MB; mb++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
              const int m = mb * 16 + 4 * g + r;
              if (m < M) P[m * 16 + j] = acc[mb][r];
            }
#pragma unroll
          for (int mb = 0; mb < MB; mb++) acc[mb] = v4i{0, 0, 0, 0};
        }
      }
    }
  }

  if (BITS == 8) {
    int32_t* R = lds + (size_t)w * M * 16;
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = mb * 16 + 4 * g + r;
        if (m < M) R[m * 16 + j] = acc[mb][r];
      }
  }
  __syncthreads();

  const int ncol = nb * 16;
  for (int o = threadIdx.x; o < M * 16; o += blockDim.x) {
    const int m = o >> 4, c = o & 15;
    if (BITS == 8) {
      int32_t s = 0;
      for (int ww = 0; ww < W; ww++) s += lds[((size_t)ww * M + m) * 16 + c];
      if (a.acc_out) {
        a.acc_out[(size_t)m * a.ldacc + ncol + c] = s;
      } else {
        const float sc = ((const float*)a.b_scale)[ncol + c] * a.a_scale[m];
        a.C[(size_t)m * a.ldc + ncol + c] = (float)s * sc;
      }
    } else {
      if (a.acc_out) {
        for (int gg = 0; gg < NG; gg++)
          a.acc_out[((size_t)gg * M + m) * a.ldacc + ncol + c] = lds[((size_t)gg * M + m) * 16 + c];
      } else {
        float cacc = 0.0f;
        for (int gg = 0; gg < NG; gg++)
          cacc = __builtin_fmaf((float)lds[((size_t)gg * M + m) * 16 + c],
                                f16_bits_to_f32(S[gg * 16 + c]), cacc);
        a.C[(size_t)m * a.ldc + ncol + c] = cacc * a.a_scale[m];
      }
    }
  }
}

template <int BITS, int MB, int KT>
hipError_t launch_decode(const GemmArgs& a, int nblocks, hipStream_t st) {
  const int KB = a.K / 64;
  int W;
  size_t lds;
  if (BITS == 4) {
    const int gk = a.group / 64, NG = KB / gk;
    // one wave per ~KT k-blocks, whole groups per wave, at most 16 waves
    W = (KB + KT - 1) / KT;
    if (W > 16) W = 16;
    if (W > NG) W = NG;
    lds = (size_t)NG * a.M * 16 * 4 + (size_t)NG * 16 * 2;
  } else {
    W = (KB + KT - 1) / KT;
    if (W > 16) W = 16;
    if (W < 1) W = 1;
    lds = (size_t)W * a.M * 16 * 4;
  }
  static bool attr_set = false;  // kernels may use up to the full 160 KB of LDS
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)decode_kernel<BITS, MB, KT>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((decode_kernel<BITS, MB, KT>), dim3(nblocks), dim3(W * 64), lds, st, a);
  return hipGetLastError();
}

}  // namespace

size_t fgm_decode_lds_bytes(int bits, int M, int K, int group) {
  const int KB = K / 64;
  if (bits == 4) {
    const int NG = KB / (group / 64);
    return (size_t)NG * M * 16 * 4 + (size_t)NG * 16 * 2;
  }
  return (size_t)16 * M * 16 * 4;
}

hipError_t fgm_launch_decode(int bits, const GemmArgs& a, int nblocks, hipStream_t st) {
  const int MB = (a.M + 15) / 16;
  if (bits == 8) {
    switch (MB) {
      case 1: return launch_decode<8, 1, 8>(a, nblocks, st);
      case 2: return launch_decode<8, 2, 4>(a, nblocks, st);
      case 3: return launch_decode<8, 3, 4>(a, nblocks, st);
      case 4: return launch_decode<8, 4, 4>(a, nblocks, st);
    }
  } else {
    const int gk = a.group / 64;
    switch (MB) {
      case 1: return launch_decode<4, 1, 8>(a, nblocks, st);
      case 2: return launch_decode<4, 2, 4>(a, nblocks, st);
      case 3: return launch_decode<4, 3, 4>(a, nblocks, st);
      case 4: return launch_decode<4, 4, 4>(a, nblocks, st);
    }
    (void)gk;
  }
  return hipErrorInvalidValue;
}
