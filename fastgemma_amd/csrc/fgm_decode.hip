// Decode / skinny GEMM (M <= 64) on gfx950: a weight stream.
//
// Replaces fgm_gemm_q8c_vnni / fgm_gemm_q4g_vnni (vnni_gemm.c:224-245,
// 291-322) for the row counts where the GEMM is bound by reading B.  One
// launch serves up to FGM_MAX_BATCH independent GEMMs of the same weight type
// (the reference issues q/k/v and gate/up as separate GEMMs on one
// activation, forward.rs:484,499-500,619-622).
//
// One workgroup owns one 16-column n-block of one GEMM and all of K.  Its W
// waves split K into contiguous ranges (whole scale groups for int4).  Every
// wave issues the weight loads of a whole chunk of KT 64-wide k-blocks first,
// then the activation fragments (L2-resident) and the group scales, and only
// then multiplies: one v_mfma_i32_16x16x64_i8 per tile and 16-row m-block.
// Loop bounds and tile indices are wave-uniform scalars; activation rows >= M
// and out-of-range scales are masked by buffer range checks, not branches.
//
// MFMA operand mapping (lane l = 16*g + j): A row j / B column j, operand byte
// 4*t + e carries k = 16*g + 4*t + e.  A fragment = one 16-byte load of the
// packed-A row; B fragment = four dwords of tile rows 4g..4g+3 (int8: row r,
// column j at byte 64*r + 4*j; int4: packed row r, dword j%8, low nibbles for
// j < 8, high nibbles for j >= 8).
//
// Epilogues, in the reference's operation order:
//   q8c: the waves' int32 partials are summed exactly in LDS, then
//        C = (float)acc * (b_scale[n] * a_scale[m])          vnni_gemm.c:206-219
//   q4g: each wave parks its per-group int32 sums in LDS ([g][m][16], so the
//        parking and the chain both touch consecutive words -- no bank
//        conflicts); after one barrier one lane per output runs the chain in
//        ascending g from C = 0:
//        C = fmaf((float)acc_g, f16(b_scale[g][n]), C), then C *= a_scale[m]
//                                                             vnni_gemm.c:258-285, 316-321
#include "fgm_common.h"
#include "fgm_kernels.h"

namespace {

constexpr int SPT = 4;  // group scales prefetched per thread

// The problem a workgroup belongs to, chosen with uniform selects so the
// kernel-argument array is never indexed dynamically.
FGM_DEV GemmProb pick(const GemmBatch& bt) {
  const int b = blockIdx.x;
  GemmProb p = bt.p[0];
  if (bt.count > 1 && b >= bt.p[1].wg0) p = bt.p[1];
  if (bt.count > 2 && b >= bt.p[2].wg0) p = bt.p[2];
  if (bt.count > 3 && b >= bt.p[3].wg0) p = bt.p[3];
  return p;
}

template <int BITS, int MB>
struct Stream {
  __amdgpu_buffer_rsrc_t rb, ra;
  uint32_t bvoff;          // lane part of the weight-tile offset
  uint32_t avoff[MB];      // lane part of the A-fragment offset (FGM_OOB if row >= M)
  int nib_shift, gk, g, j, M, KB;
  v4i acc[MB];
  int32_t* P;              // int4: group sums [g][m][16] (as float unless raw)
  bool raw;                // keep the int32 sums (raw-accumulator mode)

  // n tiles starting at k-block t0: all loads first, then the matrix work
  template <int NT>
  __device__ __forceinline__ void chunk(int t0) {
    constexpr int TB = (BITS == 8) ? 1024 : 512;
    int32_t braw[NT][4];
    v4i af[NT][MB];
#pragma unroll
    for (int u = 0; u < NT; u++)
#pragma unroll
      for (int t = 0; t < 4; t++)
        braw[u][t] = buf_load_b32(rb, bvoff + t * (BITS == 8 ? 64 : 32), (uint32_t)(t0 + u) * TB);
#pragma unroll
    for (int u = 0; u < NT; u++)
#pragma unroll
      for (int mb = 0; mb < MB; mb++) af[u][mb] = buf_load_b128(ra, avoff[mb], (uint32_t)(t0 + u) * 1024);
#pragma unroll
    for (int u = 0; u < NT; u++) {
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
      const int kb = t0 + u;
      if (BITS == 4 && ((kb + 1) % gk) == 0) {
        const int gi = kb / gk;
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const int m = mb * 16 + 4 * g + r;
            // (float)acc_g here is the conversion the epilogue would make:
            // the reference converts the exact int32 with round-to-nearest
            if (m < M) P[(gi * M + m) * 16 + j] = raw ? acc[mb][r] : __float_as_int((float)acc[mb][r]);
          }
#pragma unroll
        for (int mb = 0; mb < MB; mb++) acc[mb] = v4i{0, 0, 0, 0};
      }
    }
  }
};

template <int BITS, int MB, int KT>
__global__ __launch_bounds__(1024) void decode_kernel(GemmBatch bt) {
  extern __shared__ __attribute__((aligned(16))) int32_t lds[];
  const GemmProb a = pick(bt);
  const int W = blockDim.x >> 6;
  const int tid = threadIdx.x;
  const int w = wave_id(), l = tid & 63, g = l >> 4, j = l & 15;
  const int nb = a.n0 + (blockIdx.x - a.wg0);
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

  const bool want_scales = BITS == 4 && a.acc_out == nullptr;
  // 1. this n-block's group scales, two columns per dword (in flight with
  //    the weights; whole dwords so no load has to be waited for early)
  uint32_t sreg[SPT];
  if (want_scales) {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.b_scale, (uint32_t)NG * N * 2);
#pragma unroll
    for (int u = 0; u < SPT; u++) {
      const int i = tid + u * (int)blockDim.x;  // group i >> 3, columns 2 (i & 7) + {0, 1}
      const uint32_t off = i < NG * 8 ? (uint32_t)(((i >> 3) * N + nb * 16 + 2 * (i & 7)) * 2) : FGM_OOB;
      sreg[u] = (uint32_t)buf_load_b32(rs, off, 0);
    }
  }

  Stream<BITS, MB> s;
  const uint32_t tile_bytes = (BITS == 8) ? 1024u : 512u;
  s.rb = make_rsrc((const int8_t*)a.B + (size_t)nb * KB * tile_bytes, (uint32_t)KB * tile_bytes);
  s.ra = make_rsrc(a.A, (uint32_t)((M + 15) / 16 * KB * 1024));
  s.bvoff = (BITS == 8) ? (uint32_t)(256 * g + 4 * j) : (uint32_t)(128 * g + 4 * (j & 7));
#pragma unroll
  for (int mb = 0; mb < MB; mb++)
    s.avoff[mb] = (mb * 16 + j < M) ? (uint32_t)(mb * KB * 1024 + j * 64 + 16 * g) : FGM_OOB;
  s.nib_shift = (j >= 8) ? 4 : 0;
  s.gk = gk;
  s.g = g;
  s.j = j;
  s.M = M;
  s.KB = KB;
  s.P = lds;
  s.raw = a.acc_out != nullptr;
#pragma unroll
  for (int mb = 0; mb < MB; mb++) s.acc[mb] = v4i{0, 0, 0, 0};

  // 2. the weight stream, KT k-blocks at a time, then the remainder one by one
  int t0 = tb;
  for (; t0 + KT <= te; t0 += KT) s.template chunk<KT>(t0);
  for (; t0 < te; t0++) s.template chunk<1>(t0);

  // int4 scales in LDS, widened to f32 (exact): [g][16]
  float* SF = (float*)(lds + (size_t)NG * M * 16);
  if (want_scales) {
#pragma unroll
    for (int u = 0; u < SPT; u++) {
      const int i = tid + u * (int)blockDim.x;
      if (i < NG * 8) {
        SF[2 * i] = f16_bits_to_f32((uint16_t)(sreg[u] & 0xFFFF));
        SF[2 * i + 1] = f16_bits_to_f32((uint16_t)(sreg[u] >> 16));
      }
    }
    // the host guarantees NG * 8 <= SPT * blockDim.x
  }
  if (BITS == 8) {
    int32_t* R = lds + (size_t)w * M * 16;
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = mb * 16 + 4 * g + r;
        if (m < M) R[m * 16 + j] = s.acc[mb][r];
      }
  }
  __syncthreads();

  const int ncol = nb * 16;
  for (int o = tid; o < M * 16; o += blockDim.x) {
    const int m = o >> 4, c = o & 15;
    if (BITS == 8) {
      int32_t sum = 0;
      for (int ww = 0; ww < W; ww++) sum += lds[((size_t)ww * M + m) * 16 + c];
      if (a.acc_out) {
        a.acc_out[(size_t)m * a.ldacc + ncol + c] = sum;
      } else {
        const float sc = ((const float*)a.b_scale)[ncol + c] * a.a_scale[m];
        a.C[(size_t)m * a.ldc + ncol + c] = (float)sum * sc;
      }
    } else {
      // consecutive outputs read consecutive LDS words: conflict-free
      if (a.acc_out) {
        for (int gg = 0; gg < NG; gg++)
          a.acc_out[((size_t)gg * M + m) * a.ldacc + ncol + c] = lds[((size_t)gg * M + m) * 16 + c];
      } else {
        // the chain is serial; keep it fed: per batch of CH groups, all LDS
        // reads first, then CH back-to-back fmas on f32 operands
        const float* PF = (const float*)lds;
        constexpr int CH = 16;
        float cacc = 0.0f;
        int gg = 0;
        for (; gg + CH <= NG; gg += CH) {
          float vf[CH], sf[CH];
#pragma unroll
          for (int e = 0; e < CH; e++) {
            vf[e] = PF[((size_t)(gg + e) * M + m) * 16 + c];
            sf[e] = SF[(gg + e) * 16 + c];
          }
#pragma unroll
          for (int e = 0; e < CH; e++) cacc = __builtin_fmaf(vf[e], sf[e], cacc);
        }
        for (; gg < NG; gg++)
          cacc = __builtin_fmaf(PF[((size_t)gg * M + m) * 16 + c], SF[gg * 16 + c], cacc);
        a.C[(size_t)m * a.ldc + ncol + c] = cacc * a.a_scale[m];
      }
    }
  }
}

template <int BITS, int MB, int KT>
hipError_t launch_decode(const GemmBatch& bt, int W, size_t lds, int nwg, hipStream_t st) {
  static bool attr_set = false;  // up to the full 160 KB of LDS
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void*)decode_kernel<BITS, MB, KT>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  hipLaunchKernelGGL((decode_kernel<BITS, MB, KT>), dim3(nwg), dim3(W * 64), lds, st, bt);
  return hipGetLastError();
}

int kt_for(int MB) { return MB == 1 ? 8 : 4; }

// Waves per workgroup for one GEMM: about TPW k-blocks each (more, shorter
// waves keep more of the weight stream in flight), whole groups, at most 16;
// enough threads to hold the prefetched scales.
constexpr int TPW = 4;
int waves_for(int bits, int M, int K, int group) {
  const int KB = K / 64;
  int W = (KB + TPW - 1) / TPW;
  if (W > 16) W = 16;
  if (bits == 4) {
    const int NG = KB / (group / 64);
    if (W > NG) W = NG;
    while (W < 16 && NG * 8 > SPT * 64 * W) W++;
  }
  return W < 1 ? 1 : W;
}

size_t lds_for(int bits, int M, int K, int group, int W) {
  if (bits == 4) {
    const int NG = (K / 64) / (group / 64);
    return (size_t)NG * M * 16 * 4 + (size_t)NG * 16 * 4;
  }
  return (size_t)W * M * 16 * 4;
}

}  // namespace

size_t fgm_decode_lds_bytes(int bits, int M, int K, int group) {
  return lds_for(bits, M, K, group, bits == 4 ? waves_for(bits, M, K, group) : 16);
}

bool fgm_decode_fits(int bits, int M, int K, int group) {
  if (M < 1 || M > 64) return false;
  if ((size_t)((M + 15) / 16) * K * 16 > 0x7FFFFFFFu) return false;  // buffer offsets
  if (bits == 4) {
    const int NG = (K / 64) / (group / 64);
    if (NG * 8 > SPT * 1024) return false;
  }
  return fgm_decode_lds_bytes(bits, M, K, group) <= 160 * 1024;
}

hipError_t fgm_launch_decode(int bits, const GemmBatch& in, hipStream_t st) {
  GemmBatch bt = in;
  int W = 1, MB = 0, nwg = 0;
  size_t lds = 0;
  for (int i = 0; i < bt.count; i++) {
    GemmProb& p = bt.p[i];
    const int w = waves_for(bits, p.M, p.K, p.group);
    if (w > W) W = w;
    const int mb = (p.M + 15) / 16;
    if (mb > MB) MB = mb;
    p.wg0 = nwg;
    nwg += p.nblocks;
  }
  for (int i = 0; i < bt.count; i++) {
    const GemmProb& p = bt.p[i];
    const size_t need = lds_for(bits, p.M, p.K, p.group, W);
    if (need > lds) lds = need;
  }
  if (nwg == 0) return hipSuccess;
  if (bits == 8) {
    switch (MB) {
      case 1: return launch_decode<8, 1, 8>(bt, W, lds, nwg, st);
      case 2: return launch_decode<8, 2, 4>(bt, W, lds, nwg, st);
      case 3: return launch_decode<8, 3, 4>(bt, W, lds, nwg, st);
      case 4: return launch_decode<8, 4, 4>(bt, W, lds, nwg, st);
    }
  } else {
    switch (MB) {
      case 1: return launch_decode<4, 1, 8>(bt, W, lds, nwg, st);
      case 2: return launch_decode<4, 2, 4>(bt, W, lds, nwg, st);
      case 3: return launch_decode<4, 3, 4>(bt, W, lds, nwg, st);
      case 4: return launch_decode<4, 4, 4>(bt, W, lds, nwg, st);
    }
  }
  return hipErrorInvalidValue;
}
