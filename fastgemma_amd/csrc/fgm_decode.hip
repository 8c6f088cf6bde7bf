// Decode / skinny GEMM (M <= 64) on gfx950: a weight stream.
//
// Replaces fgm_gemm_q8c_vnni / fgm_gemm_q4g_vnni (vnni_gemm.c:224-245,
// 291-322) for the row counts where the GEMM is bound by reading B.  One
// launch serves up to FGM_MAX_BATCH independent GEMMs of the same weight type
// (the reference issues q/k/v and gate/up as separate GEMMs on one
// activation, forward.rs:484,499-500,619-622).
//
// Work decomposition (chosen on the host, plan_split and fgm_launch_decode
// below): a workgroup owns NBW 16-column n-blocks of one GEMM; each n-block's
// K is split into KS contiguous ranges of TW 64-wide k-blocks (whole scale
// groups for int4), one wave per range, so a workgroup has NBW * KS waves.
// Every wave streams about 4 KB of weights with all of its loads in flight at
// once: it issues the weight loads of up to CT tiles and their activation
// fragments (L2-resident) before it multiplies anything.  Loop bounds and
// tile indices are wave-uniform scalars; tiles past a wave's range and
// activation rows >= M are masked by buffer range checks, not branches.
//
// MFMA operand mapping (v_mfma_i32_16x16x64_i8, lane l = 16*g + j): A row j /
// B column j, operand byte 4*t + e carries k = 16*g + 4*t + e, i.e. k-tile row
// r = 4*g + t of the [k/4][n][k%4] layout.
//   int8 B: the dword of row r, column j (byte 64*r + 4*j).
//   int4 B: packed row r holds column c (c < 8) in the low and column c + 8
//     in the high nibbles of its dword c (lanes j and j + 8 load the same
//     dword).  The lane keeps its nibble in the high half of each byte:
//     (x << 4) & 0xF0F0F0F0 for j < 8, x & 0xF0F0F0F0 for j >= 8.  A two's-
//     complement nibble v in bits 7..4 of a byte is the int8 16 * v, so the
//     MFMA accumulates exactly 16 * acc with two VALU operations per dword.
//   A: one 16-byte load of the packed-A row per fragment.  M <= 8: lanes
//     j < 8 load row j of an even k-tile and lanes j >= 8 row j - 8 of the
//     following one; the odd tile's operand is moved into lanes 0-7 by a DPP
//     rotation by 8 lanes.  Rows 8-15 of those products are never read.
//     M > 8: one fragment per tile and 16-row m-block.
//
// Epilogues, in the reference's operation order:
//   q8c: the KS waves' int32 partials of an n-block are summed exactly in LDS,
//        C = (float)acc * (b_scale[n] * a_scale[m])          vnni_gemm.c:206-219
//   q4g: each wave parks (float)(16 * acc_g) of its groups in LDS, laid out
//        [m][column][group] with a padded group pitch so that the chain below
//        reads four groups per 16-byte load without bank conflicts; the group
//        scales are parked the same way, as f32(b_scale) / 16.  Both factors are powers of
//        two, so (16 a) * (s / 16) is the exact product a * s and every fmaf
//        rounds the same value as the reference's.  After one barrier one lane
//        per output runs the chain in ascending g from 0:
//        C = fmaf((float)acc_g, f16(b_scale[g][n]), C), then C *= a_scale[m]
//                                                             vnni_gemm.c:258-285, 316-321
#include "fgm_common.h"
#include "fgm_kernels.h"

namespace {

constexpr int MAX_WAVES = 16;
constexpr int SPT = 4;             // group-scale dwords prefetched per thread
constexpr int DPP_ROW_ROR8 = 0x128;

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

// the value of lane l ^ 8 (a rotation by 8 within every 16-lane row)
FGM_DEV int ror8(int v) { return __builtin_amdgcn_mov_dpp(v, DPP_ROW_ROR8, 0xF, 0xF, false); }

// Group pitch (words) of the parked int4 sums and scales: a multiple of four
// with an odd number of quads, so that 16-byte reads of 16 consecutive
// columns hit distinct banks.
__host__ __device__ inline int group_pitch(int ng) {
  const int r4 = (ng + 3) / 4 * 4;
  return ((r4 / 4) & 1) ? r4 : r4 + 4;
}

template <int BITS, int MB, bool HALF, int CT, bool RAW>
struct Stream {
  static constexpr uint32_t TB = (BITS == 8) ? 1024u : 512u;  // bytes per k-tile
  static constexpr int NA = HALF ? (CT + 1) / 2 : CT;         // A fragments per chunk
  __amdgpu_buffer_rsrc_t rb, ra;
  uint32_t bvoff;          // lane part of the weight-tile offset
  uint32_t avoff[MB];      // lane part of the A-fragment offset (FGM_OOB if row >= M)
  int h, sh;               // h = j >> 3; int4 nibble shift (4 for j < 8, else 0)
  v4i acc[MB];
  int32_t braw[CT][4];
  v4i af[NA][MB];
  int32_t* pb[MB][4];      // int4: group 0 of row 16 mb + 4 g + r, column j, in the
                           // parked sums ([m][column][group]); null: not parked
  int gk, gpos, gi;        // group length in k-blocks, position in it, group index

  // Loads of cnt (1..CT, wave-uniform) tiles starting at k-block t0, in the
  // order the multiplies consume them (weights and activations of tile u
  // before those of tile u + 1) so that each multiply waits for its own data.
  __device__ __forceinline__ void issue(int t0, int cnt) {
#pragma unroll
    for (int u = 0; u < CT; u++) {
      const uint32_t sb = (uint32_t)(t0 + u) * TB;
      const uint32_t bo = u < cnt ? bvoff : FGM_OOB;
#pragma unroll
      for (int t = 0; t < 4; t++) braw[u][t] = buf_load_b32(rb, bo + t * (BITS == 8 ? 64u : 32u), sb);
      if (HALF) {
        if ((u & 1) == 0)
          af[u >> 1][0] = buf_load_b128(ra, (u + h < cnt) ? avoff[0] : FGM_OOB, (uint32_t)(t0 + u) * 1024u);
      } else {
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
          af[u][mb] = buf_load_b128(ra, u < cnt ? avoff[mb] : FGM_OOB, (uint32_t)(t0 + u) * 1024u);
      }
    }
  }

  // int4: the finished group's sums into LDS
  __device__ __forceinline__ void park(int grp) {
    if (HALF) {
      if (pb[0][0]) {  // lanes of rows 0-7
#pragma unroll
        for (int r = 0; r < 4; r++) pb[0][r][grp] = RAW ? acc[0][r] : __float_as_int((float)acc[0][r]);
      }
    } else {
#pragma unroll
      for (int mb = 0; mb < MB; mb++)
#pragma unroll
        for (int r = 0; r < 4; r++)
          if (pb[mb][r]) pb[mb][r][grp] = RAW ? acc[mb][r] : __float_as_int((float)acc[mb][r]);
    }
  }

  // G1: one k-block per group (group 64), so tile u of a chunk is group gi + u
  template <bool G1>
  __device__ __forceinline__ void compute(int cnt) {
#pragma unroll
    for (int u = 0; u < CT; u++) {
      if (u >= cnt) break;
      v4i bv;
#pragma unroll
      for (int t = 0; t < 4; t++)
        bv[t] = BITS == 8 ? braw[u][t] : (int)(((uint32_t)braw[u][t] << sh) & 0xF0F0F0F0u);
      const bool fresh = BITS == 4 && (G1 || gpos == 0);
      if (HALF) {
        // lanes j >= 8 feed rows 8-15 of the product, which are never read:
        // they keep whatever the other tile of the pair puts there
        const v4i x = af[u >> 1][0];
        v4i av;
#pragma unroll
        for (int q = 0; q < 4; q++) av[q] = (u & 1) ? ror8(x[q]) : x[q];
        acc[0] = fresh ? mfma16(av, bv, v4i{0, 0, 0, 0}) : mfma16(av, bv, acc[0]);
      } else {
#pragma unroll
        for (int mb = 0; mb < MB; mb++)
          acc[mb] = fresh ? mfma16(af[u][mb], bv, v4i{0, 0, 0, 0}) : mfma16(af[u][mb], bv, acc[mb]);
      }
      if (BITS == 4) {
        if (G1) {
          park(gi + u);
        } else if (++gpos == gk) {
          park(gi++);
          gpos = 0;
        }
      }
    }
    if (BITS == 4 && G1) gi += cnt;
  }
};

template <int BITS, int MB, bool HALF, int CT, bool G1, bool RAW>
__global__ __launch_bounds__(1024) void decode_kernel(GemmBatch bt) {
  extern __shared__ __attribute__((aligned(16))) int32_t lds[];
  const GemmProb a = pick(bt);
  const int tid = threadIdx.x;
  const int w = wave_id(), l = tid & 63, g = l >> 4, j = l & 15;
  const int M = a.M, N = a.N, KB = a.K >> 6;
  const int Mp = HALF ? 8 : M;  // rows of the parked sums
  const int KS = a.ks, NBW = a.nbw, TW = a.tw;
  const int gk = (BITS == 4) ? (a.group >> 6) : 1;
  const int NG = (BITS == 4) ? KB / gk : 1;
  const int NGP = group_pitch(NG);
  const int nb_first = a.n0 + (int)(blockIdx.x - a.wg0) * NBW;
  const int nb_here = min(NBW, a.n0 + a.nblocks - nb_first);  // n-blocks in this workgroup
  const int nbi = w / KS, s = w - nbi * KS;                    // wave-uniform
  const bool want_scales = BITS == 4 && !RAW;
  const int psz = Mp * 16 * NGP;                                // parked words per n-block

  // 1. the first chunk of this wave's weight stream
  Stream<BITS, MB, HALF, CT, RAW> st;
  const bool streaming = nbi < nb_here;
  const int tb = s * TW, te = min(KB, tb + TW);
  if (streaming) {
    const int nb = nb_first + nbi;
    st.rb = make_rsrc((const int8_t*)a.B + (size_t)nb * KB * st.TB, (uint32_t)KB * st.TB);
    st.ra = make_rsrc(a.A, (uint32_t)((M + 15) / 16 * KB * 1024));
    st.h = j >> 3;
    st.sh = j < 8 ? 4 : 0;
    st.bvoff = BITS == 8 ? (uint32_t)(256 * g + 4 * j) : (uint32_t)(128 * g + 4 * (j & 7));
    if (HALF) {
      const int r = j & 7;
      st.avoff[0] = r < M ? (uint32_t)(st.h * 1024 + r * 64 + 16 * g) : FGM_OOB;
    } else {
#pragma unroll
      for (int mb = 0; mb < MB; mb++)
        st.avoff[mb] = (mb * 16 + j < M) ? (uint32_t)(mb * KB * 1024 + j * 64 + 16 * g) : FGM_OOB;
    }
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = mb * 16 + 4 * g + r;
        st.pb[mb][r] = m < Mp ? lds + (size_t)nbi * psz + (size_t)(m * 16 + j) * NGP : nullptr;
      }
    st.gk = gk;
    st.gpos = 0;
    st.gi = tb / gk;
#pragma unroll
    for (int mb = 0; mb < MB; mb++) st.acc[mb] = v4i{0, 0, 0, 0};
    st.issue(tb, min(CT, te - tb));
  }

  // 2. group scales of this workgroup's columns, two columns per dword, in
  //    flight behind the weights.  NBW is a power of two; dword i holds group
  //    i >> lg, columns 16 * nb_first + 2 * (i & (8 * NBW - 1)) + {0, 1}.
  const int lg = __builtin_ctz(NBW) + 3;
  const int nsd = NG << lg;  // host: <= SPT * blockDim
  uint32_t sreg[SPT];
  if (want_scales) {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.b_scale, (uint32_t)NG * N * 2);
#pragma unroll
    for (int u = 0; u < SPT; u++) {
      const int i = tid + u * (int)blockDim.x;
      const int gi = i >> lg, c2 = i & ((1 << lg) - 1);
      const bool ok = i < nsd && (c2 >> 3) < nb_here;
      sreg[u] = (uint32_t)buf_load_b32(rs, ok ? (uint32_t)((gi * N + nb_first * 16 + 2 * c2) * 2) : FGM_OOB, 0);
    }
  }

  // per-row activation scales, and (int8) per-column weight scales of this
  // workgroup, for the epilogue
  float rscale = 0.0f, cscale = 0.0f;
  if (!RAW) {
    const __amdgpu_buffer_rsrc_t ras = make_rsrc(a.a_scale, (uint32_t)M * 4);
    rscale = __int_as_float(buf_load_b32(ras, tid < M ? (uint32_t)tid * 4 : FGM_OOB, 0));
    if (BITS == 8) {
      const __amdgpu_buffer_rsrc_t rbs = make_rsrc(a.b_scale, (uint32_t)N * 4);
      const int col = nb_first * 16 + tid;
      cscale = __int_as_float(buf_load_b32(rbs, tid < nb_here * 16 ? (uint32_t)col * 4 : FGM_OOB, 0));
    }
  }

  // 3. the multiplies, then the rest of the stream (waves with more than CT
  //    k-blocks: long K, or groups wider than CT k-blocks)
  if (streaming) {
    st.template compute<G1>(min(CT, te - tb));
    for (int t0 = tb + CT; t0 < te; t0 += CT) {
      st.issue(t0, min(CT, te - t0));
      st.template compute<G1>(min(CT, te - t0));
    }
    if (BITS == 8) {
      int32_t* R = lds + (size_t)w * Mp * 16;
#pragma unroll
      for (int mb = 0; mb < MB; mb++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int m = mb * 16 + 4 * g + r;
          if (m < Mp) R[m * 16 + j] = st.acc[mb][r];
        }
    }
  }

  // int4 scales in LDS as f32 / 16 (exact): [n-block][column][group], pitch NGP
  float* SF = (float*)(lds + (size_t)NBW * psz);
  if (want_scales) {
#pragma unroll
    for (int u = 0; u < SPT; u++) {
      const int i = tid + u * (int)blockDim.x;
      const int gi = i >> lg, c2 = i & ((1 << lg) - 1);
      if (i < nsd && (c2 >> 3) < nb_here) {
        const int q = c2 >> 3, c = 2 * (c2 & 7);
        float* d = SF + ((size_t)q * 16 + c) * NGP + gi;
        d[0] = f16_bits_to_f32((uint16_t)(sreg[u] & 0xFFFF)) * 0.0625f;
        d[NGP] = f16_bits_to_f32((uint16_t)(sreg[u] >> 16)) * 0.0625f;
      }
    }
  }
  // epilogue scales: a_scale [Mp], then (int8) b_scale [NBW * 16]
  float* ASC = BITS == 4 ? SF + (size_t)NBW * 16 * NGP : (float*)(lds + (size_t)(blockDim.x >> 6) * Mp * 16);
  float* BSC = ASC + Mp;
  if (!RAW) {
    if (tid < M) ASC[tid] = rscale;
    if (BITS == 8 && tid < nb_here * 16) BSC[tid] = cscale;
  }
  __syncthreads();

  // 4. epilogue: one thread per output of the workgroup's n-blocks
  const int per_nb = Mp * 16;
  for (int o = tid; o < nb_here * per_nb; o += blockDim.x) {
    const int q = o / per_nb, rem = o - q * per_nb;
    const int m = rem >> 4, c = rem & 15;
    if (m >= M) continue;
    const int ncol = (nb_first + q) * 16 + c;
    if (BITS == 8) {
      int32_t sum = 0;
      for (int ss = 0; ss < KS; ss++) sum += lds[((size_t)(q * KS + ss) * Mp + m) * 16 + c];
      if (RAW) {
        a.acc_out[(size_t)m * a.ldacc + ncol] = sum;
      } else {
        const float sc = BSC[q * 16 + c] * ASC[m];
        a.C[(size_t)m * a.ldc + ncol] = (float)sum * sc;
      }
    } else {
      const int32_t* pr = lds + (size_t)q * psz + (size_t)(m * 16 + c) * NGP;
      if (RAW) {
        for (int gg = 0; gg < NG; gg++) a.acc_out[((size_t)gg * M + m) * a.ldacc + ncol] = pr[gg] >> 4;
      } else {
        // the chain is serial: four groups per 16-byte read of the sums and
        // of the scales, the reads of the next quad issued before the fmas
        const float* pf = (const float*)pr;
        const float* sr = SF + ((size_t)q * 16 + c) * NGP;
        const int nq = NG >> 2;
        float cacc = 0.0f;
        if (nq > 0) {
          float4 pv = *(const float4*)pf, sv = *(const float4*)sr;
          for (int qq = 1; qq < nq; qq++) {
            const float4 pn = *(const float4*)(pf + 4 * qq), sn = *(const float4*)(sr + 4 * qq);
            cacc = __builtin_fmaf(pv.x, sv.x, cacc);
            cacc = __builtin_fmaf(pv.y, sv.y, cacc);
            cacc = __builtin_fmaf(pv.z, sv.z, cacc);
            cacc = __builtin_fmaf(pv.w, sv.w, cacc);
            pv = pn;
            sv = sn;
          }
          cacc = __builtin_fmaf(pv.x, sv.x, cacc);
          cacc = __builtin_fmaf(pv.y, sv.y, cacc);
          cacc = __builtin_fmaf(pv.z, sv.z, cacc);
          cacc = __builtin_fmaf(pv.w, sv.w, cacc);
        }
        for (int gg = 4 * nq; gg < NG; gg++) cacc = __builtin_fmaf(pf[gg], sr[gg], cacc);
        a.C[(size_t)m * a.ldc + ncol] = cacc * ASC[m];
      }
    }
  }
}

// Tiles per chunk: about 4 KB of weights per wave, fewer with more m-blocks
// (each tile then needs MB activation fragments in registers).
#ifndef FGM_CT4
#define FGM_CT4 8
#endif
constexpr int ct_for(int bits, int MB) {
  return bits == 4 ? (MB == 1 ? FGM_CT4 : (MB == 2 ? 4 : 2)) : (MB == 1 ? 4 : (MB == 2 ? 2 : 1));
}

template <int BITS, int MB, bool HALF, bool G1, bool RAW>
hipError_t launch_variant(const GemmBatch& bt, int W, size_t lds, int nwg, hipStream_t st) {
  constexpr int CT = ct_for(BITS, MB);
  auto k = decode_kernel<BITS, MB, HALF, CT, G1, RAW>;
  static hipError_t attr = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL(k, dim3(nwg), dim3(W * 64), lds, st, bt);
  return hipGetLastError();
}

template <int BITS, int MB, bool HALF>
hipError_t launch_decode(const GemmBatch& bt, bool g1, bool raw, int W, size_t lds, int nwg, hipStream_t st) {
  if constexpr (BITS == 8) {
    return raw ? launch_variant<BITS, MB, HALF, false, true>(bt, W, lds, nwg, st)
               : launch_variant<BITS, MB, HALF, false, false>(bt, W, lds, nwg, st);
  }
  if (raw) return g1 ? launch_variant<BITS, MB, HALF, true, true>(bt, W, lds, nwg, st)
                     : launch_variant<BITS, MB, HALF, false, true>(bt, W, lds, nwg, st);
  return g1 ? launch_variant<BITS, MB, HALF, true, false>(bt, W, lds, nwg, st)
            : launch_variant<BITS, MB, HALF, false, false>(bt, W, lds, nwg, st);
}

// K split of one GEMM: TW k-blocks per wave (a multiple of the group's
// k-blocks), KS = ceil(KB / TW) <= MAX_WAVES waves per n-block.
void plan_split(int bits, int M, int K, int group, int* tw, int* ks) {
  const int KB = K / 64, MB = (M + 15) / 16;
  const int gk = bits == 4 ? group / 64 : 1;
  const int ct = ct_for(bits, MB);
  int t = ct >= gk ? (ct / gk) * gk : gk;
  int s = (KB + t - 1) / t;
  if (s > MAX_WAVES) {
    t = (KB + MAX_WAVES - 1) / MAX_WAVES;
    t = (t + gk - 1) / gk * gk;
    s = (KB + t - 1) / t;
  }
  *tw = t;
  *ks = s;
}

size_t lds_need(int bits, int M, int K, int group, int nbw, int W) {
  const int Mp = M <= 8 ? 8 : M;
  const size_t esc = (size_t)Mp + (size_t)nbw * 16;  // epilogue scales
  if (bits == 4) {
    const int NG = (K / 64) / (group / 64);
    return ((size_t)nbw * (Mp + 1) * 16 * group_pitch(NG) + esc) * 4;
  }
  return ((size_t)W * Mp * 16 + esc) * 4;
}

}  // namespace

bool fgm_decode_fits(int bits, int M, int K, int group) {
  if (M < 1 || M > 64) return false;
  if ((size_t)((M + 15) / 16) * K * 16 > 0x7FFFFFFFu) return false;  // buffer offsets
  int tw, ks;
  plan_split(bits, M, K, group, &tw, &ks);
  if (bits == 4) {
    const int NG = (K / 64) / (group / 64);
    if (NG * 8 > SPT * 64 * ks) return false;  // scale prefetch of one n-block
  }
  return lds_need(bits, M, K, group, 1, ks) <= 160 * 1024;
}

size_t fgm_decode_lds_bytes(int bits, int M, int K, int group) {
  int tw, ks;
  plan_split(bits, M, K, group, &tw, &ks);
  return lds_need(bits, M, K, group, 1, ks);
}

// Every problem of the batch gets the same workgroup size W = the largest
// K split; a problem with a smaller split packs W / KS n-blocks into each
// workgroup, as far as LDS and the scale prefetch allow.
hipError_t fgm_launch_decode(int bits, const GemmBatch& in, hipStream_t st) {
  // one kernel variant per launch: split a batch that mixes raw-accumulator
  // and scaled problems, or (int4) group 64 with wider groups
  for (int i = 1; i < in.count; i++) {
    const GemmProb &p = in.p[i], &q = in.p[0];
    if ((p.acc_out != nullptr) != (q.acc_out != nullptr) ||
        (bits == 4 && (p.group == 64) != (q.group == 64))) {
      GemmBatch a{}, b{};
      for (int k = 0; k < in.count; k++) {
        const GemmProb& r = in.p[k];
        const bool same = (r.acc_out != nullptr) == (q.acc_out != nullptr) &&
                          (bits != 4 || (r.group == 64) == (q.group == 64));
        GemmBatch& d = same ? a : b;
        d.p[d.count++] = r;
      }
      hipError_t e = fgm_launch_decode(bits, a, st);
      return e != hipSuccess ? e : fgm_launch_decode(bits, b, st);
    }
  }
  // problems with the longest K first: their workgroups are dispatched
  // first, and their epilogue chains are the longest
  GemmBatch bt = in;
  for (int i = 1; i < bt.count; i++)
    for (int k = i; k > 0 && bt.p[k].K > bt.p[k - 1].K; k--) {
      const GemmProb t = bt.p[k];
      bt.p[k] = bt.p[k - 1];
      bt.p[k - 1] = t;
    }
  int W = 1, MB = 0, Mmax = 0;
  for (int i = 0; i < bt.count; i++) {
    GemmProb& p = bt.p[i];
    plan_split(bits, p.M, p.K, p.group, &p.tw, &p.ks);
    if (p.ks > W) W = p.ks;
    const int mb = (p.M + 15) / 16;
    if (mb > MB) MB = mb;
    if (p.M > Mmax) Mmax = p.M;
  }
  int nwg = 0;
  size_t lds = 0;
  for (int i = 0; i < bt.count; i++) {
    GemmProb& p = bt.p[i];
    // a power of two (the kernel maps scale dwords with shifts)
    int nbw = 1;
    while (nbw * 2 * p.ks <= W && nbw * 2 <= p.nblocks) nbw *= 2;
    while (nbw > 1 && lds_need(bits, p.M, p.K, p.group, nbw, W) > 160 * 1024) nbw /= 2;
    if (bits == 4) {
      const int NG = (p.K / 64) / (p.group / 64);
      while (nbw > 1 && nbw * NG * 8 > SPT * 64 * W) nbw /= 2;
    }
    p.nbw = nbw;
    p.wg0 = nwg;
    nwg += (p.nblocks + nbw - 1) / nbw;
    const size_t need = lds_need(bits, p.M, p.K, p.group, nbw, W);
    if (need > lds) lds = need;
  }
  if (nwg == 0) return hipSuccess;
  const bool half = MB == 1 && Mmax <= 8;
  const bool g1 = bits == 4 && bt.p[0].group == 64;
  const bool raw = bt.p[0].acc_out != nullptr;
  if (bits == 8) {
    if (half) return launch_decode<8, 1, true>(bt, g1, raw, W, lds, nwg, st);
    switch (MB) {
      case 1: return launch_decode<8, 1, false>(bt, g1, raw, W, lds, nwg, st);
      case 2: return launch_decode<8, 2, false>(bt, g1, raw, W, lds, nwg, st);
      case 3: return launch_decode<8, 3, false>(bt, g1, raw, W, lds, nwg, st);
      case 4: return launch_decode<8, 4, false>(bt, g1, raw, W, lds, nwg, st);
    }
  } else {
    if (half) return launch_decode<4, 1, true>(bt, g1, raw, W, lds, nwg, st);
    switch (MB) {
      case 1: return launch_decode<4, 1, false>(bt, g1, raw, W, lds, nwg, st);
      case 2: return launch_decode<4, 2, false>(bt, g1, raw, W, lds, nwg, st);
      case 3: return launch_decode<4, 3, false>(bt, g1, raw, W, lds, nwg, st);
      case 4: return launch_decode<4, 4, false>(bt, g1, raw, W, lds, nwg, st);
    }
  }
  return hipErrorInvalidValue;
}
