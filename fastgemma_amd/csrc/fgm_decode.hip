// Decode / skinny GEMM (M <= 64) on gfx950: a weight stream.
//
// Replaces fgm_gemm_q8c_vnni / fgm_gemm_q4g_vnni (vnni_gemm.c:224-245,
// 291-322) for the row counts where the GEMM is bound by reading B.  One
// launch serves up to FGM_MAX_BATCH independent GEMMs of the same weight type
// (the reference issues q/k/v and gate/up as separate GEMMs on one
// activation, forward.rs:484,499-500,619-622).
//
// Work decomposition (plan_split / fgm_launch_decode below): a workgroup owns
// NBW 16-column n-blocks of one GEMM and has NWS >= NBW * KS waves (those past
// NBW * KS only take part in the barriers).  Each n-block's K is cut into 1 KB
// units (two int4
// k-tiles or one int8 k-tile) that its KS stream waves share round-robin:
// unit u * KS + s belongs to wave s, so round u (one unit per wave) covers
// TR = KS * (tiles per unit) consecutive k-tiles.
//
// Weight stream: each unit is one buffer_load_dwordx4 ... lds per wave (1 KB,
// 16 contiguous bytes per lane, non-temporal) into a per-wave LDS ring of D
// slots, up to D - 1 units in flight.  The lane loads a permuted 16-byte chunk
// so that the fragment reads below are free of bank conflicts:
//   int4 unit (two 512-byte tiles, 16-byte chunk c = 32 tile + 2 row + half):
//     LDS chunk p holds HBM chunk p ^ (((p >> 3) & 3) << 1);
//   int8 unit (one 1 KB tile, chunk c = 4 row + quarter):
//     LDS chunk p holds HBM chunk p ^ (((p >> 4) & 3) << 2).
// Activation fragments are plain 16-byte buffer loads (L2-resident), issued
// with the unit they belong to: X vector-memory instructions per unit.  Units
// are issued in order and never past a wave's last unit; the epilogue scales
// (PRE loads) follow the first units.  So s_waitcnt vmcnt(X * units issued
// after it + PRE if those came later) waits for exactly the unit that is
// about to be multiplied.
//
// MFMA operand mapping (v_mfma_i32_16x16x64_i8, lane l = 16*g + j): A row j /
// B column j, operand byte 4*t + e carries k = 16*g + 4*t + e, i.e. k-tile row
// r = 4*g + t of the [k/4][n][k%4] layout.
//   int8 B: dword j of row r.
//   int4 B: packed row r holds column c (c < 8) in the low and column c + 8
//     in the high nibbles of its dword c (lanes j and j + 8 read the same
//     dword, an LDS broadcast).  The lane keeps its nibble in the high half of
//     each byte: (x << 4) & 0xF0F0F0F0 for j < 8, x & 0xF0F0F0F0 for j >= 8.
//     A two's-complement nibble v in bits 7..4 of a byte is the int8 16 * v,
//     so the MFMA accumulates exactly 16 * acc.
//   A: one 16-byte load of the packed-A row per fragment.  M <= 8 (HALF):
//     lanes j < 8 load row j of the unit's first tile and lanes j >= 8 row
//     j - 8 of its second; the second tile's operand is moved into lanes 0-7
//     by a DPP rotation by 8 lanes.  Rows 8-15 of those products are unused.
//     M > 8: one fragment per tile and 16-row m-block.
//   Output: lane l, register r holds D[4*g + r][j].
//
// Epilogues, in the reference's operation order:
//   q8c: each stream wave accumulates int32 over its units; the KS partial
//        sums of an n-block are added exactly in LDS, then
//        C = (float)acc * (b_scale[n] * a_scale[m])          vnni_gemm.c:206-219
//   q4g: the stream waves park every k-tile's sums (int32, 16 * acc) in LDS;
//        after the stream one thread per output runs its chain in ascending
//        k: the tile sums of a scale group are added exactly, and at the
//        group's end
//        C = fmaf((float)acc_g, f16(b_scale[g][n]), C)          vnni_gemm.c:258-285
//        (the scale is kept as f32(b_scale) / 16: (16 a) * (s / 16) is the
//        exact product a * s, so every fmaf rounds the reference's value);
//        at the end C *= a_scale[m]                            vnni_gemm.c:316-321
#include "fgm_common.h"
#include "fgm_kernels.h"

namespace {

constexpr int MAX_WAVES = 16;
constexpr int DPP_ROW_ROR8 = 0x128;
constexpr int SPT = 4;            // int4 group-scale dwords prefetched per thread
constexpr int CHP = 4;            // group-64 chain: pairs of 4-k-tile chunks in flight
#ifndef FGM_DEC_UPW
#define FGM_DEC_UPW 4             // target units (1 KB) per stream wave
#endif
#ifndef FGM_DEC_NWMIN
#define FGM_DEC_NWMIN 4           // smallest number of stream waves per workgroup
#endif
#ifndef FGM_DEC_PIR_MIN_WGS
#define FGM_DEC_PIR_MIN_WGS 2048  // workgroups above which int4 sums are parked in the ring
#endif
#ifndef FGM_DEC_PIR_NPW
#define FGM_DEC_PIR_NPW 2         // n-blocks per wave of the decode_pir2_kernel grids (2 or 4)
#endif
#ifndef FGM_DEC_PIR2_MIN_WGS
#define FGM_DEC_PIR2_MIN_WGS 2048 // above which, where the shapes allow, two n-blocks share a wave
#endif

// Two 16-byte LDS reads by byte address, and waits for all but the last six
// LDS operations (or for all of them) that also order the use of the given
// registers after the wait.  LDS operations complete in issue order.
template <int OFF>
FGM_DEV void lds_read2x128(v4i& r0, v4i& r1, uint32_t a0, uint32_t a1) {
  asm volatile("ds_read_b128 %0, %2 offset:%4\n\tds_read_b128 %1, %3 offset:%4"
               : "=&v"(r0), "=&v"(r1)
               : "v"(a0), "v"(a1), "n"(OFF)
               : "memory");
}
typedef int v2i __attribute__((ext_vector_type(2)));
// One group of the parked-in-ring chain: four parked pairs 1 KB apart and
// their eight scales, six LDS reads; waits for all but the last group read.
FGM_DEV void pir_read(v2i (&p)[4], v4i (&sc)[2], uint32_t pa, uint32_t sa) {
  asm volatile(
      "ds_read_b64 %0, %6\n\tds_read_b64 %1, %6 offset:1024\n\t"
      "ds_read_b64 %2, %6 offset:2048\n\tds_read_b64 %3, %6 offset:3072\n\t"
      "ds_read_b128 %4, %7\n\tds_read_b128 %5, %7 offset:16"
      : "=&v"(p[0]), "=&v"(p[1]), "=&v"(p[2]), "=&v"(p[3]), "=&v"(sc[0]), "=&v"(sc[1])
      : "v"(pa), "v"(sa)
      : "memory");
}
FGM_DEV void pir_wait6(v2i (&p)[4], v4i (&sc)[2]) {
  asm volatile("s_waitcnt lgkmcnt(6)" : "+v"(p[0]), "+v"(p[1]), "+v"(p[2]), "+v"(p[3]), "+v"(sc[0]), "+v"(sc[1]) : : "memory");
}
FGM_DEV void pir_wait0(v2i (&p)[4], v4i (&sc)[2]) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(p[0]), "+v"(p[1]), "+v"(p[2]), "+v"(p[3]), "+v"(sc[0]), "+v"(sc[1]) : : "memory");
}
// Three 16-byte LDS reads (two at a0, a0 + 16 plus OA; one at a1 plus OB),
// and a wait for all but the last N LDS operations that also orders the use
// of the given registers after it.
template <int OA, int OB>
FGM_DEV void lds_read3x128(v4i& r0, v4i& r1, v4i& r2, uint32_t a0, uint32_t a1) {
  asm volatile("ds_read_b128 %0, %3 offset:%5\n\tds_read_b128 %1, %3 offset:%6\n\tds_read_b128 %2, %4 offset:%7"
               : "=&v"(r0), "=&v"(r1), "=&v"(r2)
               : "v"(a0), "v"(a1), "n"(OA), "n"(OA + 16), "n"(OB)
               : "memory");
}
template <int N>
FGM_DEV void lgkm_wait3(v4i& r0, v4i& r1, v4i& r2) {
  asm volatile("s_waitcnt lgkmcnt(%3)" : "+v"(r0), "+v"(r1), "+v"(r2) : "n"(N) : "memory");
}
// The f16 in the low / high half of a dword, widened (exactly) to f32.
FGM_DEV float f16lo(int x) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(x & 0xFFFF)); }
FGM_DEV float f16hi(int x) { return (float)__builtin_bit_cast(_Float16, (uint16_t)((uint32_t)x >> 16)); }
template <int N>
FGM_DEV void lgkm_wait(v4i& r0, v4i& r1) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(r0), "+v"(r1) : "n"(N) : "memory");
}
FGM_DEV void lgkm_wait6(v4i& r0, v4i& r1) {
  asm volatile("s_waitcnt lgkmcnt(6)" : "+v"(r0), "+v"(r1) : : "memory");
}
FGM_DEV void lgkm_wait0(v4i& r0, v4i& r1) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r0), "+v"(r1) : : "memory");
}

// the value of lane l ^ 8 (a rotation by 8 within every 16-lane row)
FGM_DEV int ror8(int v) { return __builtin_amdgcn_mov_dpp(v, DPP_ROW_ROR8, 0xF, 0xF, false); }

// Pitch (words) of a row of parked tile sums or group scales: a multiple of
// four with an odd number of quads, so that 16-byte reads by consecutive rows
// hit distinct banks.
__host__ __device__ inline int pitch4(int n) {
  const int r4 = (n + 3) / 4 * 4;
  return ((r4 / 4) & 1) ? r4 : r4 + 4;
}

// Ring slots per stream wave.  M <= 8: fewer units in flight per wave suit
// the grids of one round of workgroups (measured with 2-5 slots, ~4 units per
// wave: the cfg2 pair 7.9 -> 7.7 us with 4 slots, the int8 M = 1 GEMV 5.45 ->
// 5.26 us with 3); the park in the ring needs a slot for every unit of a
// wave, so it keeps 5.
__host__ __device__ constexpr int ring_depth(int bits, int MB, bool half, bool pir = false) {
  return half ? (pir ? 5 : (bits == 8 ? 3 : 4))
              : (bits == 8 ? 4 : (MB == 1 ? 4 : (MB == 2 ? 3 : 2)));
}

// Shape constants of a kernel variant.
template <int BITS, int MB, bool HALF, bool PIR = false>
struct Geo {
  static constexpr int TPU = BITS == 4 ? 2 : 1;       // k-tiles per 1 KB unit
  static constexpr int OUT = HALF ? 128 : 256 * MB;   // outputs per n-block
  static constexpr int NA = HALF ? 1 : MB * TPU;      // activation loads per unit
  static constexpr int X = 1 + NA;                    // vector-memory instructions per unit
  static constexpr int D = ring_depth(BITS, MB, HALF, PIR);
};

// LDS layout of one workgroup (bytes), shared by the host (sizing) and the
// kernel: the weight rings (also the q8c reduction area afterwards), then
// (int4) the parked tile sums of every k-tile ([n-block][output][k-tile],
// pitch pp) and the group scales ([n-block][column][group], pitch ngp, zero
// past the last group); then the epilogue scales.  With the park in the ring
// (pir) the tile sums go back into the slot their weights came from and the
// park area is empty.
struct Lay {
  uint32_t ring, park, scl, asc, bsc, total;
  int slots, pp, ngp, ngh;
  __host__ __device__ Lay(int bits, int out, int d, int ks, int upw, int nws, int nbw, int kb, int mp,
                          bool pir = false) {
    const int tpu = bits == 4 ? 2 : 1;
    slots = upw < d ? upw : d;
    ring = 0;
    uint32_t o = (uint32_t)nws * slots * 1024;
    // int4: parked k-tiles (K rounded up to whole rounds and to pairs of
    // 4-tile chunks) and f32 scales padded to whole 4-tile chunks; group 64
    // keeps its scales as f16 (ngh halves per row: whole 16-byte units, an
    // odd number of them, so 16-byte reads by consecutive rows hit distinct
    // banks) in the same area
    pp = pitch4((tpu * ks * upw + 7) / 8 * 8);
    ngp = pitch4((kb + 3) / 4 * 4);
    ngh = (kb + 7) / 8 * 8;
    if (((ngh / 8) & 1) == 0) ngh += 8;
    park = o;
    o += (bits == 4 && !pir) ? (uint32_t)nbw * out * pp * 4 : 0;
    scl = o;
    o += bits == 4 ? (uint32_t)nbw * 16 * (ngp * 4 > ngh * 2 ? ngp * 4 : ngh * 2) : 0;
    asc = o;
    o += (uint32_t)(mp + 3) / 4 * 16;
    bsc = o;
    o += (uint32_t)nbw * 64;
    // pir: the chain's last group of pair reads may run up to 3 KB past the
    // ring (and its scale reads 32 bytes past the scale rows); the areas
    // after the ring absorb most of it, pad the rest so the reads stay inside
    // the workgroup's LDS
    if (pir) {
      const uint32_t ring_end = (uint32_t)nws * slots * 1024, need = ring_end + 3072 + 32;
      if (o < need) o = need;
    }
    // the group-64 chain reads up to 2 CHP - 2 pairs (32 bytes of sums, 16 of
    // scales) past a row
    if (bits == 4) o += 32 * (2 * CHP - 2);
    total = o;
  }
};

// PIR: the tile sums are parked in the ring slot their weights came from
// (int4, M <= 8, group 64, every slot filled once: UPW <= D).
template <int BITS, int MB, bool HALF, bool G1, bool RAW, bool PIR = false>
__global__ __launch_bounds__(1024) void decode_kernel(GemmBatch bt) {
  using G = Geo<BITS, MB, HALF, PIR>;
  static_assert(!PIR || (BITS == 4 && HALF && G1 && !RAW), "park in ring: int4, M <= 8, group 64");
  constexpr int TPU = G::TPU, OUT = G::OUT, NA = G::NA, X = G::X, D = G::D;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const GemmProb a = pick_problem(bt);
  fetch_all(a);
  if ((int)blockIdx.x >= a.nwg) return;  // past this problem's workgroups
  const int tid = threadIdx.x, NT = blockDim.x;
  const int w = wave_id(), l = tid & 63, g = l >> 4, j = l & 15;
  const int M = a.M, N = a.N, KB = a.K >> 6;
  const int KS = a.ks, NBW = a.nbw, UPW = a.tw;
  const int NWS = NT >> 6, NWP = KS * NBW;         // waves, waves with an n-block
  const int TR = TPU * KS;                         // k-tiles per round
  const int gk = BITS == 4 ? a.group >> 6 : 1;
  const int NG = BITS == 4 ? KB / gk : 0;
  const int Mp = HALF ? 8 : 16 * MB;
  // Workgroups go round-robin over the 8 XCDs: for int4, give each XCD a
  // contiguous run of n-blocks, so that the workgroups sharing a 128-byte
  // line of group scales (four n-blocks) share an L2 and fetch it from HBM
  // once.  (int8 scales are one float per column, nothing is shared, and
  // the interleaved order measured faster: cfg1 5.45 against 6.3 us.)  The
  // grid's width is a multiple of 8, so workgroup x of every problem runs on
  // XCD x % 8.
  int lb = (int)blockIdx.x;
  const int nwgp = a.nwg;
  if (BITS == 4 && (nwgp & 7) == 0) lb = (lb & 7) * (nwgp >> 3) + (lb >> 3);
  const int nb_first = a.n0 + lb * NBW;
  const int nb_here = min(NBW, a.n0 + a.nblocks - nb_first);
  const Lay L(BITS, OUT, D, KS, UPW, NWS, NBW, KB, Mp, PIR);
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
  constexpr uint32_t TB = BITS == 4 ? 512u : 1024u;  // bytes per k-tile

  // ---- the stream: this wave's weights (an empty range if it has no
  // n-block), packed A
  // KS and NBW are powers of two (the launcher's split): shifts, not divisions
  const int lks = __builtin_ctz(KS), lnbw = __builtin_ctz(NBW);
  const int q = w >> lks, s = w & (KS - 1);        // wave's n-block, K slice
  const bool live = w < NWP && q < nb_here;
  const int UPWw = w < NWP ? UPW : 0;              // units this wave streams
  const v4i rb = rsrc_words((const int8_t*)a.B + (size_t)(nb_first + (live ? q : 0)) * KB * TB,
                            live ? (uint32_t)KB * TB : 0u);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(a.A, (uint32_t)((M + 15) / 16) * KB * 1024);
  const uint32_t bsw = BITS == 4 ? 16u * (uint32_t)(l ^ (((l >> 3) & 3) << 1))
                                 : 16u * (uint32_t)(l ^ (((l >> 4) & 3) << 2));
  uint32_t avoff[NA];
  if (HALF) {
    const int r = j & 7;
    const bool ok = r < M && (BITS == 4 || j < 8);
    avoff[0] = ok ? (uint32_t)((j >> 3) * 1024 + r * 64 + 16 * g) : FGM_OOB;
  } else {
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
      for (int e = 0; e < TPU; e++)
        avoff[mb * TPU + e] = (16 * mb + j < M) ? (uint32_t)(mb * KB * 1024 + e * 1024 + j * 64 + 16 * g)
                                                : FGM_OOB;
  }
  const uint32_t ring_w = lds0 + L.ring + (uint32_t)w * L.slots * 1024;

  // one DMA of 1 KB of weights into ring slot sl, and the activation
  // fragments of the same k-tiles into af[sl]
  v4i af[D][NA];
  auto issue = [&](int u, auto slc) __attribute__((always_inline)) {
    constexpr int sl = decltype(slc)::value;
    // unit index in the n-block: round robin over the KS waves, or (PIR)
    // a contiguous run per wave, so that the parked pairs lie in k order
    const uint32_t gu = PIR ? (uint32_t)(s * UPW + u) : (uint32_t)(u * KS + s);
    dma16<true>(rb, ring_w + sl * 1024, bsw, gu * 1024u);
#pragma unroll
    for (int x = 0; x < NA; x++) af[sl][x] = buf_load_b128(ra, avoff[x], gu * TPU * 1024u);
  };
  // units 0 .. D - 2 in flight
  sfor<0, D - 1>([&](auto ic) {
    if (decltype(ic)::value < UPWw) issue(decltype(ic)::value, ic);
  });

  // ---- PRE: epilogue scales, after the first units (the stream starts
  // first); they are only read after the stream
  constexpr int PRE = (BITS == 4 && !RAW ? SPT : 0) + (RAW ? 0 : (BITS == 8 ? 2 : 1));
  uint32_t sreg[SPT];
  float rscale = 0.0f, cscale = 0.0f;
  if (BITS == 4 && !RAW) {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.b_scale, (uint32_t)NG * N * 2);
    const int per_g = 8 * NBW;  // dwords per group (two columns each)
#pragma unroll
    for (int v = 0; v < SPT; v++) {
      const int i = tid + v * NT, gi = i >> (3 + lnbw), c2 = i - gi * per_g, qq = c2 >> 3;
      const bool ok = gi < NG && qq < nb_here;
      sreg[v] = (uint32_t)buf_load_b32(rs, ok ? (uint32_t)((gi * N + (nb_first + qq) * 16 + 2 * (c2 & 7)) * 2) : FGM_OOB, 0);
    }
  }
  if (!RAW) {
    const __amdgpu_buffer_rsrc_t ras = make_rsrc(a.a_scale, (uint32_t)M * 4);
    rscale = __int_as_float(buf_load_b32(ras, tid < M ? (uint32_t)tid * 4 : FGM_OOB, 0));
    if (BITS == 8) {
      const __amdgpu_buffer_rsrc_t rbs = make_rsrc(a.b_scale, (uint32_t)N * 4);
      cscale = __int_as_float(
          buf_load_b32(rbs, tid < nb_here * 16 ? (uint32_t)(nb_first * 16 + tid) * 4 : FGM_OOB, 0));
    }
  }

  // per-lane B fragment offsets within a unit (tile e adds 512 for int4)
  uint32_t boff[4];
#pragma unroll
  for (int t = 0; t < 4; t++) {
    const int c = BITS == 4 ? ((8 * g + 2 * t + ((j & 7) >> 2)) ^ (g << 1))
                            : ((16 * g + 4 * t + (j >> 2)) ^ (g << 2));
    boff[t] = 16u * (uint32_t)c + 4u * (uint32_t)(j & 3);
  }
  const int sh = j < 8 ? 4 : 0;
  v4i acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; mb++) acc[mb] = v4i{0, 0, 0, 0};
  const int npro = min(D - 1, UPWw);             // units issued before PRE
  // group 64: the chain reads the parked sums eight k-tiles at a time, up to
  // k-tile 8 ceil(KB / 8); the stream parks TR * UPW of them (zeros past K).
  // When that is fewer (K of one or two k-tiles per round), the rest is set to
  // zero here -- LDS left by an earlier workgroup may hold any bits, a NaN
  // among them, and 0 * NaN would reach the output.  The barrier before the
  // chain orders these writes.
  if (BITS == 4 && G1 && !RAW && !PIR) {
    const int lo = TR * UPW, hi = ((KB + 7) >> 3) * 8;
    if (hi > lo) {
      float* Pz = (float*)(smem + L.park);
      for (int i = tid; i < NBW * OUT * (hi - lo); i += NT) {
        const int o = i / (hi - lo);
        Pz[o * L.pp + lo + (i - o * (hi - lo))] = 0.0f;
      }
    }
  }

  for (int u0 = 0; u0 < UPWw; u0 += D) {
    sfor<0, D>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      const int u = u0 + i;
      if (u < UPWw) {
        // unit u landed: min(D - 2, UPW - 1 - u) later units, and PRE if
        // it was issued after unit u, may still be in flight
        const int later = min(D - 2, UPWw - 1 - u);
        if (u < npro) {
          sfor<0, D - 1>([&](auto kc) {
            constexpr int k = decltype(kc)::value;
            if (later == k) wait_vm<k * X + PRE>();
          });
        } else {
          sfor<0, D - 1>([&](auto kc) {
            constexpr int k = decltype(kc)::value;
            if (later == k) wait_vm<k * X>();
          });
        }
        // B fragments of unit u
        const char* slot = smem + L.ring + ((size_t)w * L.slots + i) * 1024;
        v4i bv[TPU];
#pragma unroll
        for (int e = 0; e < TPU; e++)
#pragma unroll
          for (int t = 0; t < 4; t++) {
            const uint32_t x = *(const uint32_t*)(slot + e * 512 + boff[t]);
            bv[e][t] = BITS == 8 ? (int)x : (int)((x << sh) & 0xF0F0F0F0u);
          }
        // refill the slot consumed one step ago
        if (u + D - 1 < UPWw) issue(u + D - 1, std::integral_constant<int, (i + D - 1) % D>{});
        if (BITS == 8) {
#pragma unroll
          for (int mb = 0; mb < MB; mb++) acc[mb] = mfma16(af[i][HALF ? 0 : mb], bv[0], acc[mb]);
        } else {
          v4i ts[TPU][MB];  // tile sums (16 * acc)
          if (HALF) {
            const v4i x = af[i][0];
            v4i x1;
#pragma unroll
            for (int d = 0; d < 4; d++) x1[d] = ror8(x[d]);
            ts[0][0] = mfma16(x, bv[0], v4i{0, 0, 0, 0});
            ts[1][0] = mfma16(x1, bv[1], v4i{0, 0, 0, 0});
          } else {
#pragma unroll
            for (int mb = 0; mb < MB; mb++)
#pragma unroll
              for (int e = 0; e < TPU; e++) ts[e][mb] = mfma16(af[i][mb * TPU + e], bv[e], v4i{0, 0, 0, 0});
          }
          // park [n-block][output][k-tile], k-tile TR u + 2 s + e; PIR: the
          // slot just read holds [output][e] (its B fragments are in
          // registers, and no DMA refills it)
          int32_t* P = (int32_t*)(smem + L.park) + (q * OUT) * L.pp + TR * u + 2 * s;
          float* Pr = (float*)(smem + L.ring + ((size_t)w * L.slots + i) * 1024);
          if (!HALF || g < 2) {
#pragma unroll
            for (int mb = 0; mb < MB; mb++)
#pragma unroll
              for (int r = 0; r < 4; r++) {
                const int oo = (16 * mb + 4 * g + r) * 16 + j;
                // group 64: the sum is a whole group's, parked as the float
                // the chain multiplies (exact: |16 acc| < 2^24)
                if (PIR)
                  *(float2*)(Pr + 2 * oo) = float2{(float)ts[0][mb][r], (float)ts[1][mb][r]};
                else if (G1 && !RAW)
                  *(float2*)(P + oo * L.pp) = float2{(float)ts[0][mb][r], (float)ts[1][mb][r]};
                else
                  *(int2*)(P + oo * L.pp) = int2{ts[0][mb][r], ts[1][mb][r]};
              }
          }
        }
      }
    });
  }
  wait_vm<0>();  // the stream and PRE landed; no DMA still writes the ring

  float* ASC = (float*)(smem + L.asc);
  if (!RAW && tid < M) ASC[tid] = rscale;

  if (BITS == 4) {
    // ---- q4g: group scales into LDS, zero past the last group (padded
    // k-tiles add +0): group 64 as the f16 bits (the chain's mixed fma takes
    // them as they are), other group sizes as f32 / 16; then one thread per
    // output runs its chain
    float* S = (float*)(smem + L.scl);
    if (!RAW) {
      const int per_g = 8 * NBW;
#pragma unroll
      for (int v = 0; v < SPT; v++) {
        const int ii = tid + v * NT, gi = ii >> (3 + lnbw), c2 = ii - gi * per_g, qq = c2 >> 3;
        const bool ok = gi < NG && qq < nb_here;
        if (G1 && !PIR) {
          if (gi < ((KB + 7) >> 3) * 8 && qq < NBW) {
            uint16_t* d = (uint16_t*)S + (qq * 16 + 2 * (c2 & 7)) * L.ngh + gi;
            d[0] = ok ? (uint16_t)(sreg[v] & 0xFFFF) : (uint16_t)0;
            d[L.ngh] = ok ? (uint16_t)(sreg[v] >> 16) : (uint16_t)0;
          }
        } else if (gi < L.ngp && qq < NBW) {
          float* d = S + (qq * 16 + 2 * (c2 & 7)) * L.ngp + gi;
          d[0] = ok ? f16_bits_to_f32((uint16_t)(sreg[v] & 0xFFFF)) * 0.0625f : 0.0f;
          d[L.ngp] = ok ? f16_bits_to_f32((uint16_t)(sreg[v] >> 16)) * 0.0625f : 0.0f;
        }
      }
    }
    __syncthreads();
    for (int o = tid; o < NBW * OUT; o += NT) {
      const int qq = o / OUT, oo = o - qq * OUT, m = oo >> 4, c = oo & 15;
      if (qq >= nb_here || m >= M) continue;
      const int32_t* P = (const int32_t*)(smem + L.park) + (qq * OUT + oo) * L.pp;
      const float* Sc = S + (qq * 16 + c) * L.ngp;
      const int n = (nb_first + qq) * 16 + c;
      if constexpr (PIR) {
        // group = k-tile, parked in the ring: wave qq KS + s parked units
        // s UPW .. s UPW + UPW - 1 in its slots, so pair p (k-tiles 2p,
        // 2p + 1, 8 bytes per output) lies at 1 KB x p; its scales are floats
        // 2p, 2p + 1 of the column's row.  Groups of four pairs, read one
        // group ahead (inline asm, waited for with lgkmcnt).  Every read and
        // wait is unconditional -- the prefetch after the last group re-reads
        // the last group, the pairs past the last one are skipped -- so no
        // register of a read still in flight reaches a branch's join, where
        // the compiler could copy it before it lands.
        const int np = (KB + 1) >> 1, ng = (np + 3) >> 2, nfg = np >> 2;
        const uint32_t pb = lds0 + L.ring + (uint32_t)(qq * KS * L.slots) * 1024u + (uint32_t)oo * 8u;
        const uint32_t sb = lds0 + L.scl + (uint32_t)((qq * 16 + c) * L.ngp) * 4u;
        float cacc = 0.0f;
        v2i pv[2][4];
        v4i sv[2][2];
        pir_read(pv[0], sv[0], pb, sb);
        // group gg from slot h (gg % 2), the next group into the other slot
        auto fold = [&](int gg, auto hc, auto partial) {
          constexpr int h = decltype(hc)::value;
          const int gn = gg + 1 < ng ? gg + 1 : ng - 1;
          pir_read(pv[h ^ 1], sv[h ^ 1], pb + 4096u * gn, sb + 32u * gn);
          pir_wait6(pv[h], sv[h]);
#pragma unroll
          for (int b = 0; b < 4; b++)
            if (!decltype(partial)::value || 4 * gg + b < np) {
              const int sx = sv[h][b >> 1][2 * (b & 1)], sy = sv[h][b >> 1][2 * (b & 1) + 1];
              cacc = __builtin_fmaf(__int_as_float(pv[h][b].x), __int_as_float(sx), cacc);
              cacc = __builtin_fmaf(__int_as_float(pv[h][b].y), __int_as_float(sy), cacc);
            }
        };
        int gg = 0;
        for (; gg + 2 <= nfg; gg += 2) {
          fold(gg, std::integral_constant<int, 0>{}, std::false_type{});
          fold(gg + 1, std::integral_constant<int, 1>{}, std::false_type{});
        }
        // the (at most two) groups left, either of them partial or past the end
        fold(gg, std::integral_constant<int, 0>{}, std::true_type{});
        fold(gg + 1, std::integral_constant<int, 1>{}, std::true_type{});
        pir_wait0(pv[0], sv[0]);
        pir_wait0(pv[1], sv[1]);
        a.C[(size_t)m * a.ldc + n] = cacc * ASC[m];
      } else if (G1 && !RAW) {
        // group = k-tile: pairs of 4-k-tile chunks, the sums of a pair in
        // two 16-byte reads and its eight f16 scales in one (rows of the
        // parked sums and of the scales are 16-byte aligned), CHP - 1 pairs
        // read ahead of the pair being folded.  v_fma_mix_f32 takes the f16
        // scale as it is (an exact widening, one rounding), so the chain runs
        // on 16 acc and the unscaled s: every partial value is exactly 16
        // times the reference's (never subnormal: nonzero sums of integer x f16
        // products are at least 2^-24), and the 16 comes off exactly at the
        // end.  LDS reads by address (inline asm, waited for with lgkmcnt):
        // the compiler would otherwise sink the prefetch next to its use.
        // Reads up to 2 CHP - 2 pairs past a row stay inside the workgroup's
        // LDS (the layout's tail pad) and are not used.
        const uint32_t pa0 = lds0 + L.park + (uint32_t)((qq * OUT + oo) * L.pp) * 4u;
        const uint32_t sa0 = lds0 + L.scl + (uint32_t)((qq * 16 + c) * L.ngh) * 2u;
        const int npr = (KB + 7) >> 3;           // k-tiles past K hold zeros (parked or set above)
        float cacc = 0.0f;
        v4i p0[CHP], p1[CHP], sv[CHP];
        sfor<0, CHP - 1>([&](auto bc) {
          constexpr int b = decltype(bc)::value;
          lds_read3x128<32 * b, 16 * b>(p0[b], p1[b], sv[b], pa0, sa0);
        });
        // whole blocks of CHP pairs, then the last, partial block with a
        // per-pair test (outside the blocks the test would put a select on
        // the fma chain's dependence path)
        auto block = [&](int pr, auto partial) {
          const uint32_t pb = pa0 + 32u * pr, sb = sa0 + 16u * pr;
          sfor<0, CHP>([&](auto bc) {
            constexpr int b = decltype(bc)::value, nb = (b + CHP - 1) % CHP;
            lds_read3x128<32 * (b + CHP - 1), 16 * (b + CHP - 1)>(p0[nb], p1[nb], sv[nb], pb, sb);
            lgkm_wait3<3 * (CHP - 1)>(p0[b], p1[b], sv[b]);
            if (!decltype(partial)::value || pr + b < npr) {
              cacc = __builtin_fmaf(__int_as_float(p0[b].x), f16lo(sv[b].x), cacc);
              cacc = __builtin_fmaf(__int_as_float(p0[b].y), f16hi(sv[b].x), cacc);
              cacc = __builtin_fmaf(__int_as_float(p0[b].z), f16lo(sv[b].y), cacc);
              cacc = __builtin_fmaf(__int_as_float(p0[b].w), f16hi(sv[b].y), cacc);
              cacc = __builtin_fmaf(__int_as_float(p1[b].x), f16lo(sv[b].z), cacc);
              cacc = __builtin_fmaf(__int_as_float(p1[b].y), f16hi(sv[b].z), cacc);
              cacc = __builtin_fmaf(__int_as_float(p1[b].z), f16lo(sv[b].w), cacc);
              cacc = __builtin_fmaf(__int_as_float(p1[b].w), f16hi(sv[b].w), cacc);
            }
          });
        };
        const int nfull = npr / CHP * CHP;
        for (int pr = 0; pr < nfull; pr += CHP) block(pr, std::false_type{});
        if (nfull < npr) block(nfull, std::true_type{});
        sfor<0, CHP>([&](auto bc) {
          constexpr int b = decltype(bc)::value;
          lgkm_wait3<0>(p0[b], p1[b], sv[b]);
        });
        a.C[(size_t)m * a.ldc + n] = (cacc * 0.0625f) * ASC[m];
      } else {
        // any group size, and the raw per-group sums
        float cacc = 0.0f;
        int gsum = 0;
        for (int kt = 0; kt < KB; kt++) {
          gsum += P[kt];
          if ((kt + 1) % gk == 0) {
            if (RAW) a.acc_out[((size_t)(kt / gk) * M + m) * a.ldacc + n] = gsum >> 4;
            else cacc = __builtin_fmaf((float)gsum, Sc[kt / gk], cacc);
            gsum = 0;
          }
        }
        if (!RAW) a.C[(size_t)m * a.ldc + n] = cacc * ASC[m];
      }
    }
    return;
  }

  // ---- q8c: the KS partial sums of an n-block, added in LDS (the ring is
  // free now)
  float* BSC = (float*)(smem + L.bsc);
  if (!RAW && tid < nb_here * 16) BSC[tid] = cscale;
  __syncthreads();
  int32_t* R = (int32_t*)(smem + L.ring);
  if (w < NWP && (!HALF || g < 2)) {
#pragma unroll
    for (int mb = 0; mb < MB; mb++)
#pragma unroll
      for (int r = 0; r < 4; r++) R[w * OUT + (16 * mb + 4 * g + r) * 16 + j] = acc[mb][r];
  }
  __syncthreads();
  for (int o = tid; o < NBW * OUT; o += NT) {
    const int qq = o / OUT, oo = o - qq * OUT, m = oo >> 4, c = oo & 15;
    if (qq >= nb_here || m >= M) continue;
    int32_t sum = 0;
    for (int ss = 0; ss < KS; ss++) sum += R[(qq * KS + ss) * OUT + oo];
    const int n = (nb_first + qq) * 16 + c;
    if (RAW) a.acc_out[(size_t)m * a.ldacc + n] = sum;
    else a.C[(size_t)m * a.ldc + n] = (float)sum * (BSC[qq * 16 + c] * ASC[m]);
  }
}

// Park-in-ring grids whose waves stream four units per n-block (UPW = 4:
// K = 2048, 4096, 8192 with 4, 8, 16 waves): each wave streams ITS k-slice
// of TWO consecutive n-blocks, so one activation fragment serves two weight
// units (a wave's fragments are as many bytes as its weights otherwise, and
// they cost: the 134 MB stream ran 30.0 us with them, 26 us without).  A
// workgroup: 2 n-blocks, KS waves; wave s holds units s * 4 .. s * 4 + 3 of
// both in eight ring slots (n-block i's unit u in slot 4 i + u) and parks
// each unit's sums in its slot, so n-block i's pair p = 4 s + u lies at
// 1 KB x (8 s + 4 i + u): groups of four pairs (one wave's units) 8 KB
// apart.  Per n-block the arithmetic is decode_kernel's park-in-ring path,
// so the bytes are too.
//
// Vector-memory order of a wave: per unit u, n-block 0's and n-block 1's
// weights and the unit's activation fragment (X2 = 3), all four units at
// once; then PRE.  So unit u has landed when at most (3 - u) X2 + PRE remain.
template <int NPW>
__global__ __launch_bounds__(1024) void decode_pir2_kernel(GemmBatch bt) {
  constexpr int OUT = 128, UPW = 4, X2 = NPW + 1, PRE = SPT + 1, LNPW = NPW == 4 ? 2 : 1;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const GemmProb a = pick_problem(bt);
  fetch_all(a);
  if ((int)blockIdx.x >= a.nwg) return;
  const int tid = threadIdx.x, NT = blockDim.x;
  const int w = wave_id(), l = tid & 63, g = l >> 4, j = l & 15;
  const int M = a.M, N = a.N, KB = a.K >> 6;
  const int KS = NT >> 6, NG = KB;
  const Lay L(4, OUT, NPW * UPW, KS, NPW * UPW, KS, NPW, KB, 8, true);
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
  const int s = w;
  int lb = (int)blockIdx.x;
  const int nwgp = a.nwg;
  if ((nwgp & 7) == 0) lb = (lb & 7) * (nwgp >> 3) + (lb >> 3);
  const int nb_first = a.n0 + lb * NPW;
  const int nb_here = min(NPW, a.n0 + a.nblocks - nb_first);

  // ---- the stream: both n-blocks' units and the activation fragments
  const uint32_t bsw = 16u * (uint32_t)(l ^ (((l >> 3) & 3) << 1));
  v4i rbs[NPW];
#pragma unroll
  for (int i = 0; i < NPW; i++)
    rbs[i] = rsrc_words((const int8_t*)a.B + (size_t)(nb_first + (i < nb_here ? i : 0)) * KB * 512,
                        i < nb_here ? (uint32_t)KB * 512 : 0u);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(a.A, (uint32_t)((M + 15) / 16) * KB * 1024);
  const int r8 = j & 7;
  const uint32_t avoff = r8 < M ? (uint32_t)((j >> 3) * 1024 + r8 * 64 + 16 * g) : FGM_OOB;
  const uint32_t ring_w = lds0 + L.ring + (uint32_t)w * L.slots * 1024;
  v4i af[UPW];
#pragma unroll
  for (int u = 0; u < UPW; u++) {
    const uint32_t gu = (uint32_t)(s * UPW + u);
#pragma unroll
    // (the default cache policy: on these grids of many rounds of workgroups
    // it streams better than the non-temporal one the one-round grids use,
    // 134 MB stream 29.25 -> 28.05 us)
    for (int i = 0; i < NPW; i++) dma16<false>(rbs[i], ring_w + (i * UPW + u) * 1024, bsw, gu * 1024u);
    af[u] = buf_load_b128(ra, avoff, gu * 2048u);
  }
  // ---- PRE: group scales of both n-blocks, a_scale
  uint32_t sreg[SPT];
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.b_scale, (uint32_t)NG * N * 2);
  constexpr int per_g = 8 * NPW;  // dwords per group: NPW n-blocks of 16 columns, two columns a dword
#pragma unroll
  for (int v = 0; v < SPT; v++) {
    const int i = tid + v * NT, gi = i >> (3 + LNPW), c2 = i - gi * per_g, qq = c2 >> 3;
    const bool ok = gi < NG && qq < nb_here;
    sreg[v] = (uint32_t)buf_load_b32(rs, ok ? (uint32_t)((gi * N + (nb_first + qq) * 16 + 2 * (c2 & 7)) * 2) : FGM_OOB, 0);
  }
  const __amdgpu_buffer_rsrc_t ras = make_rsrc(a.a_scale, (uint32_t)M * 4);
  const float rscale = __int_as_float(buf_load_b32(ras, tid < M ? (uint32_t)tid * 4 : FGM_OOB, 0));

  uint32_t boff[4];
#pragma unroll
  for (int t = 0; t < 4; t++) {
    const int c = (8 * g + 2 * t + ((j & 7) >> 2)) ^ (g << 1);
    boff[t] = 16u * (uint32_t)c + 4u * (uint32_t)(j & 3);
  }
  const int sh = j < 8 ? 4 : 0;

  sfor<0, UPW>([&](auto uc) {
    constexpr int u = decltype(uc)::value;
    wait_vm<(UPW - 1 - u) * X2 + PRE>();
    const v4i x0 = af[u];
    v4i x1;
#pragma unroll
    for (int d = 0; d < 4; d++) x1[d] = ror8(x0[d]);
#pragma unroll
    for (int i = 0; i < NPW; i++) {
      char* slot = smem + L.ring + ((size_t)w * L.slots + i * UPW + u) * 1024;
      v4i bv[2];
#pragma unroll
      for (int e = 0; e < 2; e++)
#pragma unroll
        for (int t = 0; t < 4; t++) {
          const uint32_t x = *(const uint32_t*)(slot + e * 512 + boff[t]);
          bv[e][t] = (int)((x << sh) & 0xF0F0F0F0u);
        }
      const v4i t0 = mfma16(x0, bv[0], v4i{0, 0, 0, 0});
      const v4i t1 = mfma16(x1, bv[1], v4i{0, 0, 0, 0});
      // park: the slot just read holds [output][k-tile of the unit]
      float* Pr = (float*)slot;
      if (g < 2) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int oo = (4 * g + r) * 16 + j;
          *(float2*)(Pr + 2 * oo) = float2{(float)t0[r], (float)t1[r]};
        }
      }
    }
  });
  wait_vm<0>();  // the stream and PRE landed; no DMA still writes the ring

  float* ASC = (float*)(smem + L.asc);
  if (tid < M) ASC[tid] = rscale;
  // group scales into LDS as f32 / 16 ([n-block][column][group], pitch ngp;
  // zero past the last group)
  float* S = (float*)(smem + L.scl);
#pragma unroll
  for (int v = 0; v < SPT; v++) {
    const int ii = tid + v * NT, gi = ii >> (3 + LNPW), c2 = ii - gi * per_g, qq = c2 >> 3;
    const bool ok = gi < NG && qq < nb_here;
    if (gi < L.ngp && qq < NPW) {
      float* d = S + (qq * 16 + 2 * (c2 & 7)) * L.ngp + gi;
      d[0] = ok ? f16_bits_to_f32((uint16_t)(sreg[v] & 0xFFFF)) * 0.0625f : 0.0f;
      d[L.ngp] = ok ? f16_bits_to_f32((uint16_t)(sreg[v] >> 16)) * 0.0625f : 0.0f;
    }
  }
  __syncthreads();
  for (int o = tid; o < NPW * OUT; o += NT) {
    const int qq = o / OUT, oo = o - qq * OUT, m = oo >> 4, c = oo & 15;
    if (qq >= nb_here || m >= M) continue;
    const int n = (nb_first + qq) * 16 + c;
    // decode_kernel's park-in-ring chain with this layout's group stride
    const int np = (KB + 1) >> 1, ng = (np + 3) >> 2, nfg = np >> 2;
    const uint32_t pb = lds0 + L.ring + (uint32_t)(qq * UPW) * 1024u + (uint32_t)oo * 8u;
    const uint32_t sb = lds0 + L.scl + (uint32_t)((qq * 16 + c) * L.ngp) * 4u;
    float cacc = 0.0f;
    v2i pv[2][4];
    v4i sv[2][2];
    pir_read(pv[0], sv[0], pb, sb);
    auto fold = [&](int gg, auto hc, auto partial) {
      constexpr int h = decltype(hc)::value;
      const int gn = gg + 1 < ng ? gg + 1 : ng - 1;
      pir_read(pv[h ^ 1], sv[h ^ 1], pb + 4096u * NPW * gn, sb + 32u * gn);
      pir_wait6(pv[h], sv[h]);
#pragma unroll
      for (int b = 0; b < 4; b++)
        if (!decltype(partial)::value || 4 * gg + b < np) {
          const int sx = sv[h][b >> 1][2 * (b & 1)], sy = sv[h][b >> 1][2 * (b & 1) + 1];
          cacc = __builtin_fmaf(__int_as_float(pv[h][b].x), __int_as_float(sx), cacc);
          cacc = __builtin_fmaf(__int_as_float(pv[h][b].y), __int_as_float(sy), cacc);
        }
    };
    int gg = 0;
    for (; gg + 2 <= nfg; gg += 2) {
      fold(gg, std::integral_constant<int, 0>{}, std::false_type{});
      fold(gg + 1, std::integral_constant<int, 1>{}, std::false_type{});
    }
    fold(gg, std::integral_constant<int, 0>{}, std::true_type{});
    fold(gg + 1, std::integral_constant<int, 1>{}, std::true_type{});
    pir_wait0(pv[0], sv[0]);
    pir_wait0(pv[1], sv[1]);
    a.C[(size_t)m * a.ldc + n] = cacc * ASC[m];
  }
}

int pow2ceil(int x) {
  int p = 1;
  while (p < x) p *= 2;
  return p;
}

// K split of one GEMM: KS stream waves per n-block (a power of two), each
// with UPW units of 1 KB.
void plan_split(int bits, int M, int K, int* ks, int* upw) {
  const int KB = K / 64, tpu = bits == 4 ? 2 : 1;
  const int kbu = (KB + tpu - 1) / tpu;
  int k = pow2ceil((kbu + FGM_DEC_UPW - 1) / FGM_DEC_UPW);
  if (k > MAX_WAVES) k = MAX_WAVES;
  *ks = k;
  *upw = (kbu + k - 1) / k;
}

Lay lay_for(int bits, int M, int K, int ks, int nws, int nbw, bool pir = false) {
  const int MB = (M + 15) / 16;
  const bool half = M <= 8;
  const int out = half ? 128 : 256 * MB;
  const int tpu = bits == 4 ? 2 : 1;
  const int upw = ((K / 64 + tpu - 1) / tpu + ks - 1) / ks;
  return Lay(bits, out, ring_depth(bits, MB, half, pir), ks, upw, nws, nbw, K / 64, half ? 8 : 16 * MB, pir);
}

// Does one problem fit a workgroup of nws waves with nbw n-blocks?
bool fits_wg(int bits, int M, int K, int group, int nws, int ks, int nbw, bool pir = false) {
  if (ks * nbw > nws || nws > MAX_WAVES) return false;
  const Lay L = lay_for(bits, M, K, ks, nws, nbw, pir);
  if (bits == 4) {
    // the group-scale prefetch covers every padded group slot
    const int slots_g = L.ngp > (K / 64 + 7) / 8 * 8 ? L.ngp : (K / 64 + 7) / 8 * 8;
    if (8 * nbw * slots_g > SPT * 64 * nws) return false;
    (void)group;
  } else {
    // the q8c reduction reuses the rings
    const int out = M <= 8 ? 128 : 256 * ((M + 15) / 16);
    if ((size_t)nws * out * 4 > (size_t)nws * L.slots * 1024) return false;
  }
  return L.total <= 160 * 1024;
}

template <int BITS, int MB, bool HALF, bool G1, bool RAW, bool PIR = false>
hipError_t launch_variant(const GemmBatch& bt, int nw, size_t lds, int nwg, hipStream_t st) {
  // one grid row per problem, as wide as the widest, a multiple of 8
  auto k = decode_kernel<BITS, MB, HALF, G1, RAW, PIR>;
  static hipError_t attr = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  if (attr != hipSuccess) return attr;
  hipLaunchKernelGGL(k, dim3((nwg + 7) / 8 * 8, bt.count), dim3(nw * 64), lds, st, bt);
  return hipGetLastError();
}

template <int BITS, int MB, bool HALF>
hipError_t launch_decode(const GemmBatch& bt, bool g1, bool raw, bool pir, int nw, size_t lds, int nwg,
                         hipStream_t st) {
  if constexpr (BITS == 4 && HALF) {
    if (pir) return launch_variant<4, 1, true, true, false, true>(bt, nw, lds, nwg, st);
  }
  if constexpr (BITS == 8) {
    return raw ? launch_variant<BITS, MB, HALF, false, true>(bt, nw, lds, nwg, st)
               : launch_variant<BITS, MB, HALF, false, false>(bt, nw, lds, nwg, st);
  }
  if (raw) return launch_variant<BITS, MB, HALF, false, true>(bt, nw, lds, nwg, st);
  return g1 ? launch_variant<BITS, MB, HALF, true, false>(bt, nw, lds, nwg, st)
            : launch_variant<BITS, MB, HALF, false, false>(bt, nw, lds, nwg, st);
}

}  // namespace

bool fgm_decode_fits(int bits, int M, int K, int group) {
  (void)group;
  if (M < 1 || M > 64) return false;
  if ((size_t)((M + 15) / 16) * K * 16 > 0x7FFFFFFFu) return false;  // buffer offsets
  int ks, upw;
  plan_split(bits, M, K, &ks, &upw);
  const int nws = ks < FGM_DEC_NWMIN ? FGM_DEC_NWMIN : ks;
  return fits_wg(bits, M, K, group, nws, ks, 1);
}

size_t fgm_decode_lds_bytes(int bits, int M, int K, int group) {
  (void)group;
  int ks, upw;
  plan_split(bits, M, K, &ks, &upw);
  const int nws = ks < FGM_DEC_NWMIN ? FGM_DEC_NWMIN : ks;
  return lay_for(bits, M, K, ks, nws, 1).total;
}

// Every problem of the batch gets the same number of stream waves NWS = the
// largest K split (at least FGM_DEC_NWMIN); a problem with a smaller split
// packs NWS / KS n-blocks into each workgroup, as far as LDS and the scale
// prefetch allow (waves without an n-block only take part in the barriers).
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
  // problems with the longest K first: their workgroups are dispatched first
  GemmBatch bt = in;
  for (int i = 1; i < bt.count; i++)
    for (int k = i; k > 0 && bt.p[k].K > bt.p[k - 1].K; k--) {
      const GemmProb t = bt.p[k];
      bt.p[k] = bt.p[k - 1];
      bt.p[k - 1] = t;
    }
  int NWS = FGM_DEC_NWMIN, MB = 0, Mmax = 0;
  for (int i = 0; i < bt.count; i++) {
    GemmProb& p = bt.p[i];
    plan_split(bits, p.M, p.K, &p.ks, &p.tw);
    if (p.ks > NWS) NWS = p.ks;
    const int mb = (p.M + 15) / 16;
    if (mb > MB) MB = mb;
    if (p.M > Mmax) Mmax = p.M;
  }
  const bool half = MB == 1 && Mmax <= 8;
  const int Mv = half ? 8 : 16 * MB;  // the variant's row blocking
  const bool g1 = bits == 4 && bt.p[0].group == 64;
  const bool raw = bt.p[0].acc_out != nullptr;
  // The tile sums go back into the ring when every slot is filled once --
  // and only for grids of many rounds of workgroups, where the smaller LDS
  // footprint buys occupancy (134 MB int4 stream, 8192 workgroups: 37.6 ->
  // 32.8 us).  Smaller grids keep the park area and the round-robin unit
  // order (the cfg2 pair, 256 workgroups: 7.75 us, 9.3 us with the park in
  // the ring; the cfg4 gate/up batch, 1024: 8.3 us, 8.8 us).
  bool pir = bits == 4 && half && g1 && !raw;
  long nwg_plain = 0;
  for (int i = 0; i < bt.count; i++) {
    const GemmProb& p = bt.p[i];
    pir = pir && p.tw <= ring_depth(4, 1, true, true);
    nwg_plain += (p.nblocks + NWS / p.ks - 1) / (NWS / p.ks);
  }
  pir = pir && nwg_plain > FGM_DEC_PIR_MIN_WGS;
  // two n-blocks per wave (decode_pir2_kernel): int4 group 64, M <= 8, four
  // units per wave and n-block, every problem split over all the waves
  bool two = bits == 4 && half && g1 && !raw && nwg_plain > FGM_DEC_PIR2_MIN_WGS;
  for (int i = 0; i < bt.count; i++) two = two && bt.p[i].tw == 4 && bt.p[i].ks == NWS;
  int nwg = 0;
  size_t lds = 0;
  for (int i = 0; i < bt.count; i++) {
    GemmProb& p = bt.p[i];
    int nbw = NWS / p.ks;
    while (nbw > 1 && (nbw > p.nblocks || !fits_wg(bits, Mv, p.K, p.group, NWS, p.ks, nbw, pir))) nbw /= 2;
    if (!fits_wg(bits, Mv, p.K, p.group, NWS, p.ks, nbw, pir)) return hipErrorInvalidValue;
    // the kernel splits waves and scale dwords by shifts
    if ((nbw & (nbw - 1)) || (p.ks & (p.ks - 1))) return hipErrorInvalidValue;
    p.nbw = nbw;
    p.nwg = (p.nblocks + nbw - 1) / nbw;
    nwg = std::max(nwg, p.nwg);
    const size_t need = lay_for(bits, Mv, p.K, p.ks, NWS, nbw, pir).total;
    if (need > lds) lds = need;
  }
  if (nwg == 0) return hipSuccess;
  // the kernel derives a problem's stream waves as KS * NBW; pad the others
  // up to the launch's NWS with idle n-blocks is not needed: every problem
  // uses NBW = NWS / KS unless its n-blocks run out
  const int NW = NWS;
  if (two) {
    GemmBatch b2 = bt;
    int nwg2 = 0;
    size_t lds2 = 0;
    constexpr int NPW = FGM_DEC_PIR_NPW;
    for (int i = 0; i < b2.count; i++) {
      GemmProb& p = b2.p[i];
      p.nbw = NPW;
      p.nwg = (p.nblocks + NPW - 1) / NPW;
      nwg2 = std::max(nwg2, p.nwg);
      lds2 = std::max(lds2, (size_t)Lay(4, 128, 4 * NPW, p.ks, 4 * NPW, NW, NPW, p.K / 64, 8, true).total);
    }
    if (lds2 <= 160 * 1024) {
      static hipError_t attr = hipFuncSetAttribute((const void*)decode_pir2_kernel<NPW>,
                                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
      if (attr != hipSuccess) return attr;
      hipLaunchKernelGGL(decode_pir2_kernel<NPW>, dim3((nwg2 + 7) / 8 * 8, b2.count), dim3(NW * 64), lds2, st, b2);
      return hipGetLastError();
    }
  }
  if (bits == 8) {
    if (half) return launch_decode<8, 1, true>(bt, g1, raw, false, NW, lds, nwg, st);
    switch (MB) {
      case 1: return launch_decode<8, 1, false>(bt, g1, raw, false, NW, lds, nwg, st);
      case 2: return launch_decode<8, 2, false>(bt, g1, raw, false, NW, lds, nwg, st);
      case 3: return launch_decode<8, 3, false>(bt, g1, raw, false, NW, lds, nwg, st);
      case 4: return launch_decode<8, 4, false>(bt, g1, raw, false, NW, lds, nwg, st);
    }
  } else {
    if (half) return launch_decode<4, 1, true>(bt, g1, raw, pir, NW, lds, nwg, st);
    switch (MB) {
      case 1: return launch_decode<4, 1, false>(bt, g1, raw, false, NW, lds, nwg, st);
      case 2: return launch_decode<4, 2, false>(bt, g1, raw, false, NW, lds, nwg, st);
      case 3: return launch_decode<4, 3, false>(bt, g1, raw, false, NW, lds, nwg, st);
      case 4: return launch_decode<4, 4, false>(bt, g1, raw, false, NW, lds, nwg, st);
    }
  }
  return hipErrorInvalidValue;
}
