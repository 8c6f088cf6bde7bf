// Dense prefill GEMM on gfx950 MFMA: the M > 64 replacement for
// fgm_gemm_q8c / fgm_gemm_q4g (amx_gemm.c:333-372, 444-475) and their VNNI
// twins (vnni_gemm.c:224-322).
//
// Workgroup tile BM x BN, WGM x WGN waves, each wave WMT x WNT tiles of
// v_mfma_i32_32x32x32_i8 (the i8 MFMA with the highest issue rate on gfx950).
// One 64-wide k-block per pipeline stage; NS stages in an LDS ring filled by
// buffer loads that write LDS directly (no registers, one 1 KB block per wave
// instruction), so NS - 1 k-blocks of loads stay in flight while the waves
// multiply; one barrier per k-block.
//
// MFMA operand mapping (lane l, h = l >> 5, row / column l & 31): step s of
// the k-block (two 32-wide steps) gives operand byte b = 4t + e of half h the
// k = 32s + 16h + 4t + e, i.e. k-tile row r = 8s + 4h + t of the weight tile.
// Output: lane l, register r holds row 8(r/4) + 4h + r%4, column l & 31.
//
// LDS layouts are permutations of the HBM bytes chosen so that every fragment
// read is free of bank conflicts:
//   A, per 16-row m-block (1 KB): row i at 64 i, its 16-byte chunk q at slot
//     q ^ ((i >> 2) & 3); the fragment of step s, half h is chunk 2s + h of
//     the row: one ds_read_b128.
//   int8 B, per n-block (1 KB + 64 B pad): weight row r (4 k, 16 columns) at
//     row position rho(r) = 8s + 4h + ((t + 2h) & 3); a fragment is four
//     ds_read_b32 (rows 8s + 4h + t, column c).
//   int4 B, per pair of n-blocks (1 KB): the second n-block's rows rotated by
//     two; four ds_read_b32 per fragment, then the lane keeps its column's
//     nibbles in the high half of each byte (x16, see fgm_decode.hip).
//
// Epilogues are the reference's: int8 is exact int32 over all of K, then
// (float)acc * (b_scale * a_scale) (vnni_gemm.c:206-219); int4 drains its
// int32 accumulators into an fp32 fma chain at the end of every scale group,
// in ascending group order, then multiplies by a_scale (vnni_gemm.c:258-285,
// 316-321).  The int4 sums are 16 * acc and the parked scales f32(s) / 16, an
// exact product.
#include <type_traits>

#include "fgm_common.h"
#include "fgm_kernels.h"

namespace {

typedef int v16i __attribute__((ext_vector_type(16)));

FGM_DEV v16i mfma32(v4i a, v4i b, v16i c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

// Row position of weight-tile row r in the int8 LDS layout (an involution).
FGM_DEV int rho(int r) { return (r & ~3) | ((r + 2 * ((r >> 2) & 1)) & 3); }

template <int BITS, int WMT, int WNT, int WGM, int WGN, int NS, int KS, int KW>
struct Cfg {
  // KW groups of WGM x WGN waves; group g multiplies the k-blocks of stages
  // g, g + KW, ... with a ring of its own (KW > 1: int8 only)
  static constexpr int NWG = WGM * WGN, NW = NWG * KW, T = 64 * NW;
  static constexpr int BM = 32 * WMT * WGM, BN = 32 * WNT * WGN;
  static constexpr int MBL = BM / 16, NBL = BN / 16;
  static constexpr int BUNIT = BITS == 8 ? 1088 : 1024;     // LDS bytes per B unit
  static constexpr int BUNITS = BITS == 8 ? NBL : NBL / 2;  // B units per stage
  static constexpr int A_BYTES = MBL * 1024;
  static constexpr int B_BYTES = BUNITS * BUNIT;
  static constexpr int S_BYTES = BITS == 4 ? 1024 : 0;      // int4 group scales
  static constexpr int KBLK = A_BYTES + B_BYTES + S_BYTES;  // one k-block
  static constexpr int STAGE = KS * KBLK;                     // KS k-blocks per ring slot
  // DMA instructions per wave per k-block (A units, B units, the int4
  // scales) and per stage
  static constexpr int UK = (MBL + NWG - 1) / NWG + (BUNITS + NWG - 1) / NWG + (BITS == 4 ? 1 : 0);
  static constexpr int U = KS * UK;
  static_assert((NS - 2) * U <= 63, "vmcnt range");
  // the ring, a 1 KB sink for the zero loads that keep the per-wave load
  // count fixed, the epilogue scales
  static constexpr size_t TRASH = (size_t)KW * NS * STAGE;
  static constexpr size_t LDS = TRASH + 1024 + (BM + (BN + 63) / 64 * 64) * 4;
  static_assert(BITS == 8 || NBL % 2 == 0, "int4 tiles come in n-block pairs");
  static_assert(KW == 1 || BITS == 8, "K groups: int8 (exact int32 partial sums)");
  // the groups' partial tiles are summed through the ring, one group at a
  // time, once the stream is done
  static_assert(KW == 1 || (size_t)BM * BN * 4 <= TRASH, "K-group reduction space");
  static_assert(LDS <= 160 * 1024, "LDS per workgroup");
  static_assert(BM % 64 == 0, "the epilogue's a_scale arrives in 64-row chunks");
};

template <int BITS, int WMT, int WNT, int WGM, int WGN, int NS, int KS, int KW, bool RAW, bool G1, bool ROT,
          bool BNT = false>
__global__ __launch_bounds__(64 * WGM * WGN * KW) void gemm_kernel(GemmBatch bt) {
  using C = Cfg<BITS, WMT, WNT, WGM, WGN, NS, KS, KW>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const GemmProb a = pick_problem(bt);
  fetch_all(a);
  const int tid = threadIdx.x, wv = wave_id(), l = tid & 63, h = l >> 5, l32 = l & 31;
  // K group kg, wave w within it
  const int kg = wv / C::NWG, w = wv - kg * C::NWG;
  const int wm = w % WGM, wn = w / WGM;

  const int M = a.M, N = a.N, KB = a.K >> 6;
  const int MT = (M + C::BM - 1) / C::BM;
  const int NT = (a.nblocks + C::NBL - 1) / C::NBL;
  const int ntiles = MT * NT;
  int bid = blockIdx.x;
  if (bid >= a.nwg) return;  // past this problem's tiles
  // Workgroup ids go round-robin over the 8 XCDs (the grid's width is a
  // multiple of 8, so workgroup x of every problem runs on XCD x % 8): give
  // each XCD a contiguous run of tiles in grouped order (GM m-tiles at a
  // time, n within a group), so that the tiles an L2 serves at once share A
  // rows and B columns.
  if ((ntiles & 7) == 0) bid = (bid & 7) * (ntiles >> 3) + (bid >> 3);
  const int GM = MT < 4 ? MT : 4;
  const int grp = bid / (GM * NT), inr = bid - grp * GM * NT;
  const int gm = (MT - grp * GM) < GM ? (MT - grp * GM) : GM;  // m-tiles in this group
  const int mtile = grp * GM + inr % gm, ntile = inr / gm;
  const int MBtot = (M + 15) >> 4;
  const int mb0 = mtile * C::MBL;              // first m-block of the tile
  const int nb0 = a.n0 + ntile * C::NBL;       // first n-block of the tile
  const int nbend = a.n0 + a.nblocks;
  const int gk = BITS == 4 ? a.group >> 6 : 1;

  // ---- DMA plan: wave w issues A units w, w + NW, ..., B units likewise,
  // and wave 0 the int4 scale unit; slots past the unit count load zeros
  // (FGM_OOB), so every wave issues exactly U loads per stage
  constexpr int UA = (C::MBL + C::NWG - 1) / C::NWG, UB = (C::BUNITS + C::NWG - 1) / C::NWG;
  constexpr int US = BITS == 4 ? 1 : 0;
  static_assert(UA + UB + US == C::UK, "unit plan");
  const v4i ra = rsrc_words(a.A, (uint32_t)MBtot * KB * 1024);
  const v4i rb = rsrc_words(a.B, (uint32_t)nbend * KB * (BITS == 8 ? 1024 : 512));
  // int4 group scales (raw-accumulator mode has none: an empty range, every
  // lane out of range)
  const v4i rsc = rsrc_words(a.b_scale, (BITS == 4 && !RAW) ? (uint32_t)(KB / gk) * N * 2 : 0);
  uint32_t avoffs[UA], alds[UA], bvoffs[UB], blds[UB], svoff = FGM_OOB;
  // LDS offsets are relative to a stage; a slot past the unit count targets
  // the sink (TRASH - stage base is resolved in issue())
  constexpr uint32_t SINK = 0xFFFFFFFFu;
#pragma unroll
  for (int i = 0; i < UA; i++) {
    const int u = w + C::NWG * i, mb = mb0 + u, row = l >> 2, q = (l & 3) ^ ((row >> 2) & 3);
    alds[i] = u < C::MBL ? u * 1024 : SINK;
    avoffs[i] = (u < C::MBL && mb < MBtot) ? (uint32_t)mb * KB * 1024 + row * 64 + 16 * q : FGM_OOB;
  }
#pragma unroll
  for (int i = 0; i < UB; i++) {
    const int u = w + C::NWG * i;
    blds[i] = u < C::BUNITS ? C::A_BYTES + u * C::BUNIT : SINK;
    bvoffs[i] = FGM_OOB;
    if (BITS == 8) {
      const int nb = nb0 + u, R = l >> 2, q = l & 3;
      if (u < C::BUNITS && nb < nbend) bvoffs[i] = (uint32_t)nb * KB * 1024 + rho(R) * 64 + 16 * q;
    } else {
      const int n2 = l >> 5, R = (l & 31) >> 1, q = l & 1;
      const int nb = nb0 + 2 * u + n2, r = n2 ? ((R - 2) & 15) : R;
      if (u < C::BUNITS && nb < nbend) bvoffs[i] = (uint32_t)nb * KB * 512 + r * 32 + 16 * q;
    }
  }
  if (BITS == 4 && !RAW && w == 0) {
    const int col = nb0 * 16 + 8 * l;
    if (l < C::BN / 8 && col < nbend * 16) svoff = (uint32_t)col * 2;
  }
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
  const uint32_t sink = lds0 + (uint32_t)C::TRASH;
  // this K group's ring
  const uint32_t ring0 = lds0 + (uint32_t)(kg * NS * C::STAGE);
  const char* const gring = smem + kg * NS * C::STAGE;
  // ROT (int8, whose int32 sum is exact in any k order): workgroup b walks K
  // from k-block 5 b mod KB, so the tiles that share A rows or B columns read
  // different k-blocks at a time instead of the same lines at once (M = 256,
  // N = 2048, K = 8192, weights rotating over 20 copies: 15.9 -> 15.6 us;
  // 15.8 -> 13.7 us in a bare stream of launches on constant-filled
  // operands; for M = 2048 the shared lines are what the L2 reuses, and the
  // rotation doubles the time)
  static_assert(!ROT || BITS == 8, "k rotation: int8 only");
  const int rot = ROT ? (int)((uint32_t)bid * 5u % (uint32_t)KB) : 0;
  // loads of k-block j of the group's stage sidx (k-blocks KS * (KW * sidx +
  // kg) ...) into ring slot `slot`; zeros past K, which land in k-blocks that
  // are never multiplied
  auto issue_part = [&](int sidx, int slot, int j) {
    int kb = (sidx * KW + kg) * KS + j;
    const bool live = kb < KB;
    if (ROT && live) kb = kb + rot < KB ? kb + rot : kb + rot - KB;
    const uint32_t sb = ring0 + slot * C::STAGE + j * C::KBLK;
#pragma unroll
    for (int i = 0; i < UA; i++)
      dma16(ra, alds[i] == SINK ? sink : sb + alds[i], live ? avoffs[i] : FGM_OOB, (uint32_t)kb * 1024);
#pragma unroll
    for (int i = 0; i < UB; i++)
      dma16<BNT>(rb, blds[i] == SINK ? sink : sb + blds[i], live ? bvoffs[i] : FGM_OOB,
            (uint32_t)kb * (BITS == 8 ? 1024 : 512));
    if (BITS == 4)
      dma16(rsc, w == 0 ? sb + C::A_BYTES + C::B_BYTES : sink, live ? svoff : FGM_OOB,
            live ? (uint32_t)(kb / gk) * N * 2 : 0);
  };
  auto issue = [&](int sidx, int slot) {
#pragma unroll
    for (int j = 0; j < KS; j++) issue_part(sidx, slot, j);
  };

  // epilogue scales in LDS, after the ring: a_scale [BM], (int8) b_scale [BN],
  // brought in by 256-byte DMA chunks issued before the first stage, so that
  // the wait for stage 0 covers them; rows past M and columns past n1 read
  // zeros
  float* ASC = (float*)(smem + C::TRASH + 1024);
  float* BSC = ASC + C::BM;
  {
    constexpr int NCA = RAW ? 0 : C::BM / 64;
    constexpr int NCB = (RAW || BITS == 4) ? 0 : (C::BN + 63) / 64;
    constexpr int CH = (NCA + NCB + C::NW - 1) / C::NW;
    const v4i rsa = rsrc_words(a.a_scale, RAW ? 0u : (uint32_t)M * 4);
    const v4i rsb = rsrc_words(a.b_scale, NCB ? (uint32_t)nbend * 64 : 0u);
#pragma unroll
    for (int i = 0; i < CH; i++) {
      const int c = wv + C::NW * i;
      if (c < NCA)
        dma4(rsa, lds0 + (uint32_t)C::TRASH + 1024 + c * 256, (uint32_t)(mtile * C::BM + 64 * c + l) * 4, 0);
      else if (c < NCA + NCB)
        dma4(rsb, lds0 + (uint32_t)C::TRASH + 1024 + C::BM * 4 + (c - NCA) * 256,
             (uint32_t)(nb0 * 16 + 64 * (c - NCA) + l) * 4, 0);
      else
        dma4(rsa, sink, FGM_OOB, 0);
    }
  }

  v16i acc[WMT][WNT];
  float cf[BITS == 4 ? WMT : 1][BITS == 4 ? WNT : 1][16];
#pragma unroll
  for (int x = 0; x < WMT; x++)
#pragma unroll
    for (int y = 0; y < WNT; y++) {
      acc[x][y] = v16i{};
      if (BITS == 4)
#pragma unroll
        for (int r = 0; r < 16; r++) cf[x][y][r] = 0.0f;
    }

  // per-lane fragment addresses within a stage
  uint32_t aoff[WMT][2];  // [m tile][step]: ds_read_b128
#pragma unroll
  for (int x = 0; x < WMT; x++) {
    const int row = wm * WMT * 32 + x * 32 + l32, mbl = row >> 4, i = row & 15;
#pragma unroll
    for (int s = 0; s < 2; s++) aoff[x][s] = mbl * 1024 + i * 64 + 16 * ((2 * s + h) ^ ((i >> 2) & 3));
  }
  uint32_t boff[WNT];     // + row offset below
  int bsh = 0;            // int4: nibble shift of this lane's column
#pragma unroll
  for (int y = 0; y < WNT; y++) {
    const int col = wn * WNT * 32 + y * 32 + l32, nbl = col >> 4, c = col & 15;
    if (BITS == 8) {
      boff[y] = C::A_BYTES + nbl * C::BUNIT + 4 * c;
    } else {
      boff[y] = C::A_BYTES + (nbl >> 1) * 1024 + (nbl & 1) * 512 + 4 * (c & 7);
      bsh = c < 8 ? 4 : 0;
    }
  }
  // int4: this lane's column of the staged scales, per n tile
  uint32_t soffl[WNT];
#pragma unroll
  for (int y = 0; y < WNT; y++) soffl[y] = C::A_BYTES + C::B_BYTES + 2 * (wn * WNT * 32 + y * 32 + l32);

  // Fragments of one k-block in NG groups: group g is step s = g / (WMT + WNT)
  // and then an A fragment (m tile r < WMT) or a B fragment (n tile r - WMT);
  // the int4 group scale rides with the last B group.
  constexpr int NG = 2 * (WMT + WNT), NM = 2 * WMT * WNT;
  v4i af[2][2][WMT], bf[2][2][WNT];
  float scl[2][WNT];
  auto fetch_grp = [&](auto bufc, auto gc, const char* st) {
    constexpr int buf = decltype(bufc)::value, g = decltype(gc)::value;
    constexpr int s = g / (WMT + WNT), r = g % (WMT + WNT);
    if constexpr (r < WMT) {
      af[buf][s][r] = *(const v4i*)(st + aoff[r][s]);
    } else {
      constexpr int y = r - WMT;
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const int rr = 8 * s + 4 * h + t;
        if (BITS == 8) {
          bf[buf][s][y][t] = *(const int32_t*)(st + boff[y] + rho(rr) * 64);
        } else {
          const int nbl = ((wn * WNT * 32 + y * 32 + l32) >> 4) & 1;
          const uint32_t xv = *(const uint32_t*)(st + boff[y] + ((rr + 2 * nbl) & 15) * 32);
          bf[buf][s][y][t] = (int)((xv << bsh) & 0xF0F0F0F0u);
        }
      }
      if constexpr (BITS == 4 && !RAW && s == 1)
        scl[buf][y] = f16_bits_to_f32(*(const uint16_t*)(st + soffl[y])) * 0.0625f;
    }
  };

  // The multiplies of one k-block (register set cur) with the next k-block's
  // fragment reads and one DMA part of a refill placed between them, so that
  // LDS latency and load issue hide behind the matrix cores.  An int4 group
  // starts from a zero accumulator (every k-block when the group is 64).
  auto mma = [&](auto setc, bool fresh, int rs, int rslot, int rj, const char* nst) {
    constexpr int cur = decltype(setc)::value;
    sfor<0, NM>([&](auto mc) {
      constexpr int m = decltype(mc)::value;
      constexpr int s = m / (WMT * WNT), x = (m / WNT) % WMT, y = m % WNT;
      if constexpr (BITS == 4 && s == 0) {
        if constexpr (G1) acc[x][y] = mfma32(af[cur][0][x], bf[cur][0][y], v16i{});
        else acc[x][y] = mfma32(af[cur][0][x], bf[cur][0][y], fresh ? v16i{} : acc[x][y]);
      } else {
        acc[x][y] = mfma32(af[cur][s][x], bf[cur][s][y], acc[x][y]);
      }
      if constexpr (m == 0) issue_part(rs, rslot, rj);
      sfor<m * NG / NM, (m + 1) * NG / NM>(
          [&](auto gc) { fetch_grp(std::integral_constant<int, cur ^ 1>{}, gc, nst); });
      __builtin_amdgcn_sched_barrier(0);
    });
  };
  // int4: at the end of a scale group, fold the group's sums into the fp32
  // chain (or dump them raw)
  auto drain = [&](auto setc, int kb) {
    constexpr int cur = decltype(setc)::value;
    if (BITS != 4 || kb >= KB || ((kb + 1) % gk) != 0) return;
    const int gi = kb / gk;
#pragma unroll
    for (int y = 0; y < WNT; y++) {
      const int n = nb0 * 16 + wn * WNT * 32 + y * 32 + l32;
      if (RAW) {
#pragma unroll
        for (int x = 0; x < WMT; x++)
#pragma unroll
          for (int r = 0; r < 16; r++) {
            const int m = mtile * C::BM + wm * WMT * 32 + x * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (m < M && n < nbend * 16) a.acc_out[((size_t)gi * M + m) * a.ldacc + n] = acc[x][y][r] >> 4;
          }
      } else {
        const float sc = scl[cur][y];
#pragma unroll
        for (int x = 0; x < WMT; x++)
#pragma unroll
          for (int r = 0; r < 16; r++) cf[x][y][r] = __builtin_fmaf((float)acc[x][y][r], sc, cf[x][y][r]);
      }
    }
  };

  // ---- prologue: stages 0 .. NS - 2 in flight, stage 0 landed, part 0 of
  // stage NS - 1 issued (its other parts go out during stage 0)
#pragma unroll
  for (int s = 0; s < NS - 1; s++) issue(s, s);
  wait_vm<(NS - 2) * C::U>();
  __syncthreads();
  issue_part(NS - 1, NS - 1, 0);
  sfor<0, NG>([&](auto gc) {  // in group order, as the loop reads them
    fetch_grp(std::integral_constant<int, 0>{}, gc, gring);
    __builtin_amdgcn_sched_barrier(0);
  });

  // ---- main loop.  Stage sidx, k-block j: while k-block j multiplies, part
  // j + 1 of the refill of the previous stage's slot goes out and k-block
  // j + 1 is read.  At the last k-block of a stage the wave first waits for
  // stage sidx + 1 (all its parts were issued during stage sidx) and the
  // barrier frees slot sidx, whose refill (stage sidx + NS) starts.  Trips of
  // U2 stages keep the register set of every k-block a constant; k-blocks
  // past K hold zeros.
  // One trip covers UR stages, a whole number of ring rounds (and an even
  // number of k-blocks, so the register set of every k-block is a constant):
  // every stage's ring slot is then a constant too and its fragment
  // addresses fold into the reads' immediate offsets instead of being
  // recomputed per stage.  Stages past the last one holding k-blocks of K
  // are skipped (the condition is the same for every wave of the workgroup).
  constexpr int U2 = KS % 2 == 0 ? 1 : 2;
  constexpr int UR = NS % U2 == 0 ? NS : (U2 % NS == 0 ? U2 : NS * U2);
  const int NSTG = (KB + KS * KW - 1) / (KS * KW);
  for (int sb = 0; sb < NSTG; sb += UR) {
    sfor<0, UR * KS>([&](auto ic) {
      constexpr int i = decltype(ic)::value, u = i / KS, j = i % KS, cur = i & 1;
      constexpr int slot = u % NS, prev = (u + NS - 1) % NS, next = (u + 1) % NS;
      const int sidx = sb + u;
      if (sidx < NSTG) {
        const int kb = (sidx * KW + kg) * KS + j;
        const bool fresh = BITS == 4 && (kb % gk) == 0;
        if constexpr (j + 1 < KS) {
          mma(std::integral_constant<int, cur>{}, fresh, sidx - 1 + NS, prev, j + 1,
              gring + slot * C::STAGE + (j + 1) * C::KBLK);
        } else {
          wait_vm<(NS - 2) * C::U>();
          __syncthreads();
          mma(std::integral_constant<int, cur>{}, fresh, sidx + NS, slot, 0, gring + next * C::STAGE);
        }
        drain(std::integral_constant<int, cur>{}, kb);
      }
    });
  }
  wait_vm<0>();

  // ---- K groups: group gg = 1 .. KW - 1 in turn parks its int32 tile in
  // the ring and group 0 adds it (exact); group 0 runs the epilogue
  if constexpr (KW > 1) {
    int32_t* R = (int32_t*)smem;
    auto at = [&](int x, int y, int r) { return (((w * WMT + x) * WNT + y) * 16 + r) * 64 + l; };
    for (int gg = 1; gg < KW; gg++) {
      __syncthreads();  // every group is done with its ring / the last sum is read
      if (kg == gg) {
#pragma unroll
        for (int x = 0; x < WMT; x++)
#pragma unroll
          for (int y = 0; y < WNT; y++)
#pragma unroll
            for (int r = 0; r < 16; r++) R[at(x, y, r)] = acc[x][y][r];
      }
      __syncthreads();
      if (kg == 0) {
#pragma unroll
        for (int x = 0; x < WMT; x++)
#pragma unroll
          for (int y = 0; y < WNT; y++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[x][y][r] += R[at(x, y, r)];
      }
    }
    if (kg > 0) return;
  }

  // ---- epilogue: one buffer store per output.  The buffer starts at the
  // tile's first row and column (callers may pass C shifted so that column
  // 16 n0 is its first stored one) and ends after the tile's last stored
  // element: rows past M fall outside it, columns past n1 are masked.
  if (BITS == 4 && RAW) return;
  const int mrow0 = mtile * C::BM;
  const int mrows = M - mrow0 < C::BM ? M - mrow0 : C::BM;
  const int ld = RAW ? a.ldacc : a.ldc;
  const int ncols = nbend * 16 - nb0 * 16 < C::BN ? nbend * 16 - nb0 * 16 : C::BN;
  const size_t o0 = (size_t)mrow0 * ld + (size_t)nb0 * 16;
  const void* obase = RAW ? (const void*)(a.acc_out + o0) : (const void*)(a.C + o0);
  const __amdgpu_buffer_rsrc_t ro =
      make_rsrc(obase, ((uint32_t)(mrows - 1) * (uint32_t)ld + (uint32_t)ncols) * 4u);
#pragma unroll
  for (int y = 0; y < WNT; y++) {
    const int coll = wn * WNT * 32 + y * 32 + l32, n = nb0 * 16 + coll;
    if (n >= nbend * 16) continue;
    const float bsn = (BITS == 8 && !RAW) ? BSC[coll] : 0.0f;
#pragma unroll
    for (int x = 0; x < WMT; x++)
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int rowq = wm * WMT * 32 + x * 32 + 8 * q + 4 * h;  // rows rowq .. rowq + 3
        const float4 as4 = RAW ? float4{} : *(const float4*)(ASC + rowq);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int r = 4 * q + e;
          const float ase = e == 0 ? as4.x : e == 1 ? as4.y : e == 2 ? as4.z : as4.w;
          uint32_t v;
          if (BITS == 8 && RAW) v = (uint32_t)acc[x][y][r];
          else if (BITS == 8) v = __float_as_uint((float)acc[x][y][r] * (bsn * ase));
          else v = __float_as_uint(cf[x][y][r] * ase);
          // non-temporal (cache policy nt): every tile stores at once at the
          // end, and streaming the outputs out beats parking them in L2 for
          // the kernel's final write-back (M = 256 gate / up 9.3 -> 8.6 us,
          // layer 46.5 -> 45.0 us on one weight copy; M = 2048 down 39.4 ->
          // 38.0 us)
          __builtin_amdgcn_raw_buffer_store_b32(v, ro, (int)(((uint32_t)(rowq + e) * (uint32_t)ld + (uint32_t)coll) * 4u), 0,
                                                FGM_CPOL_NT);
        }
      }
  }
}

template <int BITS, int WMT, int WNT, int WGM, int WGN, int NS, int KS, int KW, bool RAW, bool G1, bool ROT,
          bool BNT>
hipError_t launch_cfg(const GemmBatch& in, hipStream_t st) {
  using C = Cfg<BITS, WMT, WNT, WGM, WGN, NS, KS, KW>;
  auto k = gemm_kernel<BITS, WMT, WNT, WGM, WGN, NS, KS, KW, RAW, G1, ROT, BNT>;
  static hipError_t attr =
      hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)C::LDS);
  if (attr != hipSuccess) return attr;
  GemmBatch b = in;
  int nwg = 0;
  for (int i = 0; i < b.count; i++) {
    GemmProb& p = b.p[i];
    // the epilogue addresses one m-tile of C with 32-bit buffer offsets
    if ((size_t)C::BM * (size_t)(p.acc_out ? p.ldacc : p.ldc) * 4 > 0xFFFFFFFFull) return hipErrorInvalidValue;
    p.nwg = ((p.M + C::BM - 1) / C::BM) * ((p.nblocks + C::NBL - 1) / C::NBL);
    nwg = nwg > p.nwg ? nwg : p.nwg;
  }
  if (nwg == 0) return hipSuccess;
  // one grid row per problem, as wide as the widest, a multiple of 8
  hipLaunchKernelGGL(k, dim3((nwg + 7) / 8 * 8, b.count), dim3(C::T), C::LDS, st, b);
  return hipGetLastError();
}

// Variant: raw-accumulator dumps or scaled outputs; int4 with 64-wide groups
// (a fresh accumulator every k-block) or the general group size.
template <int BITS, int WMT, int WNT, int WGM, int WGN, int NS, int KS, int KW = 1, bool ROT = false, bool BNT = false>
hipError_t launch_any(const GemmBatch& b, hipStream_t st) {
  if (b.p[0].acc_out) return launch_cfg<BITS, WMT, WNT, WGM, WGN, NS, KS, KW, true, false, ROT, BNT>(b, st);
  bool g1 = BITS == 4;
  for (int i = 0; i < b.count; i++) g1 = g1 && b.p[i].group == 64;
  return g1 ? launch_cfg<BITS, WMT, WNT, WGM, WGN, NS, KS, KW, false, BITS == 4, ROT, BNT>(b, st)
            : launch_cfg<BITS, WMT, WNT, WGM, WGN, NS, KS, KW, false, false, ROT, BNT>(b, st);
}

// Shortest K of a batch.
int kmin(const GemmBatch& b) {
  int k = b.p[0].K;
  for (int i = 1; i < b.count; i++) k = b.p[i].K < k ? b.p[i].K : k;
  return k;
}

// Most rows of a batch's problems.
int mmax(const GemmBatch& b) {
  int m = b.p[0].M;
  for (int i = 1; i < b.count; i++) m = b.p[i].M > m ? b.p[i].M : m;
  return m;
}

// Workgroup tiles of a batch for a BM x BN tile.
long tiles(const GemmBatch& b, int bm, int bn) {
  long t = 0;
  for (int i = 0; i < b.count; i++) t += (long)((b.p[i].M + bm - 1) / bm) * ((b.p[i].nblocks + bn / 16 - 1) / (bn / 16));
  return t;
}

}  // namespace

hipError_t fgm_launch_gemm(int bits, const GemmBatch& in, hipStream_t st) {
  // one kernel variant per launch: raw-accumulator and scaled problems apart
  for (int i = 1; i < in.count; i++)
    if ((in.p[i].acc_out != nullptr) != (in.p[0].acc_out != nullptr)) {
      GemmBatch x{}, y{};
      for (int k = 0; k < in.count; k++) {
        GemmBatch& d = (in.p[k].acc_out != nullptr) == (in.p[0].acc_out != nullptr) ? x : y;
        d.p[d.count++] = in.p[k];
      }
      hipError_t e = fgm_launch_gemm(bits, x, st);
      return e != hipSuccess ? e : fgm_launch_gemm(bits, y, st);
    }
  // Tile and ring, from measured sweeps on MI355X: the largest tile that
  // still puts a workgroup on (nearly) every CU; rings of NS slots of KS
  // k-blocks.  Small int8 problems (the M = 256 projections) split K over
  // groups of waves inside the workgroup: a wave's loads are issued at a
  // bounded rate (about 16 GB/s per wave from L2 on MI355X), so a small tile
  // needs more waves streaming it, and each group walks a quarter or half of
  // K (q 7.5 -> 6.9 us, down 19 -> 13 us, q + k + v 9.1 -> 7.6 us at M = 256;
  // M = 2048 down, K = 8192: 42.4 -> 38.9 us).  One k-block per stage, four
  // stages per K group, for long K and for the 64x32 tiles (M = 2048 down
  // 34.8 -> 31.0 us; M = 256 q 7.4 -> 7.2 us, down 15.7 -> 15.4 us, weights
  // from HBM; the k rotation on the down projection 15.9 -> 15.6 us).  Eight
  // K groups of 16 waves, or the 128x64 tile on eight 32x32 waves, measured
  // slower (q 8.4, gate 12.9 us).
  if (bits == 8) {
    // With at most 256 rows, two to four m-tiles share a weight tile and the
    // weights are read with the non-temporal policy (M = 256, weights from
    // HBM: q / o 6.85 -> 6.65 us, gate 10.2 -> 9.7 us, the 4-launch layer
    // 50.3 -> 47.0 us); the down projection's k-rotated tiles (15.1 -> 15.8
    // us) and every M = 2048 shape (down 38.7 -> 45.6 us: sixteen m-tiles
    // share a weight tile there) keep the default policy.
    const bool bnt = mmax(in) <= 256;
    if (tiles(in, 256, 128) >= 480) return launch_any<8, 4, 2, 2, 2, 2, 1>(in, st);
    if (tiles(in, 128, 128) >= 240) {  // long K (the down projection): two K groups
      if (kmin(in) >= 4096) return launch_any<8, 2, 2, 2, 2, 4, 1, 2>(in, st);
      return bnt ? launch_any<8, 2, 2, 2, 2, 4, 2, 1, false, true>(in, st)
                 : launch_any<8, 2, 2, 2, 2, 4, 2>(in, st);
    }
    if (tiles(in, 128, 64) >= 240)
      return bnt ? launch_any<8, 2, 1, 2, 2, 4, 2, 1, false, true>(in, st) : launch_any<8, 2, 1, 2, 2, 4, 2>(in, st);
    if (tiles(in, 64, 64) >= 160)
      return bnt ? launch_any<8, 1, 1, 2, 2, 3, 2, 2, false, true>(in, st) : launch_any<8, 1, 1, 2, 2, 3, 2, 2>(in, st);
    if (kmin(in) >= 8192) return launch_any<8, 1, 1, 2, 1, 4, 1, 4, true>(in, st);
    return bnt ? launch_any<8, 1, 1, 2, 1, 4, 1, 4, false, true>(in, st) : launch_any<8, 1, 1, 2, 1, 4, 1, 4>(in, st);
  }
  if (tiles(in, 128, 128) >= 480) return launch_any<4, 2, 2, 2, 2, 2, 2>(in, st);
  if (tiles(in, 128, 64) >= 240) return launch_any<4, 2, 1, 2, 2, 2, 2>(in, st);
  return launch_any<4, 1, 1, 2, 1, 4, 2>(in, st);
}
