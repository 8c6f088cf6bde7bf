// Internal launcher interface between the C-ABI layer (fgm_api.hip) and the
// kernels.  All pointers are device pointers; shapes are validated by the
// caller before any launch.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

// Independent problems served by one launch.
constexpr int FGM_MAX_BATCH = 4;

// Problem i of a batch is row blockIdx.y = i of a 2-D grid and owns its
// workgroups blockIdx.x = 0 .. p[i].nwg - 1; the grid is as wide as the
// widest problem and the others' surplus workgroups exit at once.  The
// problem is read at an address every workgroup knows when it starts: one
// round of argument fetches at kernel start, not a fetch to find the problem
// and a second to read it (each is a memory round trip while the argument
// lines are cold).
template <class Batch>
__device__ __forceinline__ auto pick_problem(const Batch& bt) {
  return bt.p[blockIdx.y];
}

struct GemmProb {
  const int8_t* A;        // packed A [ceil(M/16)][K/64][16][64]
  const float* a_scale;   // [M]
  const void* B;          // int8 tiles, or packed int4 tiles
  const void* b_scale;    // f32 [N] (q8c) or f16 bits [K/group][N] (q4g)
  float* C;
  int32_t* acc_out;       // raw int32 accumulators instead of C when non-null
  int M, N, K, group, ldc, ldacc;
  int n0, nblocks;        // n-block range [n0, n0 + nblocks)
  int nwg;                // workgroups of this problem (set by the launcher)
  int tw, ks, nbw;        // skinny path: k-blocks per wave, waves per n-block,
                          // n-blocks per workgroup (set by the launcher)
};

struct GemmBatch {
  GemmProb p[FGM_MAX_BATCH];
  int count;
};

struct PrepProb {
  const float* src;
  float* rot;      // may be null (device API only)
  int8_t* qa;      // may be null (device API only)
  float* qs;
  int8_t* pa;      // null for quant_act
  int lda, m, k, hsz, r0, r1;
  float fwht_scale;
  int nwg;         // workgroups of this problem (set by the launcher)
  // fused producer applied to each row before the rotation (one kind per
  // batch): PREP_RMSNORM normalises src by aux (NULL: no scale) with eps;
  // PREP_GELU_MUL takes gelu(src) * aux, aux rows lda apart.  pre, when set,
  // receives that result as [m][k] (the reference's xn / act buffer).
  int preop;
  const float* aux;
  float* pre;
  float eps;
};
// Every field of the problem (and the workgroup size) in registers at once:
// the kernels test whether a workgroup is past its problem first, and the
// compiler would otherwise fetch the fields that test needs, branch, and
// fetch the rest in a second dependent round.
__device__ __forceinline__ void fetch_all(const GemmProb& a) {
  asm volatile("" ::"s"(a.A), "s"(a.a_scale), "s"(a.B), "s"(a.b_scale), "s"(a.C), "s"(a.acc_out),
               "s"(a.M), "s"(a.N), "s"(a.K), "s"(a.group), "s"(a.ldc), "s"(a.ldacc), "s"(a.n0),
               "s"(a.nblocks), "s"(a.nwg), "s"(a.tw), "s"(a.ks), "s"(a.nbw), "s"(blockDim.x));
}
__device__ __forceinline__ void fetch_all(const PrepProb& a) {
  asm volatile("" ::"s"(a.src), "s"(a.rot), "s"(a.qa), "s"(a.qs), "s"(a.pa), "s"(a.lda), "s"(a.m),
               "s"(a.k), "s"(a.hsz), "s"(a.r0), "s"(a.r1), "s"(a.fwht_scale), "s"(a.nwg),
               "s"(a.preop), "s"(a.aux), "s"(a.pre), "s"(a.eps), "s"(blockDim.x));
}

enum { PREP_COPY = 0, PREP_RMSNORM = 1, PREP_GELU_MUL = 2 };

struct PrepBatch {
  PrepProb p[FGM_MAX_BATCH];
  int count;
};

// The calling thread's drop-in staging (fgm_api.hip): its stream, a device
// and a pinned host buffer of at least the given sizes; status as the C ABI.
int fgm_stage(size_t dev_bytes, size_t pin_bytes, void** dev, void** pin, hipStream_t* st);

// Every problem of a batch has the same preop; a preop needs k % 64 == 0 (no
// scalar tails).
hipError_t fgm_launch_prep(const PrepBatch& b, hipStream_t st);
hipError_t fgm_launch_pack_a(int M, int K, const int8_t* A, int8_t* Ap, hipStream_t st);
hipError_t fgm_launch_fwht(float* x, int n, int hsz, float scale, hipStream_t st);

// Skinny weight-stream path, M <= 64 (all problems of a batch share the
// weight type and are served by one launch).
bool fgm_decode_fits(int bits, int M, int K, int group);
size_t fgm_decode_lds_bytes(int bits, int M, int K, int group);
hipError_t fgm_launch_decode(int bits, const GemmBatch& b, hipStream_t st);

// Dense MFMA path (any M).
hipError_t fgm_launch_gemm(int bits, const GemmBatch& b, hipStream_t st);

// f32 elementwise primitives (fgm_elem.hip).  rows x n contiguous rows for
// rmsnorm (w NULL: no scale); gelu: up NULL for in-place gelu (out may be
// gate); rope: cs [rows][head_dim / 2][2] (cos, sin); binop: 0 add, 1 mul,
// 2 scale by s.
hipError_t fgm_launch_rmsnorm(float* out, const float* x, const float* w, int rows, int n, float eps,
                              hipStream_t st);
hipError_t fgm_launch_gelu(float* out, const float* gate, const float* up, int n, hipStream_t st);
hipError_t fgm_launch_softcap(float* x, int n, float cap, hipStream_t st);
hipError_t fgm_launch_rope(float* x, int rows, int n_heads, int head_dim, const float* cs, hipStream_t st);
hipError_t fgm_launch_binop(float* a, const float* b, int n, int op, float s, hipStream_t st);
// zeros into rows x cols floats with row stride ld (no memset node in a graph)
hipError_t fgm_launch_fill_zero(float* p, int ld, int rows, int cols, hipStream_t st);

// int8-KV attention (fgm_attn.hip).  Rows are grouped into sequences: rows
// [row0, row0 + nrows) of one sequence read one layer cache and sit at
// positions pos0, pos0 + 1, ...; a row at position p attends [st, p + 1) with
// st = window > 0 ? max(p + 1 - window, 0) : lo.  q and out are
// [m][n_heads][head_dim]; only heads [h0, h1) are computed and written.
constexpr int FGM_ATTN_MAX_SEQ = 16;
constexpr int FGM_ATTN_MAX_SPAN = 32768;  // positions per row (softmax row in LDS)
struct AttnSeq {
  const int8_t* kc;   // [k_len][kv_heads * head_dim]
  const float* ks;    // [k_len]
  const int8_t* vc;   // transposed, [ceil(k_len / 4)][kv_heads * head_dim][4]
  const float* vs;    // [k_len]
  int k_len, ring, pos0, lo, nrows, row0;
};
struct AttnArgs {
  AttnSeq seq[FGM_ATTN_MAX_SEQ];
  int nseq, m, nh, kvh, hd, window, h0, h1;
  float* out;
  const float* q;
  // scratch
  float* sc;          // scores / exponentials [m][nh][sc_stride]
  int sc_stride;
  int8_t* wpl;        // weight planes [m][kvh][wpl_blocks][3][grp][16]
  int wpl_blocks;
  int32_t* part;      // P.V partial sums [m][kvh][p3_chunks][grp][hd]
  float* wq;          // per (row, head) dequantisation step, 0 = zero output
  int p1_chunk;       // positions per score workgroup
  int p1_chunks;      // score workgroups per (row, kv head) in the grid
  int p3_spw;         // 64-slot steps per wave in a P.V workgroup
  int p3_chunks;      // P.V slot chunks (4 * p3_spw steps) per (row, kv head)
};
// A row's attended range and the reference's slot runs (ops.c:560-572) as
// four-slot-aligned spans [lo, hi); the P.V slot domain is
// [dom_lo, dom_lo + 64 dom_steps).  Shared by the host (grid sizing) and the
// kernels.
struct AttnSpan {
  int st, en, n, nrun, lo0, hi0, lo1, hi1, dom_lo, dom_steps;
};
__host__ __device__ inline AttnSpan attn_span(int en, int lo, int window, int ring) {
  AttnSpan g;
  g.en = en;
  g.st = window > 0 ? (en - window > 0 ? en - window : 0) : lo;
  g.n = g.en - g.st;
  g.lo1 = g.hi1 = 0;
  if (!ring) {
    g.lo0 = g.st, g.hi0 = g.en, g.nrun = 1;
  } else if (g.n >= ring) {
    g.lo0 = 0, g.hi0 = ring, g.nrun = 1;
  } else {
    const int s0 = g.st % ring;
    if (s0 + g.n <= ring) {
      g.lo0 = s0, g.hi0 = s0 + g.n, g.nrun = 1;
    } else {
      g.lo0 = s0, g.hi0 = ring, g.lo1 = 0, g.hi1 = s0 + g.n - ring, g.nrun = 2;
    }
  }
  g.lo0 &= ~3, g.hi0 = (g.hi0 + 3) & ~3;
  g.lo1 &= ~3, g.hi1 = (g.hi1 + 3) & ~3;
  g.dom_lo = (g.nrun == 2 ? 0 : g.lo0) & ~63;
  g.dom_steps = (g.hi0 - g.dom_lo + 63) >> 6;
  return g;
}
// P.V slot chunks per (row, kv head): enough workgroups to fill the chip
// (about 2048), at most 32.
inline int attn_pv_chunks(int m, int kvh, int hd) {
  const int per = (2048 + m * kvh * (hd / 64) - 1) / (m * kvh * (hd / 64));
  return per < 1 ? 1 : (per > 32 ? 32 : per);
}
// scratch layout for `m` rows whose spans (max over rows of end - start and
// of the ring size) are at most max_span; returns the bytes and fills the
// scratch pointers of `a` when base != nullptr.
size_t fgm_attn_layout(AttnArgs* a, void* base, int m, int nh, int kvh, int hd, int max_span);
hipError_t fgm_launch_attn(const AttnArgs& a, int max_n, hipStream_t st);
// V row scatter into the transposed cache (ops.c:653-657).
hipError_t fgm_launch_store_v_t(int8_t* vt, const int8_t* src, int n, int slot, hipStream_t st);
// Quantise m K and V rows (quant_act per row) into one cache at slots
// (pos0 + r) % ring (ring 0: pos0 + r): K in place, V transposed.
hipError_t fgm_launch_kv_store(const float* k, const float* v, int m, int row_len, int8_t* kc,
                               float* ks, int8_t* vt, float* vs, int pos0, int ring, hipStream_t st);
