/*
 * fgm_hip.h -- C ABI of the MI355X (gfx950) implementation of fastgemma's
 * fgm-kernels quantized-matmul path.  Library: fastgemma_amd/libfgm_hip.so.
 *
 * Two layers:
 *
 *  1. Drop-in entry points.  Same parameter lists, argument meaning and
 *     layouts as the reference's C symbols that the Rust crate binds in
 *     crates/fgm-kernels/src/lib.rs:13-80; the suffix follows the reference's
 *     `_vnni` convention (vnni_gemm.c:224,291).  All pointers are HOST
 *     pointers.  Weight (B) and weight-scale buffers are treated as immutable
 *     for the process lifetime -- they are the mmapped .fgm blobs
 *     (model.rs:120-141, forward.rs:264-291) -- and are uploaded to the GPU on
 *     first use and cached by host address.  A, scales and C move per call.
 *     Like the reference (void returns, panic = "abort"), a failed
 *     precondition or HIP call prints a message and aborts.
 *
 *  2. Device-resident API (fgm_hip_*).  Device pointers, an explicit HIP
 *     stream (passed as void*; NULL = the null stream), int status (0 = ok,
 *     otherwise an FGM_HIP_E* code with fgm_hip_last_error() describing it).
 *     Launches are asynchronous on the given stream.  This is the layer the
 *     benchmarks and a GPU-resident forward pass use.
 *
 * Layouts (unchanged from the .fgm file and the reference kernels):
 *   packed A  [ceil(M/16)][K/64][16][64] int8, rows >= M zero (ops.c:279-290)
 *   int8 B    [N/16][K/64] tiles of 1024 B, (K=64,N=16) as [k/4][n][k%4]
 *             (quant.py:96-107); b_scale f32 [N]
 *   int4 B    the int8 stream nibble-packed per 64-B block,
 *             packed[i] = q[i] & 15 | q[i+32] << 4 (quant.py:76-82), two's
 *             complement nibbles; b_scale f16 bits [K/group][N] (quant.py:165)
 *   C         f32 [M][ldc]; only rows < M and columns [16*n0, 16*n1) written.
 *
 * Preconditions (the reference asserts them in debug Rust only,
 * lib.rs:161-163,176-177,201-202,521; they are always checked here):
 *   K % 64 == 0, N % 16 == 0, 0 <= n0 <= n1 <= N/16, (n1 - n0) % 4 == 0,
 *   ldc >= 16*n1, q4g: group % 64 == 0 and K % group == 0,
 *   prep_rows: r0 % 16 == 0, k % 64 == 0, k <= 32768 (a row is staged in LDS);
 *   fwht: hsz a power of two, n % hsz == 0.
 */
#ifndef FGM_HIP_H
#define FGM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------ status codes */
#define FGM_HIP_OK 0
#define FGM_HIP_EINVAL 1   /* a precondition on shapes / pointers failed   */
#define FGM_HIP_EHIP 2     /* a HIP runtime call failed                     */
#define FGM_HIP_ENODEV 3   /* no usable gfx950 device                       */

/* ================================================================ drop-in */

/* replaces fgm_pack_a (lib.rs:19; ops.c:279-290) */
void fgm_pack_a_hip(int m, int k, const int8_t *a, int8_t *ap);

/* replaces fgm_prep_rows (lib.rs:20-23; ops.c:293-314) */
void fgm_prep_rows_hip(const float *src, int lda, float *rot, int8_t *qa, float *qs,
                       int8_t *pa, int m, int k, int hsz, int r0, int r1);

/* replaces fgm_gemm_q4g / fgm_gemm_q4g_vnni (lib.rs:24-28,36-40;
 * amx_gemm.c:333-372, vnni_gemm.c:291-322).  b_scale: f16 bits. */
void fgm_gemm_q4g_hip(int m, int n, int k, const int8_t *a, const float *a_scale,
                      const uint8_t *bq, const uint16_t *b_scale, int group, float *c,
                      int ldc, int n0, int n1);

/* replaces fgm_gemm_q8c / fgm_gemm_q8c_vnni (lib.rs:29-33,41-45;
 * amx_gemm.c:444-475, vnni_gemm.c:224-245) */
void fgm_gemm_q8c_hip(int m, int n, int k, const int8_t *a, const float *a_scale,
                      const int8_t *b, const float *b_scale, float *c, int ldc, int n0,
                      int n1);

/* replaces fgm_fwht (lib.rs:52; ops.c:153-175) */
void fgm_fwht_hip(float *x, int n, int hsz);

/* replaces fgm_quant_act (lib.rs:53; ops.c:181-204) */
void fgm_quant_act_hip(const float *x, int rows, int k, int8_t *q, float *scale);

/* replaces fgm_cpu_has_amx / fgm_cpu_has_avx512_vnni as the backend probe
 * (lib.rs:34-35,112-137): 1 when a gfx950 device is usable, else 0. */
int fgm_hip_available(void);

/* Drop the cached device copies of host weight buffers (for callers that
 * unmap or rewrite a weight file). */
void fgm_hip_weight_cache_clear(void);

/* Device bytes the weight cache holds: replaced = 0, the current copies;
 * replaced = 1, copies replaced after a buffer was rewritten at the same
 * address that a call still held at the last upload (freed at the next
 * one).  No counterpart in the reference: memory accounting for callers. */
size_t fgm_hip_weight_cache_bytes(int replaced);

/* ======================================================= device-resident */

/* Select and check the device (gfx950).  Optional: every entry point
 * initialises the current device on first use. */
int fgm_hip_init(int device);

/* Message for the last non-zero status returned on this thread. */
const char *fgm_hip_last_error(void);

int fgm_hip_gemm_q8c_dev(int m, int n, int k, const int8_t *a, const float *a_scale,
                         const int8_t *b, const float *b_scale, float *c, int ldc, int n0,
                         int n1, void *stream);

int fgm_hip_gemm_q4g_dev(int m, int n, int k, const int8_t *a, const float *a_scale,
                         const uint8_t *bq, const uint16_t *b_scale, int group, float *c,
                         int ldc, int n0, int n1, void *stream);

/* Raw int32 accumulators (no reference counterpart: the reference never
 * exposes them; this is the evidence for "int32 bit-exact").
 *   q8c: acc[m * ldacc + n]              = sum_k A[m][k] * B[k][n]
 *   q4g: acc[(g * M + m) * ldacc + n]    = sum_{k in group g} A[m][k] * B[k][n]
 * for m < M, n in [16*n0, 16*n1). */
int fgm_hip_acc_q8c_dev(int m, int n, int k, const int8_t *a, const int8_t *b, int32_t *acc,
                        int ldacc, int n0, int n1, void *stream);
int fgm_hip_acc_q4g_dev(int m, int n, int k, const int8_t *a, const uint8_t *bq, int group,
                        int32_t *acc, int ldacc, int n0, int n1, void *stream);

/* fgm_prep_rows on device buffers.  rot and qa may be NULL (not written);
 * the reference always writes them.  pa rows of r1's tile block that lie in
 * [r1, m) are copied from qa, which must then be non-NULL (ops.c:308-311). */
int fgm_hip_prep_rows_dev(const float *src, int lda, float *rot, int8_t *qa, float *qs,
                          int8_t *pa, int m, int k, int hsz, int r0, int r1, void *stream);

int fgm_hip_quant_act_dev(const float *x, int rows, int k, int8_t *q, float *scale,
                          void *stream);
int fgm_hip_pack_a_dev(int m, int k, const int8_t *a, int8_t *ap, void *stream);
int fgm_hip_fwht_dev(float *x, int n, int hsz, void *stream);

/* ----------------------------------------------- elementwise primitives
 * The forward pass's f32 operations that sit between the GEMMs (ops.c), so
 * that activations stay on the GPU.  Results equal the reference's bytes
 * (same operations in the same order), except the scalar tails of gelu and
 * softcap when n % 16 != 0 (libm tanhf on the CPU, the device tanhf here;
 * within a few ulp; no model dimension has such a tail). */

/* drop-ins, host pointers, same parameters as the reference's symbols */
void fgm_rmsnorm_hip(float *out, const float *x, const float *w, int n, float eps); /* lib.rs:47, ops.c:59-74 */
void fgm_rmsnorm_noscale_hip(float *out, const float *x, int n, float eps);        /* lib.rs:48, ops.c:77-91 */
void fgm_gelu_mul_hip(float *out, const float *gate, const float *up, int n);       /* lib.rs:49, ops.c:119-128 */
void fgm_gelu_hip(float *x, int n);                                                 /* lib.rs:50, ops.c:109-116 */
void fgm_rope_hip(float *x, int n_heads, int head_dim, const float *inv_freq, int pos); /* lib.rs:51, ops.c:135-147 */
void fgm_add_hip(float *a, const float *b, int n);                                  /* lib.rs:56, ops.c:317-322 */
void fgm_mul_hip(float *a, const float *b, int n);                                  /* lib.rs:57, ops.c:324-329 */
void fgm_scale_hip(float *a, float s, int n);                                       /* lib.rs:58, ops.c:331-337 */
void fgm_softcap_hip(float *x, int n, float cap);                                   /* lib.rs:59, ops.c:340-351 */

/* device API: rmsnorm of `rows` contiguous rows of n floats each (w NULL:
 * no scale, fgm_rmsnorm_noscale); gelu_mul with up NULL is gelu (out may be
 * gate); rope on x [rows][n_heads][head_dim] with cs [rows][head_dim/2][2] =
 * (cos, sin) pairs from fgm_hip_rope_table (host, the host's libm, as
 * ops.c:138-139); add / mul / scale in place on a. */
int fgm_hip_rmsnorm_dev(float *out, const float *x, const float *w, int rows, int n, float eps,
                        void *stream);
int fgm_hip_gelu_mul_dev(float *out, const float *gate, const float *up, int n, void *stream);
int fgm_hip_softcap_dev(float *x, int n, float cap, void *stream);
void fgm_hip_rope_table(float *cs, const float *inv_freq, int head_dim, int pos);
int fgm_hip_rope_dev(float *x, int rows, int n_heads, int head_dim, const float *cs, void *stream);
int fgm_hip_add_dev(float *a, const float *b, int n, void *stream);
int fgm_hip_mul_dev(float *a, const float *b, int n, void *stream);
int fgm_hip_scale_dev(float *a, float s, int n, void *stream);

/* ------------------------------------------------------ int8-KV attention
 * The forward pass's attention over the int8 KV cache (ops.c:353-877,
 * kv.rs).  Cache layout per layer (kv.rs:13-50): K [k_len][kv_heads *
 * head_dim] int8 with one f32 scale per slot; V transposed in groups of four
 * slots, vt[((slot/4) * kvd + j) * 4 + slot%4], with one scale per slot;
 * slot = ring ? pos % ring : pos.  q and out are [rows][n_heads][head_dim] f32.
 * Results equal the reference's bytes; the only operation evaluated
 * differently is exp on the n % 16 tail of the softmax (libm expf there,
 * correctly rounded here; they differ where glibc's expf is not correctly
 * rounded).  Limits: head_dim a multiple of 64 up to 512, at most 16 query
 * heads per kv head, at most 32768 positions per row, a ring range no longer
 * than the ring (the reference's scratch layout assumes it too). */

/* drop-ins, host pointers, same parameters as the reference's symbols; the
 * caches are uploaded per call, `scratch` is not touched */
void fgm_attend_q8_hip(float *out, const float *q, const int8_t *kc, const float *ks,
                       const int8_t *vc, const float *vs, int n_heads, int kv_heads, int head_dim,
                       int start, int end, float *scratch);               /* lib.rs:60-64, ops.c:363-368 */
void fgm_attend_q8_heads_hip(float *out, const float *q, const int8_t *kc, const float *ks,
                             const int8_t *vc, const float *vs, int n_heads, int kv_heads,
                             int head_dim, int start, int end, float *scratch, int h0, int h1,
                             int ring, int cap);                           /* lib.rs:65-70, ops.c:378-637 */
void fgm_attend_q8_row_hip(float *out, const float *q, const int8_t *kc, const float *ks,
                           const int8_t *vc, const float *vs, int n_heads, int kv_heads,
                           int head_dim, int start, int end, float *scratch, int ring,
                           int cap);                                       /* lib.rs:73-78, ops.c:729-872 */
void fgm_store_v_t_hip(int8_t *vt, const int8_t *src, int n, int slot);  /* lib.rs:71, ops.c:653-657 */
void fgm_set_scalar_wfill_hip(int on);                                  /* lib.rs:72, ops.c:53-54 (no effect there either) */
int fgm_rowbatch_scratch_hip(int n_heads, int cap, int head_dim);       /* lib.rs:79, ops.c:875-877 */

/* device API.  One call covers the rows of up to 16 sequences (the
 * reference's AttnJob, pool.rs:36-65): sequence i owns the next `rows` rows
 * of q / out, at positions pos, pos + 1, ..., and reads one layer cache of
 * k_len slots (ring: ring-buffer capacity, 0 = linear).  A row at position p
 * attends [max(p + 1 - window, 0), p + 1) (window 0: [0, p + 1)), all heads,
 * kv head h / (n_heads / kv_heads).  `scratch`: device memory, 256-byte
 * aligned, at least fgm_hip_attend_scratch_bytes(total rows, ..., max_span)
 * where max_span bounds every row's range length and every ring size.  The
 * scratch is used during the call only (calls on one scratch buffer must not
 * overlap). */
typedef struct fgm_hip_attn_seq {
  const int8_t *kc;
  const float *ks;
  const int8_t *vc;
  const float *vs;
  int k_len;
  int ring;
  int pos;
  int rows;
} fgm_hip_attn_seq;

size_t fgm_hip_attend_scratch_bytes(int rows, int n_heads, int kv_heads, int head_dim, int max_span);
int fgm_hip_attend_dev(float *out, const float *q, const fgm_hip_attn_seq *seqs, int nseq,
                       int n_heads, int kv_heads, int head_dim, int window, void *scratch,
                       size_t scratch_bytes, void *stream);
/* fgm_attend_q8_heads on device pointers: one row, range [start, end), heads
 * [h0, h1) (the others are not written) */
int fgm_hip_attend_heads_dev(float *out, const float *q, const int8_t *kc, const float *ks,
                             const int8_t *vc, const float *vs, int n_heads, int kv_heads,
                             int head_dim, int start, int end, int h0, int h1, int ring, int cap,
                             void *scratch, size_t scratch_bytes, void *stream);
int fgm_hip_store_v_t_dev(int8_t *vt, const int8_t *src, int n, int slot, void *stream);
/* The forward pass's cache append (forward.rs:515-548): rows r < m of k and v
 * (f32 [m][row_len]) quantised as fgm_quant_act does, K to kc[slot], V to vt
 * transposed, scales to ks / vs, slot = ring ? (pos + r) % ring : pos + r;
 * cap: slots the cache holds (checked). */
int fgm_hip_kv_store_dev(const float *k, const float *v, int m, int row_len, int8_t *kc, float *ks,
                         int8_t *vt, float *vs, int cap, int pos, int ring, void *stream);

/* ------------------------------------------------------------- the model
 * A .fgm file (convert/fgm.py:1-16; model.rs:1-220) opened on the GPU: the file
 * is mapped read-only and, with device_resident, its tensor body is copied to
 * HBM once, so GEMMs read weights with no host traffic.  Tensor pointers stay
 * valid until fgm_hip_model_close.  NULL / non-zero status on error, with
 * fgm_hip_last_error() describing it. */
typedef struct fgm_hip_model fgm_hip_model;

typedef struct fgm_hip_tensor {
  char dtype[16];          /* q4g, q8c, q8r, q4r, f32, f16, ... */
  int ndim;
  int64_t shape[4];
  size_t offset, nbytes;   /* in the file */
  const void *host;        /* in the mapping */
  const void *dev;         /* in HBM, NULL unless resident */
  int hadamard;            /* meta.hadamard, 0 when absent */
  int group;               /* meta.group, -1 when absent */
} fgm_hip_tensor;

/* A quantised linear weight (model.rs:104-117, QLinear): bits 4 (q4g: b packed
 * int4, b_scale f16 [k/group][n]) or 8 (q8c: b int8 tiles, b_scale f32 [n]). */
typedef struct fgm_hip_linear {
  int bits, n, k, group, hadamard;
  const void *b, *b_scale;            /* device (NULL unless resident) */
  const void *b_host, *b_scale_host;  /* in the mapping */
} fgm_hip_linear;

fgm_hip_model *fgm_hip_model_open(const char *path, int device_resident);  /* Model::open, model.rs:120-128 */
void fgm_hip_model_close(fgm_hip_model *m);
int fgm_hip_model_has(const fgm_hip_model *m, const char *name);           /* model.rs:130-132 */
const char *fgm_hip_model_config(const fgm_hip_model *m);                  /* header "config", compact JSON */
const char *fgm_hip_model_meta(const fgm_hip_model *m);                    /* header "meta" */
size_t fgm_hip_model_total_bytes(const fgm_hip_model *m);                  /* model.rs:209-211 */
int fgm_hip_model_tensor_count(const fgm_hip_model *m);
const char *fgm_hip_model_tensor_name(const fgm_hip_model *m, int i);      /* sorted by name */
int fgm_hip_model_tensor(const fgm_hip_model *m, const char *name, fgm_hip_tensor *out);
int fgm_hip_model_linear(const fgm_hip_model *m, const char *name, fgm_hip_linear *out); /* model.rs:167-192 */

/* The int4 / int8 weight choice (forward.rs:26-89).  FGM_WEIGHTS = int4 -> LO,
 * int8 -> HI, auto:M -> ABOVE M (M not a number: 16), anything else or unset
 * -> ABOVE 16.  fgm_hip_model_dual resolves <name> or its int8 twin
 * <name>.i8 (model.rs:194-201, DualW::pick): the twin when it exists and sel
 * is HI, or ABOVE with rows >= threshold. */
#define FGM_HIP_SEL_LO 0
#define FGM_HIP_SEL_HI 1
#define FGM_HIP_SEL_ABOVE 2
int fgm_hip_weight_sel(const char *value, int *threshold);
int fgm_hip_model_dual(const fgm_hip_model *m, const char *name, int rows, int sel, int threshold,
                       fgm_hip_linear *out);

/* Embedding / PLE gathers (model.rs:203-213; ops.c:208-251): out[r][0..k) =
 * row rows[r] of a q8r (int8, f32 scale per row) or q4r (int4 half-split
 * nibbles, f16 scale per 64) table; exact products. */
void fgm_gather_q8r_hip(float *out, const int8_t *tbl, const float *sc, int row, int k); /* lib.rs:54, ops.c:208-217 */
void fgm_gather_q4r_hip(float *out, const uint8_t *tbl, const uint16_t *sc, int row, int k); /* lib.rs:55, ops.c:228-251 */
int fgm_hip_gather_dev(int bits, const void *tbl, const void *sc, const int *rows, int count, int k,
                       float *out, void *stream);
int fgm_hip_model_gather_dev(const fgm_hip_model *m, const char *name, const int *rows, int count,
                             float *out, void *stream);

/* The thread pool's jobs on the HIP backend (pool.rs:19-79, 285-310): one
 * launch covers all of N (GEMM) or all tile blocks (prep) instead of a split
 * over host threads.  Device pointers. */
typedef struct fgm_hip_gemm_job {
  int m, n, kdim;
  const int8_t *a;
  const float *a_scale;
  const uint8_t *bq;
  const int8_t *b8;
  const uint16_t *s4;
  const float *s8;
  int bits, group;
  float *c;
  int ldc;
} fgm_hip_gemm_job;
typedef struct fgm_hip_prep_job {
  const float *src;
  int lda;
  float *rot;
  int8_t *qa;
  float *qs;
  int8_t *pa;
  int m, k, hsz;
} fgm_hip_prep_job;
int fgm_hip_pool_gemm_dev(const fgm_hip_gemm_job *job, void *stream);
int fgm_hip_pool_prep_dev(const fgm_hip_prep_job *job, void *stream);

/* Gemm::run (forward.rs:140-158): out[m][0..n) = w . a[m][0..k) -- FWHT of
 * w.hadamard, per-row quantisation and tile packing into `scratch` (at least
 * fgm_hip_linear_scratch_bytes(m, k) bytes), then the GEMM. */
size_t fgm_hip_linear_scratch_bytes(int m, int k);
int fgm_hip_linear_run_dev(const fgm_hip_linear *w, const float *a, int m, int lda, float *out,
                           void *scratch, size_t scratch_bytes, void *stream);

/* fgm_hip_linear_run_dev without a scratch argument and with no allocation:
 * the scratch lives in a file-scope device array of
 * fgm_hip_linear_noalloc_max_bytes() bytes (8 MiB) per GPU, held until the
 * process ends.  No counterpart in the reference: it is for callers that
 * cannot allocate (code under HIP graph capture, serving loops).  Shapes
 * whose fgm_hip_linear_scratch_bytes(m, k) exceeds the limit are refused with
 * FGM_HIP_EINVAL.  All calls on one GPU share the array: calls that overlap on
 * one GPU (several streams, concurrent graphs) race. */
size_t fgm_hip_linear_noalloc_max_bytes(void);
int fgm_hip_linear_run_noalloc_dev(const fgm_hip_linear *w, const float *a, int m, int lda, float *out,
                                   void *stream);

/* Which kernel family a GEMM of m rows runs on: 0 = skinny weight-stream
 * kernel, 1 = dense MFMA kernel. */
int fgm_hip_gemm_path(int bits, int m, int k, int group);

/* Dry run of one GEMM's dispatch, host only (no device is touched, no
 * operand is read): validates the shape as fgm_hip_gemm_q8c_dev /
 * fgm_hip_gemm_q4g_dev do and stores in *launches how many kernel launch
 * calls the library would make for it (weights past 1 GiB are cut along N
 * into several).  No counterpart in the reference: a planning query for
 * tests and for callers that size graphs. */
int fgm_hip_gemm_plan(int bits, int m, int n, int k, int group, int n0, int n1, int *launches);

/* ------------------------------------------------------------ batched calls
 * No single reference counterpart: one call for the GEMMs a forward pass
 * issues back to back on the same activation (q/k/v, gate/up: forward.rs:
 * 484,499-500,619-622) or on independent ones.  Up to four GEMMs of one
 * weight type share a launch; the results equal the one-at-a-time calls
 * byte for byte.  The descriptors are read during the call only. */
typedef struct fgm_hip_gemm_desc {
  int bits;               /* 8: q8c (b int8 tiles, b_scale f32 [n]);
                             4: q4g (b packed int4, b_scale f16 bits [k/group][n]) */
  int m, n, k, group;     /* group: q4g only */
  const int8_t *a;        /* packed A (device) */
  const float *a_scale;
  const void *b;
  const void *b_scale;
  float *c;
  int ldc, n0, n1;
} fgm_hip_gemm_desc;

int fgm_hip_gemm_batch_dev(const fgm_hip_gemm_desc *descs, int count, void *stream);

/* fgm_prep_rows for several activations in one launch. */
typedef struct fgm_hip_prep_desc {
  const float *src;
  int lda;
  float *rot;             /* may be NULL */
  int8_t *qa;             /* may be NULL unless rows of r1's tile block lie in [r1, m) */
  float *qs;
  int8_t *pa;
  int m, k, hsz, r0, r1;
} fgm_hip_prep_desc;

int fgm_hip_prep_batch_dev(const fgm_hip_prep_desc *descs, int count, void *stream);

/* A GEMM input's producer fused into fgm_prep_rows over rows [0, m): the
 * result is byte-identical to the producer followed by
 * fgm_hip_prep_rows_dev(xn_or_act, k, rot, qa, qs, pa, m, k, hsz, 0, m).
 * Same constraints as prep_rows (k % 64 == 0, k <= 32768); xn / act, rot and
 * qa may be NULL; rows of the last tile block past m are zero in pa.
 *   rmsnorm:  fgm_rmsnorm / fgm_rmsnorm_noscale (w NULL) of each row of x
 *             (row stride lda), as the forward pass does before the q/k/v
 *             and gate/up GEMMs (forward.rs:477-481, 614-618; ops.c:59-91);
 *   gelu_mul: gelu(gate) * up (both row stride lda), before the down GEMM
 *             (forward.rs:621-622; ops.c:119-128). */
int fgm_hip_prep_rmsnorm_dev(const float *x, int lda, const float *w, float eps, float *xn,
                             float *rot, int8_t *qa, float *qs, int8_t *pa, int m, int k,
                             int hsz, void *stream);
int fgm_hip_prep_gelu_mul_dev(const float *gate, const float *up, int lda, float *act,
                              float *rot, int8_t *qa, float *qs, int8_t *pa, int m, int k,
                              int hsz, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* FGM_HIP_H */
