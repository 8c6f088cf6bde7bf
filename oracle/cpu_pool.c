/*
 * cpu_pool.c -- TEST / BENCH INFRASTRUCTURE ONLY (the CPU-baseline leg).
 *
 * A persistent pthread barrier pool that drives a CPU GEMM entry point with
 * fastgemma's own work split, so the CPU figure bench.py reports next to the
 * GPU figure is the reference's threading, not a made-up one:
 *
 *   GEMM : the N/16 n-blocks are grouped in fours and the groups are split
 *          evenly over the threads (crates/fgm-core/src/pool.rs:110-124,
 *          split_n / split_gemm); every thread calls the kernel on its own
 *          [n0, n1) n-block range (pool.rs:126-145).
 *   prep : 16-row tile blocks split evenly (pool.rs:206-225, 264-265); below
 *          two blocks per thread it runs on the caller (pool.rs:302-305).
 *
 * The pool is modelled on the harness in bench/kernels/gemm_bench.c:28-77
 * (persistent workers, one barrier to start, one to finish).  The kernel is
 * passed in as a function pointer, so the same pool drives the reference's
 * own C (oracle/_ref) or the oracle restatement.
 */
#define _GNU_SOURCE
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

typedef void (*q8c_fn)(int, int, int, const int8_t *, const float *, const int8_t *,
                       const float *, float *, int, int, int);
typedef void (*q4g_fn)(int, int, int, const int8_t *, const float *, const uint8_t *,
                       const uint16_t *, int, float *, int, int, int);
typedef void (*prep_fn)(const float *, int, float *, int8_t *, float *, int8_t *, int, int,
                        int, int, int);

typedef struct {
  int kind; /* 0 = q8c, 1 = q4g, 2 = prep */
  void *fn;
  int M, N, K, group, ldc, hsz, lda;
  const int8_t *A;
  const float *as;
  const void *B;
  const void *bs;
  float *C;
  const float *src;
  float *rot;
  int8_t *qa;
  float *qs;
  int8_t *pa;
} job_t;

static int g_nt = 0;
static pthread_t g_th[256];
static pthread_barrier_t g_start, g_done;
static job_t g_job;
static volatile int g_quit = 0;

static void split_n(int total, int nt, int tid, int *a, int *b) {
  int per = total / nt, extra = total % nt;
  int start = tid * per + (tid < extra ? tid : extra);
  *a = start;
  *b = start + per + (tid < extra ? 1 : 0);
}

static void run_slice(const job_t *j, int tid, int nt) {
  if (j->kind == 2) {
    int blocks = (j->M + 15) / 16, b0, b1;
    split_n(blocks, nt, tid, &b0, &b1);
    int r0 = b0 * 16, r1 = b1 * 16 < j->M ? b1 * 16 : j->M;
    if (r0 < r1)
      ((prep_fn)j->fn)(j->src, j->lda, j->rot, j->qa, j->qs, j->pa, j->M, j->K, j->hsz, r0, r1);
    return;
  }
  int g0, g1;
  split_n(j->N / 16 / 4, nt, tid, &g0, &g1);
  int n0 = g0 * 4, n1 = g1 * 4;
  if (n0 >= n1) return;
  if (j->kind == 0)
    ((q8c_fn)j->fn)(j->M, j->N, j->K, j->A, j->as, (const int8_t *)j->B, (const float *)j->bs,
                    j->C, j->ldc, n0, n1);
  else
    ((q4g_fn)j->fn)(j->M, j->N, j->K, j->A, j->as, (const uint8_t *)j->B,
                    (const uint16_t *)j->bs, j->group, j->C, j->ldc, n0, n1);
}

static void *worker(void *arg) {
  int tid = (int)(intptr_t)arg;
  for (;;) {
    pthread_barrier_wait(&g_start);
    if (g_quit) break;
    run_slice(&g_job, tid, g_nt);
    pthread_barrier_wait(&g_done);
  }
  return NULL;
}

/* Start nt - 1 workers (the caller is thread 0).  Returns nt. */
int orc_pool_start(int nt) {
  if (g_nt) return g_nt;
  if (nt < 1) nt = 1;
  if (nt > 256) nt = 256;
  g_nt = nt;
  g_quit = 0;
  pthread_barrier_init(&g_start, NULL, (unsigned)nt);
  pthread_barrier_init(&g_done, NULL, (unsigned)nt);
  for (int t = 1; t < nt; t++) pthread_create(&g_th[t], NULL, worker, (void *)(intptr_t)t);
  return nt;
}

void orc_pool_stop(void) {
  if (!g_nt) return;
  g_quit = 1;
  pthread_barrier_wait(&g_start);
  for (int t = 1; t < g_nt; t++) pthread_join(g_th[t], NULL);
  pthread_barrier_destroy(&g_start);
  pthread_barrier_destroy(&g_done);
  g_nt = 0;
}

static void run_job(const job_t *j) {
  if (j->kind == 2 && (j->M + 15) / 16 < 2 * g_nt) { /* pool.rs:302-305: inline */
    ((prep_fn)j->fn)(j->src, j->lda, j->rot, j->qa, j->qs, j->pa, j->M, j->K, j->hsz, 0, j->M);
    return;
  }
  g_job = *j;
  if (g_nt == 1) {
    run_slice(j, 0, 1);
    return;
  }
  pthread_barrier_wait(&g_start);
  run_slice(j, 0, g_nt);
  pthread_barrier_wait(&g_done);
}

static double now_s(void) {
  struct timespec t;
  clock_gettime(CLOCK_MONOTONIC, &t);
  return t.tv_sec + 1e-9 * t.tv_nsec;
}

/* Run the q8c kernel `reps` times over the pool; per-rep seconds in times[]. */
void orc_pool_q8c(void *fn, int M, int N, int K, const int8_t *A, const float *as,
                  const int8_t *B, const float *bs, float *C, int ldc, int reps, double *times) {
  job_t j;
  memset(&j, 0, sizeof j);
  j.kind = 0; j.fn = fn; j.M = M; j.N = N; j.K = K; j.A = A; j.as = as; j.B = B; j.bs = bs;
  j.C = C; j.ldc = ldc;
  for (int r = 0; r < reps; r++) {
    double t0 = now_s();
    run_job(&j);
    times[r] = now_s() - t0;
  }
}

void orc_pool_q4g(void *fn, int M, int N, int K, const int8_t *A, const float *as,
                  const uint8_t *B, const uint16_t *bs, int group, float *C, int ldc, int reps,
                  double *times) {
  job_t j;
  memset(&j, 0, sizeof j);
  j.kind = 1; j.fn = fn; j.M = M; j.N = N; j.K = K; j.A = A; j.as = as; j.B = B; j.bs = bs;
  j.group = group; j.C = C; j.ldc = ldc;
  for (int r = 0; r < reps; r++) {
    double t0 = now_s();
    run_job(&j);
    times[r] = now_s() - t0;
  }
}

void orc_pool_prep(void *fn, const float *src, int lda, float *rot, int8_t *qa, float *qs,
                   int8_t *pa, int M, int K, int hsz, int reps, double *times) {
  job_t j;
  memset(&j, 0, sizeof j);
  j.kind = 2; j.fn = fn; j.src = src; j.lda = lda; j.rot = rot; j.qa = qa; j.qs = qs;
  j.pa = pa; j.M = M; j.K = K; j.hsz = hsz;
  for (int r = 0; r < reps; r++) {
    double t0 = now_s();
    run_job(&j);
    times[r] = now_s() - t0;
  }
}
