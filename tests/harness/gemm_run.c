/*
 * gemm_run.c -- TEST INFRASTRUCTURE: drives libfgm_hip.so the way fgm-core
 * drives the reference kernels, from C, with no Python and no torch (so the
 * library runs on the system HIP runtime a Rust binary would link).
 *
 * Gemm::run (crates/fgm-core/src/forward.rs:140-158) through the drop-in C ABI
 * with host pointers:
 *   prep  fgm_prep_rows_hip over 16-row tile blocks split across the threads
 *         (pool.rs:206-225, 264-265; below two blocks per thread the caller
 *         runs it alone, pool.rs:302-305);
 *   GEMM  fgm_gemm_q4g_hip / fgm_gemm_q8c_hip called concurrently from T host
 *         threads, each on its own [n0, n1) n-block range: the n-blocks are
 *         grouped in fours and the groups split evenly (pool.rs:110-145).
 * Every output byte (qa, qs, pa of the prep; C of the GEMM) is compared with
 * the CPU oracle (oracle/liboracle.so) run single-threaded over the whole
 * range.  Then the BASELINE configs[1] step (prep + up GEMM, prep + down
 * GEMM, int4 group 64, M = 8) is timed through the same drop-ins.
 *
 *   gemm_run [threads]      exit status 0 when every case matches
 */
#define _GNU_SOURCE
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "fgm_hip.h"

/* the oracle (oracle/fgm_oracle.c) */
size_t orc_packed_a_len(int m, int k);
void orc_prep_rows(const float *src, int lda, float *rot, int8_t *qa, float *qs, int8_t *pa, int m,
                   int k, int hsz, int r0, int r1);
void orc_gemm_q8c(int M, int N, int K, const int8_t *Ap, const float *a_scale, const int8_t *B,
                  const float *b_scale, float *C, int ldc, int n0, int n1);
void orc_gemm_q4g(int M, int N, int K, const int8_t *Ap, const float *a_scale, const uint8_t *Bq,
                  const uint16_t *b_scale, int group, float *C, int ldc, int n0, int n1);
void orc_gen_i8(uint64_t seed, size_t n, int lo, int hi, int8_t *out);
void orc_gen_u8(uint64_t seed, size_t n, uint8_t *out);
void orc_gen_uniform(uint64_t seed, size_t n, float lo, float hi, float *out);
void orc_gen_normal(uint64_t seed, size_t n, float *out);
uint16_t orc_f32_to_f16(float f);

typedef struct {
  int bits, m, n, k, group, hsz;
  const float *x;
  const void *b, *bs;
  /* prep outputs, shared by all threads (disjoint rows) */
  float *rot, *qs;
  int8_t *qa, *pa;
  float *c;
  int ldc;
} Job;

typedef struct {
  const Job *j;
  int t, nt, phase; /* phase 0: prep, 1: GEMM */
} Arg;

/* pool.rs:110-124: n-blocks in groups of four, the groups split evenly */
static void split_n(int nblocks, int t, int nt, int *n0, int *n1) {
  const int groups = nblocks / 4, per = groups / nt, rem = groups % nt;
  const int g0 = t * per + (t < rem ? t : rem), g1 = g0 + per + (t < rem ? 1 : 0);
  *n0 = 4 * g0;
  *n1 = 4 * g1;
}

static void *worker(void *p) {
  const Arg *a = (const Arg *)p;
  const Job *j = a->j;
  if (a->phase == 0) {
    /* 16-row tile blocks split evenly */
    const int blocks = (j->m + 15) / 16, per = blocks / a->nt, rem = blocks % a->nt;
    const int b0 = a->t * per + (a->t < rem ? a->t : rem), b1 = b0 + per + (a->t < rem ? 1 : 0);
    const int r0 = 16 * b0, r1 = 16 * b1 < j->m ? 16 * b1 : j->m;
    if (r0 < r1)
      fgm_prep_rows_hip(j->x, j->k, j->rot, j->qa, j->qs, j->pa, j->m, j->k, j->hsz, r0, r1);
  } else {
    int n0, n1;
    split_n(j->n / 16, a->t, a->nt, &n0, &n1);
    if (n0 < n1) {
      if (j->bits == 4)
        fgm_gemm_q4g_hip(j->m, j->n, j->k, j->pa, j->qs, (const uint8_t *)j->b, (const uint16_t *)j->bs,
                         j->group, j->c, j->ldc, n0, n1);
      else
        fgm_gemm_q8c_hip(j->m, j->n, j->k, j->pa, j->qs, (const int8_t *)j->b, (const float *)j->bs, j->c,
                         j->ldc, n0, n1);
    }
  }
  return NULL;
}

/* A persistent pool, as fgm-core's (pool.rs) and the reference's bench
 * harness (bench/kernels/gemm_bench.c:28-77) keep one: workers wait on a
 * start barrier, run their share of the posted phase, meet at a done
 * barrier. */
static struct {
  int nt, quit;
  Arg args[64];
  pthread_t th[64];
  pthread_barrier_t start, done;
} pool;

static void *pool_main(void *p) {
  const int t = (int)(intptr_t)p;
  for (;;) {
    pthread_barrier_wait(&pool.start);
    if (pool.quit) return NULL;
    worker(&pool.args[t]);
    pthread_barrier_wait(&pool.done);
  }
}

static void pool_open(int nt) {
  pool.nt = nt;
  pool.quit = 0;
  pthread_barrier_init(&pool.start, NULL, nt + 1);
  pthread_barrier_init(&pool.done, NULL, nt + 1);
  for (int t = 0; t < nt; t++) pthread_create(&pool.th[t], NULL, pool_main, (void *)(intptr_t)t);
}

static void pool_close(void) {
  pool.quit = 1;
  pthread_barrier_wait(&pool.start);
  for (int t = 0; t < pool.nt; t++) pthread_join(pool.th[t], NULL);
  pthread_barrier_destroy(&pool.start);
  pthread_barrier_destroy(&pool.done);
}

/* Gemm::run on the pool's threads: the prep (on the caller below two tile
 * blocks per thread), then the GEMM; nt = 1 runs both on the caller */
static void gemm_run(const Job *j, int nt) {
  const int blocks = (j->m + 15) / 16;
  for (int phase = 0; phase < 2; phase++) {
    if (nt == 1 || (phase == 0 && blocks < 2 * nt)) {
      Arg a = {j, 0, 1, phase};
      worker(&a);
      continue;
    }
    for (int t = 0; t < nt; t++) pool.args[t] = (Arg){j, t, nt, phase};
    pthread_barrier_wait(&pool.start);
    pthread_barrier_wait(&pool.done);
  }
}

static double now_us(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return ts.tv_sec * 1e6 + ts.tv_nsec * 1e-3;
}

typedef struct {
  Job j;
  void *bufs[16];
  int nb;
} Case;

static void *keep(Case *c, size_t bytes) {
  void *p = calloc(1, bytes ? bytes : 1);
  c->bufs[c->nb++] = p;
  return p;
}

static void make_case(Case *c, int bits, int m, int n, int k, int group, int hsz, uint64_t seed) {
  memset(c, 0, sizeof *c);
  Job *j = &c->j;
  j->bits = bits, j->m = m, j->n = n, j->k = k, j->group = group, j->hsz = hsz, j->ldc = n;
  float *x = keep(c, (size_t)m * k * 4);
  orc_gen_normal(seed, (size_t)m * k, x);
  j->x = x;
  if (bits == 8) {
    int8_t *b = keep(c, (size_t)n * k);
    float *bs = keep(c, (size_t)n * 4);
    orc_gen_i8(seed + 1, (size_t)n * k, -127, 127, b);
    orc_gen_uniform(seed + 2, (size_t)n, 1e-3f, 1e-2f, bs);
    j->b = b, j->bs = bs;
  } else {
    uint8_t *b = keep(c, (size_t)n * k / 2);
    const size_t ns = (size_t)(k / group) * n;
    float *f = malloc(ns * 4);
    uint16_t *bs = keep(c, ns * 2);
    orc_gen_u8(seed + 1, (size_t)n * k / 2, b);
    orc_gen_uniform(seed + 2, ns, 5e-3f, 5e-2f, f);
    for (size_t i = 0; i < ns; i++) bs[i] = orc_f32_to_f16(f[i]);
    free(f);
    j->b = b, j->bs = bs;
  }
  j->rot = keep(c, (size_t)m * k * 4);
  j->qa = keep(c, (size_t)m * k);
  j->qs = keep(c, (size_t)m * 4);
  j->pa = keep(c, orc_packed_a_len(m, k));
  j->c = keep(c, (size_t)m * n * 4);
}

static void free_case(Case *c) {
  for (int i = 0; i < c->nb; i++) free(c->bufs[i]);
}

/* the whole Gemm::run through the oracle, single-threaded */
static int check_case(Case *c, int nt) {
  const Job *j = &c->j;
  const int m = j->m, n = j->n, k = j->k;
  const size_t plen = orc_packed_a_len(m, k);
  float *rot = calloc((size_t)m * k, 4), *qs = calloc(m, 4), *cc = calloc((size_t)m * n, 4);
  int8_t *qa = calloc((size_t)m * k, 1), *pa = calloc(plen, 1);
  orc_prep_rows(j->x, k, rot, qa, qs, pa, m, k, j->hsz, 0, m);
  if (j->bits == 4)
    orc_gemm_q4g(m, n, k, pa, qs, j->b, j->bs, j->group, cc, n, 0, n / 16);
  else
    orc_gemm_q8c(m, n, k, pa, qs, j->b, j->bs, cc, n, 0, n / 16);
  gemm_run(j, nt);
  int ok = memcmp(qa, j->qa, (size_t)m * k) == 0 && memcmp(qs, j->qs, (size_t)m * 4) == 0 &&
           memcmp(pa, j->pa, plen) == 0 && memcmp(cc, j->c, (size_t)m * n * 4) == 0;
  if (j->hsz > 0) ok = ok && memcmp(rot, j->rot, (size_t)m * k * 4) == 0;
  size_t bad = 0;
  for (size_t i = 0; i < (size_t)m * n; i++) bad += memcmp(&cc[i], &j->c[i], 4) != 0;
  printf("case bits=%d m=%d n=%d k=%d group=%d hsz=%d threads=%d: %s (%zu C words differ)\n", j->bits, m, n,
         k, j->group, j->hsz, nt, ok ? "ok" : "MISMATCH", bad);
  fflush(stdout);
  free(rot), free(qs), free(cc), free(qa), free(pa);
  return ok;
}

static int cmp_d(const void *a, const void *b) {
  const double x = *(const double *)a, y = *(const double *)b;
  return x < y ? -1 : x > y;
}

int main(int argc, char **argv) {
  const int nt = argc > 1 ? atoi(argv[1]) : 8;
  if (nt < 1 || nt > 64) return 2;
  if (!fgm_hip_available()) {
    fprintf(stderr, "no gfx950 device: %s\n", fgm_hip_last_error());
    return 2;
  }
  pool_open(nt);
  int all = 1;
  /* (bits, m, n, k, group, hsz): BASELINE configs[1] up / down, configs[0],
   * a Hadamard-rotated linear, prefill chunks of three tile blocks (prep on
   * the caller) and of sixteen (prep split over the threads) */
  const int cases[][6] = {{4, 8, 8192, 2048, 64, 0},   {4, 8, 2048, 8192, 64, 0},     {8, 1, 8192, 2048, 0, 0},
                          {4, 8, 2048, 2048, 64, 128}, {8, 40, 1024, 2048, 0, 0},     {4, 37, 512, 1024, 128, 128},
                          {8, 256, 1024, 2048, 0, 0},  {4, 256, 2048, 2048, 64, 128}};
  const int thread_counts[] = {1, nt};
  for (size_t i = 0; i < sizeof cases / sizeof cases[0]; i++)
    for (int tc = 0; tc < 2; tc++) {
      Case c;
      make_case(&c, cases[i][0], cases[i][1], cases[i][2], cases[i][3], cases[i][4], cases[i][5], 100 + i);
      all &= check_case(&c, thread_counts[tc]);
      free_case(&c);
    }

  /* the cfg2 step through the drop-ins: prep + up GEMM, prep + down GEMM,
   * from the pool's threads and from one caller thread */
  Case up, down;
  make_case(&up, 4, 8, 8192, 2048, 64, 0, 7);
  make_case(&down, 4, 8, 2048, 8192, 64, 0, 8);
  enum { REPS = 200 };
  double t[REPS];
  const int tcs[] = {nt, 1};
  for (int q = 0; q < 2; q++) {
    const int n = tcs[q];
    for (int w = 0; w < 10; w++) gemm_run(&up.j, n), gemm_run(&down.j, n);
    for (int r = 0; r < REPS; r++) {
      const double t0 = now_us();
      gemm_run(&up.j, n);
      gemm_run(&down.j, n);
      t[r] = now_us() - t0;
    }
    qsort(t, REPS, sizeof t[0], cmp_d);
    printf("cfg2 step through the drop-ins (%d thread%s): median %.1f us, min %.1f, max %.1f\n", n,
           n > 1 ? "s" : "", t[REPS / 2], t[0], t[REPS - 1]);
  }
  free_case(&up);
  free_case(&down);
  pool_close();
  printf(all ? "all ok\n" : "FAILED\n");
  return all ? 0 : 1;
}
