// C-ABI layer of libfgm_hip.so: precondition checks, kernel dispatch, the
// host-pointer drop-in entry points and their weight cache.
//
// Error convention:
//   fgm_hip_* (device API) return FGM_HIP_OK or an FGM_HIP_E* code and leave a
//   message for fgm_hip_last_error() on the calling thread;
//   the drop-in fgm_*_hip functions are void like the reference's symbols
//   (lib.rs:19-53), and like the reference's release build (panic = "abort")
//   they print the message and abort on failure.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <shared_mutex>
#include <unordered_map>
#include <vector>

#include "../../include/fgm_hip.h"
#include "fgm_kernels.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(FGM_HIP_EHIP, "%s: %s", what, hipGetErrorString(e));
}

#define HIPCHK(call)                                   \
  do {                                                 \
    hipError_t e_ = (call);                            \
    if (e_ != hipSuccess) return hip_fail(e_, #call);  \
  } while (0)

// ---------------------------------------------------------------- device
std::once_flag g_dev_once;
int g_dev_status = FGM_HIP_OK;
char g_dev_msg[256] = "";

int ensure_device() {
  std::call_once(g_dev_once, [] {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
      g_dev_status = FGM_HIP_ENODEV;
      snprintf(g_dev_msg, sizeof g_dev_msg, "no HIP device");
      return;
    }
    int dev = 0;
    (void)hipGetDevice(&dev);
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess || strncmp(p.gcnArchName, "gfx950", 6) != 0) {
      g_dev_status = FGM_HIP_ENODEV;
      snprintf(g_dev_msg, sizeof g_dev_msg, "device %d is %s, this library is built for gfx950",
               dev, p.gcnArchName);
      return;
    }
  });
  if (g_dev_status != FGM_HIP_OK) return fail(g_dev_status, "%s", g_dev_msg);
  return FGM_HIP_OK;
}

// One activation row (f32) is staged whole in LDS by the preamble kernels.
constexpr size_t ROW_LDS_LIMIT = 128 * 1024;

// ---------------------------------------------------------- validation
int check_gemm(int m, int n, int k, int ldc, int n0, int n1, int bits, int group) {
  if (m < 0 || n < 0 || k < 0) return fail(FGM_HIP_EINVAL, "negative shape m=%d n=%d k=%d", m, n, k);
  if (k % 64) return fail(FGM_HIP_EINVAL, "k=%d is not a multiple of 64", k);
  if (n % 16) return fail(FGM_HIP_EINVAL, "n=%d is not a multiple of 16", n);
  if (n0 < 0 || n1 < n0 || n1 > n / 16)
    return fail(FGM_HIP_EINVAL, "n-block range [%d,%d) outside [0,%d)", n0, n1, n / 16);
  if ((n1 - n0) % 4) return fail(FGM_HIP_EINVAL, "n-block range %d..%d is not a multiple of 4", n0, n1);
  if (m > 0 && n1 > n0 && ldc < 16 * n1) return fail(FGM_HIP_EINVAL, "ldc=%d < 16*n1=%d", ldc, 16 * n1);
  if (bits == 4) {
    if (group <= 0 || group % 64 || k % group)
      return fail(FGM_HIP_EINVAL, "group=%d must be a multiple of 64 dividing k=%d", group, k);
  }
  return FGM_HIP_OK;
}

// Skinny kernel for m <= 64 when its LDS fits, else the dense MFMA kernel.
int gemm_path(int bits, int m, int k, int group) {
  return fgm_decode_fits(bits, m, k, group) ? 0 : 1;
}

GemmProb make_prob(int m, int n, int k, const int8_t* a, const float* a_scale, const void* b,
                   const void* b_scale, int group, float* c, int ldc, int n0, int n1,
                   int32_t* acc, int ldacc) {
  GemmProb p;
  p.A = a;
  p.a_scale = a_scale;
  p.B = b;
  p.b_scale = b_scale;
  p.C = c;
  p.acc_out = acc;
  p.M = m;
  p.N = n;
  p.K = k;
  p.group = group;
  p.ldc = ldc;
  p.ldacc = ldacc;
  p.n0 = n0;
  p.nblocks = n1 - n0;
  p.wg0 = 0;
  p.tw = p.ks = p.nbw = 0;
  return p;
}

// Launch validated problems of one weight type: skinny ones share launches,
// dense ones share launches, FGM_MAX_BATCH per launch.  Empty problems are
// skipped; an empty contraction (k == 0) writes 0, as the reference does.
int run_probs(int bits, const GemmProb* probs, int count, hipStream_t st) {
  GemmBatch sk{}, de{};
  auto flush = [&](GemmBatch& b, int dense) -> int {
    if (!b.count) return FGM_HIP_OK;
    hipError_t e = dense ? fgm_launch_gemm(bits, b, st) : fgm_launch_decode(bits, b, st);
    b.count = 0;
    if (e != hipSuccess) return hip_fail(e, dense ? "dense GEMM launch" : "skinny GEMM launch");
    return FGM_HIP_OK;
  };
  for (int i = 0; i < count; i++) {
    const GemmProb& p = probs[i];
    if (p.M == 0 || p.nblocks == 0) continue;
    // every operand a launch reads or writes must exist
    if (!p.acc_out && !p.C) return fail(FGM_HIP_EINVAL, "gemm: c is NULL");
    if (p.K > 0 && (!p.A || !p.B)) return fail(FGM_HIP_EINVAL, "gemm: a or b is NULL");
    if (p.K > 0 && !p.acc_out && (!p.a_scale || !p.b_scale))
      return fail(FGM_HIP_EINVAL, "gemm: a_scale or b_scale is NULL");
    if (p.K == 0) {
      if (!p.acc_out)
        HIPCHK(hipMemset2DAsync(p.C + 16 * p.n0, (size_t)p.ldc * 4, 0, (size_t)p.nblocks * 64,
                                p.M, st));
      continue;
    }
    const int dense = gemm_path(bits, p.M, p.K, p.group);
    GemmBatch& b = dense ? de : sk;
    b.p[b.count++] = p;
    if (b.count == FGM_MAX_BATCH) {
      int rc = flush(b, dense);
      if (rc) return rc;
    }
  }
  int rc = flush(sk, 0);
  if (rc) return rc;
  return flush(de, 1);
}

int run_gemm(int bits, int m, int n, int k, const int8_t* a, const float* a_scale, const void* b,
             const void* b_scale, int group, float* c, int ldc, int n0, int n1, int32_t* acc,
             int ldacc, hipStream_t st) {
  GemmProb p = make_prob(m, n, k, a, a_scale, b, b_scale, group, c, ldc, n0, n1, acc, ldacc);
  return run_probs(bits, &p, 1, st);
}

float fwht_scale(int hsz) { return hsz > 0 ? 1.0f / sqrtf((float)hsz) : 1.0f; }

bool pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

// ------------------------------------------------------- drop-in support
[[noreturn]] void die(const char* where) {
  fprintf(stderr, "fastgemma_amd: %s: %s\n", where, g_err);
  abort();
}

#define DROPIN(call, where)             \
  do {                                  \
    if ((call) != FGM_HIP_OK) die(where); \
  } while (0)

// Device copies of immutable host buffers (weights and their scales), keyed
// by host address.  The reference's weights are read-only mmapped blobs that
// live as long as the model (model.rs:120-141), so one upload serves every
// later call.  A fingerprint of the size and 16 sampled 16-byte windows
// guards against a freed buffer's address being reused for other data; a
// caller that rewrites a weight buffer in place must call
// fgm_hip_weight_cache_clear().
struct CachedBuf {
  size_t bytes;
  uint64_t fp;
  void* dev;
};
struct WeightCache {
  std::shared_mutex mu;
  std::unordered_map<const void*, CachedBuf> map;
} g_wcache;

uint64_t fingerprint(const void* host, size_t bytes) {
  const unsigned char* p = (const unsigned char*)host;
  uint64_t h = 1469598103934665603ull ^ bytes;
  if (!bytes) return h;
  for (int s = 0; s < 16; s++) {
    size_t off = (bytes > 16) ? (bytes - 16) / 15 * s : 0;
    size_t len = bytes < 16 ? bytes : 16;
    for (size_t i = 0; i < len; i++) h = (h ^ p[off + i]) * 1099511628211ull;
  }
  return h;
}

int cached_upload(const void* host, size_t bytes, void** dev) {
  const uint64_t fp = fingerprint(host, bytes);
  {
    std::shared_lock<std::shared_mutex> lk(g_wcache.mu);
    auto it = g_wcache.map.find(host);
    if (it != g_wcache.map.end() && it->second.bytes == bytes && it->second.fp == fp) {
      *dev = it->second.dev;
      return FGM_HIP_OK;
    }
  }
  std::unique_lock<std::shared_mutex> lk(g_wcache.mu);
  auto it = g_wcache.map.find(host);
  if (it != g_wcache.map.end()) {
    if (it->second.bytes == bytes && it->second.fp == fp) {
      *dev = it->second.dev;
      return FGM_HIP_OK;
    }
    HIPCHK(hipFree(it->second.dev));
    g_wcache.map.erase(it);
  }
  void* d = nullptr;
  HIPCHK(hipMalloc(&d, bytes ? bytes : 1));
  HIPCHK(hipMemcpy(d, host, bytes, hipMemcpyHostToDevice));
  g_wcache.map[host] = CachedBuf{bytes, fp, d};
  *dev = d;
  return FGM_HIP_OK;
}

// Per-thread stream and grow-only device staging buffers for the drop-ins.
// They live until the process ends (no destructor: freeing device memory
// while the HIP runtime is being torn down at exit is not safe).
struct Staging {
  hipStream_t st = nullptr;
  void* buf[6] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
  size_t cap[6] = {0, 0, 0, 0, 0, 0};
};
thread_local Staging g_stage;

int staging(int slot, size_t bytes, void** out) {
  if (!g_stage.st) HIPCHK(hipStreamCreate(&g_stage.st));
  if (g_stage.cap[slot] < bytes) {
    if (g_stage.buf[slot]) HIPCHK(hipFree(g_stage.buf[slot]));
    g_stage.buf[slot] = nullptr;
    g_stage.cap[slot] = 0;
    HIPCHK(hipMalloc(&g_stage.buf[slot], bytes ? bytes : 1));
    g_stage.cap[slot] = bytes;
  }
  *out = g_stage.buf[slot];
  return FGM_HIP_OK;
}

size_t packed_a_len(int m, int k) { return (size_t)((m + 15) / 16) * 16 * (size_t)k; }

int dropin_gemm(int bits, int m, int n, int k, const int8_t* a, const float* a_scale,
                const void* b, const void* b_scale, int group, float* c, int ldc, int n0,
                int n1) {
  int rc = ensure_device();
  if (rc) return rc;
  if ((rc = check_gemm(m, n, k, ldc, n0, n1, bits, group))) return rc;
  if (m == 0 || n1 == n0) return FGM_HIP_OK;
  const size_t bbytes = bits == 8 ? (size_t)n * k : (size_t)n * k / 2;
  const size_t sbytes = bits == 8 ? (size_t)n * 4 : (size_t)(k / group) * n * 2;
  void *db = nullptr, *ds = nullptr, *da = nullptr, *das = nullptr, *dc = nullptr;
  if ((rc = cached_upload(b, bbytes, &db))) return rc;
  if ((rc = cached_upload(b_scale, sbytes, &ds))) return rc;
  const size_t abytes = packed_a_len(m, k);
  const int wcols = 16 * (n1 - n0);
  if ((rc = staging(0, abytes, &da)) || (rc = staging(1, (size_t)m * 4, &das)) ||
      (rc = staging(2, (size_t)m * wcols * 4, &dc)))
    return rc;
  hipStream_t st = g_stage.st;
  HIPCHK(hipMemcpyAsync(da, a, abytes, hipMemcpyHostToDevice, st));
  HIPCHK(hipMemcpyAsync(das, a_scale, (size_t)m * 4, hipMemcpyHostToDevice, st));
  // the kernel indexes C by absolute column; point it 16*n0 columns early
  float* cbase = (float*)dc - 16 * n0;
  if ((rc = run_gemm(bits, m, n, k, (const int8_t*)da, (const float*)das, db, ds, group, cbase,
                     wcols, n0, n1, nullptr, 0, st)))
    return rc;
  HIPCHK(hipMemcpy2DAsync(c + 16 * n0, (size_t)ldc * 4, dc, (size_t)wcols * 4, (size_t)wcols * 4,
                          m, hipMemcpyDeviceToHost, st));
  HIPCHK(hipStreamSynchronize(st));
  return FGM_HIP_OK;
}

int check_prep(const fgm_hip_prep_desc& d) {
  const int m = d.m, k = d.k, hsz = d.hsz, r0 = d.r0, r1 = d.r1, lda = d.lda;
  if (r0 >= r1) return FGM_HIP_OK;
  if (k <= 0 || k % 64) return fail(FGM_HIP_EINVAL, "prep_rows: k=%d must be a positive multiple of 64", k);
  if (r0 < 0 || r0 % 16) return fail(FGM_HIP_EINVAL, "prep_rows: r0=%d must be a multiple of 16", r0);
  if (r1 > m) return fail(FGM_HIP_EINVAL, "prep_rows: r1=%d > m=%d", r1, m);
  if (lda < k) return fail(FGM_HIP_EINVAL, "prep_rows: lda=%d < k=%d", lda, k);
  if (hsz < 0 || (hsz > 0 && (!pow2(hsz) || k % hsz)))
    return fail(FGM_HIP_EINVAL, "prep_rows: hsz=%d must be 0 or a power of two dividing k=%d", hsz, k);
  if ((size_t)k * 4 > ROW_LDS_LIMIT)
    return fail(FGM_HIP_EINVAL, "prep_rows: k=%d > 32768 (one row must fit in LDS)", k);
  if (!d.src || !d.qs || !d.pa) return fail(FGM_HIP_EINVAL, "prep_rows: src, qs and pa are required");
  const int blk_end = ((r1 + 15) / 16) * 16;
  if (r1 < m && blk_end > r1 && !d.qa)
    return fail(FGM_HIP_EINVAL, "prep_rows: rows [%d,%d) are packed from qa, which is NULL", r1,
                blk_end < m ? blk_end : m);
  return FGM_HIP_OK;
}

}  // namespace

// ====================================================================== C ABI
extern "C" {

const char* fgm_hip_last_error(void) { return g_err; }

int fgm_hip_init(int device) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n)
    return fail(FGM_HIP_ENODEV, "device %d not present (%d devices)", device, n);
  HIPCHK(hipSetDevice(device));
  return ensure_device();
}

int fgm_hip_available(void) { return ensure_device() == FGM_HIP_OK ? 1 : 0; }

int fgm_hip_gemm_path(int bits, int m, int k, int group) { return gemm_path(bits, m, k, group); }

int fgm_hip_gemm_q8c_dev(int m, int n, int k, const int8_t* a, const float* a_scale,
                         const int8_t* b, const float* b_scale, float* c, int ldc, int n0, int n1,
                         void* stream) {
  int rc = check_gemm(m, n, k, ldc, n0, n1, 8, 0);
  if (rc || (rc = ensure_device())) return rc;
  return run_gemm(8, m, n, k, a, a_scale, b, b_scale, 0, c, ldc, n0, n1, nullptr, 0,
                  (hipStream_t)stream);
}

int fgm_hip_gemm_q4g_dev(int m, int n, int k, const int8_t* a, const float* a_scale,
                         const uint8_t* bq, const uint16_t* b_scale, int group, float* c, int ldc,
                         int n0, int n1, void* stream) {
  int rc = check_gemm(m, n, k, ldc, n0, n1, 4, group);
  if (rc || (rc = ensure_device())) return rc;
  return run_gemm(4, m, n, k, a, a_scale, bq, b_scale, group, c, ldc, n0, n1, nullptr, 0,
                  (hipStream_t)stream);
}

int fgm_hip_acc_q8c_dev(int m, int n, int k, const int8_t* a, const int8_t* b, int32_t* acc,
                        int ldacc, int n0, int n1, void* stream) {
  int rc = check_gemm(m, n, k, ldacc, n0, n1, 8, 0);
  if (rc || (rc = ensure_device())) return rc;
  if (!acc) return fail(FGM_HIP_EINVAL, "acc is NULL");
  return run_gemm(8, m, n, k, a, nullptr, b, nullptr, 0, nullptr, 0, n0, n1, acc, ldacc,
                  (hipStream_t)stream);
}

int fgm_hip_acc_q4g_dev(int m, int n, int k, const int8_t* a, const uint8_t* bq, int group,
                        int32_t* acc, int ldacc, int n0, int n1, void* stream) {
  int rc = check_gemm(m, n, k, ldacc, n0, n1, 4, group);
  if (rc || (rc = ensure_device())) return rc;
  if (!acc) return fail(FGM_HIP_EINVAL, "acc is NULL");
  return run_gemm(4, m, n, k, a, nullptr, bq, nullptr, group, nullptr, 0, n0, n1, acc, ldacc,
                  (hipStream_t)stream);
}

int fgm_hip_prep_rows_dev(const float* src, int lda, float* rot, int8_t* qa, float* qs,
                          int8_t* pa, int m, int k, int hsz, int r0, int r1, void* stream) {
  fgm_hip_prep_desc d{src, lda, rot, qa, qs, pa, m, k, hsz, r0, r1};
  return fgm_hip_prep_batch_dev(&d, 1, stream);
}

int fgm_hip_prep_batch_dev(const fgm_hip_prep_desc* d, int count, void* stream) {
  if (count < 0 || (count > 0 && !d)) return fail(FGM_HIP_EINVAL, "prep batch: bad descriptor array");
  for (int i = 0; i < count; i++) {
    int rc = check_prep(d[i]);
    if (rc) return rc;
  }
  int rc = ensure_device();
  if (rc) return rc;
  PrepBatch b{};
  for (int i = 0; i < count; i++) {
    const fgm_hip_prep_desc& x = d[i];
    if (x.r0 >= x.r1) continue;
    b.p[b.count++] = PrepProb{x.src, x.rot, x.qa, x.qs, x.pa, x.lda, x.m, x.k, x.hsz, x.r0, x.r1,
                              fwht_scale(x.hsz), 0};
    if (b.count == FGM_MAX_BATCH || i == count - 1) {
      hipError_t e = fgm_launch_prep(b, (hipStream_t)stream);
      if (e != hipSuccess) return hip_fail(e, "prep launch");
      b.count = 0;
    }
  }
  if (b.count) {
    hipError_t e = fgm_launch_prep(b, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "prep launch");
  }
  return FGM_HIP_OK;
}

int fgm_hip_gemm_batch_dev(const fgm_hip_gemm_desc* d, int count, void* stream) {
  if (count < 0 || (count > 0 && !d)) return fail(FGM_HIP_EINVAL, "gemm batch: bad descriptor array");
  for (int i = 0; i < count; i++) {
    const fgm_hip_gemm_desc& x = d[i];
    if (x.bits != 4 && x.bits != 8) return fail(FGM_HIP_EINVAL, "gemm batch[%d]: bits=%d", i, x.bits);
    int rc = check_gemm(x.m, x.n, x.k, x.ldc, x.n0, x.n1, x.bits, x.group);
    if (rc) return rc;
  }
  int rc = ensure_device();
  if (rc) return rc;
  GemmProb p4[64], p8[64];
  int n4 = 0, n8 = 0;
  for (int i = 0; i < count; i++) {
    const fgm_hip_gemm_desc& x = d[i];
    GemmProb p = make_prob(x.m, x.n, x.k, x.a, x.a_scale, x.b, x.b_scale, x.group, x.c, x.ldc,
                           x.n0, x.n1, nullptr, 0);
    GemmProb* dst = x.bits == 4 ? p4 : p8;
    int& n = x.bits == 4 ? n4 : n8;
    dst[n++] = p;
    if (n == 64) {
      if ((rc = run_probs(x.bits, dst, n, (hipStream_t)stream))) return rc;
      n = 0;
    }
  }
  if (n4 && (rc = run_probs(4, p4, n4, (hipStream_t)stream))) return rc;
  if (n8 && (rc = run_probs(8, p8, n8, (hipStream_t)stream))) return rc;
  return FGM_HIP_OK;
}

int fgm_hip_quant_act_dev(const float* x, int rows, int k, int8_t* q, float* scale, void* stream) {
  if (rows <= 0 || k <= 0) return FGM_HIP_OK;
  if ((size_t)k * 4 > ROW_LDS_LIMIT) return fail(FGM_HIP_EINVAL, "quant_act: k=%d > 32768 (one row must fit in LDS)", k);
  int rc = ensure_device();
  if (rc) return rc;
  PrepBatch b{};
  b.p[0] = PrepProb{x, nullptr, q, scale, nullptr, k, rows, k, 0, 0, rows, 1.0f, 0};
  b.count = 1;
  hipError_t e = fgm_launch_prep(b, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "quant_act launch");
  return FGM_HIP_OK;
}

int fgm_hip_pack_a_dev(int m, int k, const int8_t* a, int8_t* ap, void* stream) {
  if (m < 0 || k < 0 || k % 64) return fail(FGM_HIP_EINVAL, "pack_a: k=%d must be a multiple of 64", k);
  int rc = ensure_device();
  if (rc) return rc;
  hipError_t e = fgm_launch_pack_a(m, k, a, ap, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "pack_a launch");
  return FGM_HIP_OK;
}

int fgm_hip_fwht_dev(float* x, int n, int hsz, void* stream) {
  if (!pow2(hsz)) return fail(FGM_HIP_EINVAL, "fwht: hsz=%d is not a power of two", hsz);
  if (n < 0 || n % hsz) return fail(FGM_HIP_EINVAL, "fwht: n=%d is not a multiple of hsz=%d", n, hsz);
  if ((size_t)hsz * 4 > ROW_LDS_LIMIT) return fail(FGM_HIP_EINVAL, "fwht: hsz=%d > 32768 (a block must fit in LDS)", hsz);
  int rc = ensure_device();
  if (rc) return rc;
  hipError_t e = fgm_launch_fwht(x, n, hsz, fwht_scale(hsz), (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "fwht launch");
  return FGM_HIP_OK;
}

// ---------------------------------------------------------------- drop-ins
void fgm_hip_weight_cache_clear(void) {
  std::unique_lock<std::shared_mutex> lk(g_wcache.mu);
  for (auto& kv : g_wcache.map) (void)hipFree(kv.second.dev);
  g_wcache.map.clear();
}

void fgm_gemm_q8c_hip(int m, int n, int k, const int8_t* a, const float* a_scale, const int8_t* b,
                      const float* b_scale, float* c, int ldc, int n0, int n1) {
  DROPIN(dropin_gemm(8, m, n, k, a, a_scale, b, b_scale, 0, c, ldc, n0, n1), "fgm_gemm_q8c_hip");
}

void fgm_gemm_q4g_hip(int m, int n, int k, const int8_t* a, const float* a_scale,
                      const uint8_t* bq, const uint16_t* b_scale, int group, float* c, int ldc,
                      int n0, int n1) {
  DROPIN(dropin_gemm(4, m, n, k, a, a_scale, bq, b_scale, group, c, ldc, n0, n1),
         "fgm_gemm_q4g_hip");
}

static int dropin_prep(const float* src, int lda, float* rot, int8_t* qa, float* qs, int8_t* pa,
                       int m, int k, int hsz, int r0, int r1) {
  int rc = ensure_device();
  if (rc) return rc;
  if (r0 >= r1) return FGM_HIP_OK;
  if (r1 > m || r0 < 0 || r0 % 16 || k <= 0 || k % 64 || lda < k)
    return fail(FGM_HIP_EINVAL, "prep_rows: bad rows [%d,%d) m=%d k=%d lda=%d", r0, r1, m, k, lda);
  const int n = r1 - r0;
  const int blk_end = ((r1 + 15) / 16) * 16;
  const int qa_end = blk_end < m ? blk_end : m;  // rows of qa the pack reads
  void *dsrc, *drot, *dqa, *dqs, *dpa;
  if ((rc = staging(0, (size_t)n * k * 4, &dsrc)) || (rc = staging(1, (size_t)n * k * 4, &drot)) ||
      (rc = staging(2, (size_t)(qa_end - r0) * k, &dqa)) || (rc = staging(3, (size_t)n * 4, &dqs)) ||
      (rc = staging(4, (size_t)(blk_end - r0) * k, &dpa)))
    return rc;
  hipStream_t st = g_stage.st;
  // device buffers hold rows [r0, ...) only; offset the bases so row indices stay absolute
  HIPCHK(hipMemcpy2DAsync(dsrc, (size_t)k * 4, src + (size_t)r0 * lda, (size_t)lda * 4,
                          (size_t)k * 4, n, hipMemcpyHostToDevice, st));
  if (qa_end > r1)
    HIPCHK(hipMemcpyAsync((int8_t*)dqa + (size_t)n * k, qa + (size_t)r1 * k,
                          (size_t)(qa_end - r1) * k, hipMemcpyHostToDevice, st));
  const float* bsrc = (const float*)dsrc - (size_t)r0 * k;
  float* brot = (float*)drot - (size_t)r0 * k;
  int8_t* bqa = (int8_t*)dqa - (size_t)r0 * k;
  float* bqs = (float*)dqs - r0;
  int8_t* bpa = (int8_t*)dpa - (size_t)r0 * k;  // r0 % 16 == 0: tile blocks start at r0
  if ((rc = fgm_hip_prep_rows_dev(bsrc, k, brot, bqa, bqs, bpa, m, k, hsz, r0, r1, st))) return rc;
  HIPCHK(hipMemcpyAsync(rot + (size_t)r0 * k, drot, (size_t)n * k * 4, hipMemcpyDeviceToHost, st));
  HIPCHK(hipMemcpyAsync(qa + (size_t)r0 * k, dqa, (size_t)n * k, hipMemcpyDeviceToHost, st));
  HIPCHK(hipMemcpyAsync(qs + r0, dqs, (size_t)n * 4, hipMemcpyDeviceToHost, st));
  HIPCHK(hipMemcpyAsync(pa + (size_t)r0 * k, dpa, (size_t)(blk_end - r0) * k, hipMemcpyDeviceToHost,
                        st));
  HIPCHK(hipStreamSynchronize(st));
  return FGM_HIP_OK;
}

void fgm_prep_rows_hip(const float* src, int lda, float* rot, int8_t* qa, float* qs, int8_t* pa,
                       int m, int k, int hsz, int r0, int r1) {
  DROPIN(dropin_prep(src, lda, rot, qa, qs, pa, m, k, hsz, r0, r1), "fgm_prep_rows_hip");
}

static int dropin_quant(const float* x, int rows, int k, int8_t* q, float* scale) {
  int rc = ensure_device();
  if (rc) return rc;
  if (rows <= 0 || k <= 0) return FGM_HIP_OK;
  void *dx, *dq, *ds;
  if ((rc = staging(0, (size_t)rows * k * 4, &dx)) || (rc = staging(2, (size_t)rows * k, &dq)) ||
      (rc = staging(3, (size_t)rows * 4, &ds)))
    return rc;
  hipStream_t st = g_stage.st;
  HIPCHK(hipMemcpyAsync(dx, x, (size_t)rows * k * 4, hipMemcpyHostToDevice, st));
  if ((rc = fgm_hip_quant_act_dev((const float*)dx, rows, k, (int8_t*)dq, (float*)ds, st))) return rc;
  HIPCHK(hipMemcpyAsync(q, dq, (size_t)rows * k, hipMemcpyDeviceToHost, st));
  HIPCHK(hipMemcpyAsync(scale, ds, (size_t)rows * 4, hipMemcpyDeviceToHost, st));
  HIPCHK(hipStreamSynchronize(st));
  return FGM_HIP_OK;
}

void fgm_quant_act_hip(const float* x, int rows, int k, int8_t* q, float* scale) {
  DROPIN(dropin_quant(x, rows, k, q, scale), "fgm_quant_act_hip");
}

static int dropin_pack(int m, int k, const int8_t* a, int8_t* ap) {
  int rc = ensure_device();
  if (rc) return rc;
  if (m <= 0 || k <= 0) return FGM_HIP_OK;
  void *da, *dap;
  const size_t plen = packed_a_len(m, k);
  if ((rc = staging(2, (size_t)m * k, &da)) || (rc = staging(4, plen, &dap))) return rc;
  hipStream_t st = g_stage.st;
  HIPCHK(hipMemcpyAsync(da, a, (size_t)m * k, hipMemcpyHostToDevice, st));
  if ((rc = fgm_hip_pack_a_dev(m, k, (const int8_t*)da, (int8_t*)dap, st))) return rc;
  HIPCHK(hipMemcpyAsync(ap, dap, plen, hipMemcpyDeviceToHost, st));
  HIPCHK(hipStreamSynchronize(st));
  return FGM_HIP_OK;
}

void fgm_pack_a_hip(int m, int k, const int8_t* a, int8_t* ap) {
  DROPIN(dropin_pack(m, k, a, ap), "fgm_pack_a_hip");
}

static int dropin_fwht(float* x, int n, int hsz) {
  int rc = ensure_device();
  if (rc) return rc;
  if (n <= 0) return FGM_HIP_OK;
  void* dx;
  if ((rc = staging(0, (size_t)n * 4, &dx))) return rc;
  hipStream_t st = g_stage.st;
  HIPCHK(hipMemcpyAsync(dx, x, (size_t)n * 4, hipMemcpyHostToDevice, st));
  if ((rc = fgm_hip_fwht_dev((float*)dx, n, hsz, st))) return rc;
  HIPCHK(hipMemcpyAsync(x, dx, (size_t)n * 4, hipMemcpyDeviceToHost, st));
  HIPCHK(hipStreamSynchronize(st));
  return FGM_HIP_OK;
}

void fgm_fwht_hip(float* x, int n, int hsz) { DROPIN(dropin_fwht(x, n, hsz), "fgm_fwht_hip"); }

// ------------------------------------------------ elementwise, device API
static int check_f32(const void* p, const char* name) {
  return p ? FGM_HIP_OK : fail(FGM_HIP_EINVAL, "%s is NULL", name);
}

int fgm_hip_rmsnorm_dev(float* out, const float* x, const float* w, int rows, int n, float eps,
                        void* stream) {
  int rc = ensure_device();
  if (rc) return rc;
  if (rows < 0 || n < 0) return fail(FGM_HIP_EINVAL, "rmsnorm: rows=%d n=%d", rows, n);
  if (rows == 0 || n == 0) return FGM_HIP_OK;
  if ((size_t)n * 4 > ROW_LDS_LIMIT) return fail(FGM_HIP_EINVAL, "rmsnorm: n=%d > 32768 (one row must fit in LDS)", n);
  if ((rc = check_f32(out, "rmsnorm: out")) || (rc = check_f32(x, "rmsnorm: x"))) return rc;
  hipError_t e = fgm_launch_rmsnorm(out, x, w, rows, n, eps, (hipStream_t)stream);
  return e == hipSuccess ? FGM_HIP_OK : hip_fail(e, "rmsnorm launch");
}

int fgm_hip_gelu_mul_dev(float* out, const float* gate, const float* up, int n, void* stream) {
  int rc = ensure_device();
  if (rc) return rc;
  if (n <= 0) return n < 0 ? fail(FGM_HIP_EINVAL, "gelu_mul: n=%d", n) : FGM_HIP_OK;
  if ((rc = check_f32(out, "gelu_mul: out")) || (rc = check_f32(gate, "gelu_mul: gate"))) return rc;
  hipError_t e = fgm_launch_gelu(out, gate, up, n, (hipStream_t)stream);
  return e == hipSuccess ? FGM_HIP_OK : hip_fail(e, "gelu launch");
}

int fgm_hip_softcap_dev(float* x, int n, float cap, void* stream) {
  int rc = ensure_device();
  if (rc) return rc;
  if (n <= 0) return n < 0 ? fail(FGM_HIP_EINVAL, "softcap: n=%d", n) : FGM_HIP_OK;
  if ((rc = check_f32(x, "softcap: x"))) return rc;
  hipError_t e = fgm_launch_softcap(x, n, cap, (hipStream_t)stream);
  return e == hipSuccess ? FGM_HIP_OK : hip_fail(e, "softcap launch");
}

void fgm_hip_rope_table(float* cs, const float* inv_freq, int head_dim, int pos) {
  // ops.c:133-134, on the host with the host's libm
  for (int j = 0; j < head_dim / 2; j++) {
    const float a = (float)pos * inv_freq[j];
    cs[2 * j] = cosf(a);
    cs[2 * j + 1] = sinf(a);
  }
}

int fgm_hip_rope_dev(float* x, int rows, int n_heads, int head_dim, const float* cs, void* stream) {
  int rc = ensure_device();
  if (rc) return rc;
  if (rows < 0 || n_heads < 0 || head_dim < 0 || head_dim % 2)
    return fail(FGM_HIP_EINVAL, "rope: rows=%d n_heads=%d head_dim=%d (even)", rows, n_heads, head_dim);
  if (!rows || !n_heads || !head_dim) return FGM_HIP_OK;
  if ((rc = check_f32(x, "rope: x")) || (rc = check_f32(cs, "rope: cs"))) return rc;
  hipError_t e = fgm_launch_rope(x, rows, n_heads, head_dim, cs, (hipStream_t)stream);
  return e == hipSuccess ? FGM_HIP_OK : hip_fail(e, "rope launch");
}

static int binop_dev(float* a, const float* b, int n, int op, float s, void* stream, const char* what) {
  int rc = ensure_device();
  if (rc) return rc;
  if (n <= 0) return n < 0 ? fail(FGM_HIP_EINVAL, "%s: n=%d", what, n) : FGM_HIP_OK;
  if ((rc = check_f32(a, what)) || (op < 2 && (rc = check_f32(b, what)))) return rc;
  hipError_t e = fgm_launch_binop(a, b, n, op, s, (hipStream_t)stream);
  return e == hipSuccess ? FGM_HIP_OK : hip_fail(e, what);
}
int fgm_hip_add_dev(float* a, const float* b, int n, void* stream) { return binop_dev(a, b, n, 0, 0.0f, stream, "add"); }
int fgm_hip_mul_dev(float* a, const float* b, int n, void* stream) { return binop_dev(a, b, n, 1, 0.0f, stream, "mul"); }
int fgm_hip_scale_dev(float* a, float s, int n, void* stream) { return binop_dev(a, nullptr, n, 2, s, stream, "scale"); }

// ------------------------------------------------ elementwise, drop-ins
// Host buffers through the per-thread staging buffers, synchronous, like the
// reference's calls (lib.rs:47-59).
static int up_f32(int slot, const float* h, int n, float** d) {
  void* p;
  int rc = staging(slot, (size_t)n * 4, &p);
  if (rc) return rc;
  *d = (float*)p;
  if (h) HIPCHK(hipMemcpyAsync(p, h, (size_t)n * 4, hipMemcpyHostToDevice, g_stage.st));
  return FGM_HIP_OK;
}
static int down_f32(float* h, const float* d, int n) {
  HIPCHK(hipMemcpyAsync(h, d, (size_t)n * 4, hipMemcpyDeviceToHost, g_stage.st));
  HIPCHK(hipStreamSynchronize(g_stage.st));
  return FGM_HIP_OK;
}

static int dropin_rmsnorm(float* out, const float* x, const float* w, int n, float eps) {
  int rc = ensure_device();
  if (rc || n <= 0) return rc;
  float *dx, *dw = nullptr, *dout;
  if ((rc = up_f32(0, x, n, &dx)) || (w && (rc = up_f32(1, w, n, &dw))) || (rc = up_f32(2, nullptr, n, &dout)))
    return rc;
  if ((rc = fgm_hip_rmsnorm_dev(dout, dx, dw, 1, n, eps, g_stage.st))) return rc;
  return down_f32(out, dout, n);
}
void fgm_rmsnorm_hip(float* out, const float* x, const float* w, int n, float eps) {
  DROPIN(dropin_rmsnorm(out, x, w, n, eps), "fgm_rmsnorm_hip");
}
void fgm_rmsnorm_noscale_hip(float* out, const float* x, int n, float eps) {
  DROPIN(dropin_rmsnorm(out, x, nullptr, n, eps), "fgm_rmsnorm_noscale_hip");
}

static int dropin_gelu(float* out, const float* gate, const float* up, int n) {
  int rc = ensure_device();
  if (rc || n <= 0) return rc;
  float *dg, *du = nullptr;
  if ((rc = up_f32(0, gate, n, &dg)) || (up && (rc = up_f32(1, up, n, &du)))) return rc;
  if ((rc = fgm_hip_gelu_mul_dev(dg, dg, du, n, g_stage.st))) return rc;
  return down_f32(out, dg, n);
}
void fgm_gelu_mul_hip(float* out, const float* gate, const float* up, int n) {
  DROPIN(dropin_gelu(out, gate, up, n), "fgm_gelu_mul_hip");
}
void fgm_gelu_hip(float* x, int n) { DROPIN(dropin_gelu(x, x, nullptr, n), "fgm_gelu_hip"); }

static int dropin_rope(float* x, int n_heads, int head_dim, const float* inv_freq, int pos) {
  int rc = ensure_device();
  if (rc || n_heads <= 0 || head_dim <= 0) return rc;
  const int n = n_heads * head_dim;
  std::vector<float> cs((size_t)head_dim);
  fgm_hip_rope_table(cs.data(), inv_freq, head_dim, pos);
  float *dx, *dcs;
  if ((rc = up_f32(0, x, n, &dx)) || (rc = up_f32(1, cs.data(), head_dim, &dcs))) return rc;
  if ((rc = fgm_hip_rope_dev(dx, 1, n_heads, head_dim, dcs, g_stage.st))) return rc;
  return down_f32(x, dx, n);
}
void fgm_rope_hip(float* x, int n_heads, int head_dim, const float* inv_freq, int pos) {
  DROPIN(dropin_rope(x, n_heads, head_dim, inv_freq, pos), "fgm_rope_hip");
}

static int dropin_binop(float* a, const float* b, int n, int op, float s) {
  int rc = ensure_device();
  if (rc || n <= 0) return rc;
  float *da, *db = nullptr;
  if ((rc = up_f32(0, a, n, &da)) || (op < 2 && (rc = up_f32(1, b, n, &db)))) return rc;
  if ((rc = binop_dev(da, db, n, op, s, g_stage.st, "binop"))) return rc;
  return down_f32(a, da, n);
}
void fgm_add_hip(float* a, const float* b, int n) { DROPIN(dropin_binop(a, b, n, 0, 0.0f), "fgm_add_hip"); }
void fgm_mul_hip(float* a, const float* b, int n) { DROPIN(dropin_binop(a, b, n, 1, 0.0f), "fgm_mul_hip"); }
void fgm_scale_hip(float* a, float s, int n) { DROPIN(dropin_binop(a, nullptr, n, 2, s), "fgm_scale_hip"); }

static int dropin_softcap(float* x, int n, float cap) {
  int rc = ensure_device();
  if (rc || n <= 0) return rc;
  float* dx;
  if ((rc = up_f32(0, x, n, &dx))) return rc;
  if ((rc = fgm_hip_softcap_dev(dx, n, cap, g_stage.st))) return rc;
  return down_f32(x, dx, n);
}
void fgm_softcap_hip(float* x, int n, float cap) { DROPIN(dropin_softcap(x, n, cap), "fgm_softcap_hip"); }

}  // extern "C"
