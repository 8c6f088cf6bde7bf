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

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <atomic>
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

// The kernels address packed A, B and the scales through buffer descriptors
// with 32-bit byte ranges and mask lanes with the offset FGM_OOB = 2^31, so a
// launch's ranges must stay below 2^31 bytes.  B is cut along N into launches
// of at most FGM_B_CHUNK bytes (the n-block range is contiguous in B, so a cut
// is a rebased pointer); packed A and the int4 scale table cannot be cut that
// way and are refused past the limit.
constexpr uint64_t FGM_B_CHUNK = 1ull << 30;
constexpr uint64_t FGM_RANGE_MAX = 1ull << 31;

int check_ranges(int bits, int m, int n, int k, int group) {
  const uint64_t abytes = (uint64_t)((m + 15) / 16) * 16 * (uint64_t)k;
  if (abytes >= FGM_RANGE_MAX)
    return fail(FGM_HIP_EINVAL, "gemm: packed A of %llu bytes (m=%d k=%d) reaches 2^31", (unsigned long long)abytes,
                m, k);
  if (bits == 4 && group > 0) {
    const uint64_t sbytes = (uint64_t)(k / group) * (uint64_t)n * 2;
    if (sbytes >= FGM_RANGE_MAX)
      return fail(FGM_HIP_EINVAL, "gemm: int4 scale table of %llu bytes reaches 2^31", (unsigned long long)sbytes);
  }
  return FGM_HIP_OK;
}

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
  return check_ranges(bits, m, n, k, group);
}

// The skinny weight-stream kernel up to the row count where the dense MFMA
// kernel overtakes it, when its LDS fits; else the dense kernel.  Crossovers
// measured on MI355X (bench.py --only sweep, N = 8192, K = 2048, cold
// weights; skinny / dense us): int8 M = 32: 7.3 / 7.7, M = 48: 8.6 / 8.0;
// int4 group 64 M = 48: 12.2 / 12.7, M = 64: 18.3 / 12.8; int4 wider groups
// (the skinny kernel's general-group chain) M = 16: 8.4 / 13.1, M = 32:
// 17.5 / 12.5.
int skinny_max_rows(int bits, int group) { return bits == 8 ? 32 : (group == 64 ? 48 : 16); }

int gemm_path(int bits, int m, int k, int group) {
  return (m <= skinny_max_rows(bits, group) && fgm_decode_fits(bits, m, k, group)) ? 0 : 1;
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
  p.nwg = 0;
  p.tw = p.ks = p.nbw = 0;
  return p;
}

// Launch validated problems of one weight type: skinny ones share launches,
// dense ones share launches, FGM_MAX_BATCH per launch.  Empty problems are
// skipped; an empty contraction (k == 0) writes 0, as the reference does.
int run_probs(int bits, const GemmProb* probs, int count, hipStream_t st);

// Bytes of B that a problem's launch addresses: n-blocks [0, n0 + nblocks).
uint64_t b_span(int bits, const GemmProb& p) {
  return (uint64_t)(p.n0 + p.nblocks) * (uint64_t)p.K * (bits == 8 ? 16 : 8);
}

// One problem whose B spans more than FGM_B_CHUNK bytes, as launches over
// n-block chunks: B, the scales' column, C and acc_out are rebased to the
// chunk's first column; N stays the scale table's row stride.  Each chunk
// starts at n-block 0 of its rebased B and spans at most FGM_B_CHUNK bytes,
// or is a single n-block (K * 16 bytes < 2^31, as packed A's limit implies:
// the kernels address it directly), so no chunk is cut again.
int run_chunked(int bits, const GemmProb& p, hipStream_t st) {
  const uint64_t nb_bytes = (uint64_t)p.K * (bits == 8 ? 16 : 8);
  int step = (int)std::min<uint64_t>(FGM_B_CHUNK / nb_bytes, 1u << 24);
  if (step < 1) step = 1;
  for (int c0 = p.n0; c0 < p.n0 + p.nblocks; c0 += step) {
    GemmProb q = p;
    const int cnt = std::min(step, p.n0 + p.nblocks - c0);
    q.B = (const int8_t*)p.B + (size_t)c0 * nb_bytes;
    if (p.b_scale)
      q.b_scale = bits == 8 ? (const void*)((const float*)p.b_scale + 16 * (size_t)c0)
                            : (const void*)((const uint16_t*)p.b_scale + 16 * (size_t)c0);
    if (p.C) q.C = p.C + 16 * (size_t)c0;
    if (p.acc_out) q.acc_out = p.acc_out + 16 * (size_t)c0;
    q.n0 = 0;
    q.nblocks = cnt;
    int rc = run_probs(bits, &q, 1, st);
    if (rc) return rc;
  }
  return FGM_HIP_OK;
}

// A problem is cut along N when its B span passes FGM_B_CHUNK and a cut can
// shrink it: a lone n-block at the start of B is launched as it is.
bool needs_chunks(int bits, const GemmProb& p) {
  return b_span(bits, p) > FGM_B_CHUNK && (p.n0 > 0 || p.nblocks > 1);
}

// Set by fgm_hip_gemm_plan on its own thread: run_probs then counts the
// launch calls it would make instead of making them.
thread_local int* g_plan = nullptr;

int run_probs(int bits, const GemmProb* probs, int count, hipStream_t st) {
  GemmBatch sk{}, de{};
  auto flush = [&](GemmBatch& b, int dense) -> int {
    if (!b.count) return FGM_HIP_OK;
    if (g_plan) {
      ++*g_plan;
      b.count = 0;
      return FGM_HIP_OK;
    }
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
      // a fill kernel, not a memset: this path may be captured into a graph
      if (!p.acc_out && g_plan) {
        ++*g_plan;
      } else if (!p.acc_out) {
        hipError_t e = fgm_launch_fill_zero(p.C + 16 * p.n0, p.ldc, p.M, 16 * p.nblocks, st);
        if (e != hipSuccess) return hip_fail(e, "zero fill launch");
      }
      continue;
    }
    int rc;
    if (needs_chunks(bits, p)) {
      if ((rc = run_chunked(bits, p, st))) return rc;
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
  // drop-in calls holding this copy (from the upload until their stream has
  // drained)
  std::atomic<int> users{0};
};
struct WeightCache {
  std::shared_mutex mu;
  std::unordered_map<const void*, CachedBuf*> map;
  // copies replaced after a fingerprint mismatch (a caller freed a weight
  // buffer and reused its address): another thread may still be running on
  // the old copy, so it is freed once no call holds it -- at the next
  // upload, or by fgm_hip_weight_cache_clear()
  std::vector<CachedBuf*> retired;
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

// The device copy of a host buffer, held for the caller (users + 1) until
// it calls release_copy.
int cached_upload(const void* host, size_t bytes, CachedBuf** out) {
  const uint64_t fp = fingerprint(host, bytes);
  {
    std::shared_lock<std::shared_mutex> lk(g_wcache.mu);
    auto it = g_wcache.map.find(host);
    if (it != g_wcache.map.end() && it->second->bytes == bytes && it->second->fp == fp) {
      it->second->users++;
      *out = it->second;
      return FGM_HIP_OK;
    }
  }
  std::unique_lock<std::shared_mutex> lk(g_wcache.mu);
  auto it = g_wcache.map.find(host);
  if (it != g_wcache.map.end()) {
    if (it->second->bytes == bytes && it->second->fp == fp) {
      it->second->users++;
      *out = it->second;
      return FGM_HIP_OK;
    }
    g_wcache.retired.push_back(it->second);
    g_wcache.map.erase(it);
  }
  // free the retired copies no call holds any more
  for (size_t i = 0; i < g_wcache.retired.size();) {
    CachedBuf* r = g_wcache.retired[i];
    if (r->users.load() == 0) {
      (void)hipFree(r->dev);
      delete r;
      g_wcache.retired[i] = g_wcache.retired.back();
      g_wcache.retired.pop_back();
    } else {
      i++;
    }
  }
  void* d = nullptr;
  HIPCHK(hipMalloc(&d, bytes ? bytes : 1));
  hipError_t e = hipMemcpy(d, host, bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(d);
    return hip_fail(e, "weight upload");
  }
  CachedBuf* c = new CachedBuf;
  c->bytes = bytes;
  c->fp = fp;
  c->dev = d;
  c->users = 1;
  g_wcache.map[host] = c;
  *out = c;
  return FGM_HIP_OK;
}

// Drops a drop-in call's hold on the copies it used, once the stream its
// launches went to has drained.
struct CopyHold {
  CachedBuf* c[2] = {nullptr, nullptr};
  hipStream_t st = nullptr;
  ~CopyHold() {
    if (!c[0] && !c[1]) return;
    if (st) (void)hipStreamSynchronize(st);
    for (CachedBuf* x : c)
      if (x) x->users--;
  }
};

// Per-thread stream and grow-only staging buffers for the drop-ins: device
// buffers, and pinned host buffers through which the caller's (pageable)
// arrays move, so that each call is one host-to-device DMA, the launches and
// one device-to-host DMA, with a memcpy on either side.  They live until the
// process ends (no destructor: freeing device memory while the HIP runtime is
// being torn down at exit is not safe).
struct Staging {
  hipStream_t st = nullptr;
  void* buf[8] = {};
  size_t cap[8] = {};
  void* pin[2] = {};
  size_t pcap[2] = {};
};
// A thread takes a context on its first drop-in call and hands it back to a
// free list when it exits, where the next new thread finds it: callers that
// start threads per call (or per batch) reuse the buffers and stream instead
// of leaking a set per thread.  The list is never destroyed.
struct StagingPool {
  std::mutex mu;
  std::vector<Staging*> free;
};
StagingPool& stage_pool() {
  static StagingPool* p = new StagingPool;
  return *p;
}
struct StageHolder {
  Staging* s = nullptr;
  Staging& get() {
    if (!s) {
      StagingPool& pl = stage_pool();
      std::lock_guard<std::mutex> lk(pl.mu);
      if (!pl.free.empty()) {
        s = pl.free.back();
        pl.free.pop_back();
      } else {
        s = new Staging;
      }
    }
    return *s;
  }
  ~StageHolder() {
    if (!s) return;
    StagingPool& pl = stage_pool();
    std::lock_guard<std::mutex> lk(pl.mu);
    pl.free.push_back(s);
  }
};
thread_local StageHolder g_stage_holder;
#define g_stage (g_stage_holder.get())

int pinned(int slot, size_t bytes, void** out) {
  if (g_stage.pcap[slot] < bytes) {
    if (g_stage.pin[slot]) HIPCHK(hipHostFree(g_stage.pin[slot]));
    g_stage.pin[slot] = nullptr;
    g_stage.pcap[slot] = 0;
    HIPCHK(hipHostMalloc(&g_stage.pin[slot], bytes ? bytes : 1, hipHostMallocDefault));
    g_stage.pcap[slot] = bytes;
  }
  *out = g_stage.pin[slot];
  return FGM_HIP_OK;
}

inline size_t up256(size_t x) { return (x + 255) & ~(size_t)255; }

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
  void *da = nullptr, *das = nullptr, *dc = nullptr;
  CopyHold hold;
  if (!g_stage.st) HIPCHK(hipStreamCreate(&g_stage.st));
  hold.st = g_stage.st;
  if ((rc = cached_upload(b, bbytes, &hold.c[0]))) return rc;
  if ((rc = cached_upload(b_scale, sbytes, &hold.c[1]))) return rc;
  void* db = hold.c[0]->dev;
  void* ds = hold.c[1]->dev;
  const size_t abytes = packed_a_len(m, k);
  const int wcols = 16 * (n1 - n0);
  const size_t cbytes = (size_t)m * wcols * 4;
  // in: [packed A | a_scale]; out: the written columns of C, contiguous
  const size_t inb = up256(abytes) + (size_t)m * 4;
  void *pin_in, *pin_out;
  if ((rc = staging(0, inb, &da)) || (rc = staging(2, cbytes, &dc)) || (rc = pinned(0, inb, &pin_in)) ||
      (rc = pinned(1, cbytes, &pin_out)))
    return rc;
  das = (char*)da + up256(abytes);
  hipStream_t st = g_stage.st;
  memcpy(pin_in, a, abytes);
  memcpy((char*)pin_in + up256(abytes), a_scale, (size_t)m * 4);
  HIPCHK(hipMemcpyAsync(da, pin_in, inb, hipMemcpyHostToDevice, st));
  // the kernel indexes C by absolute column; point it 16*n0 columns early
  float* cbase = (float*)dc - 16 * n0;
  if ((rc = run_gemm(bits, m, n, k, (const int8_t*)da, (const float*)das, db, ds, group, cbase,
                     wcols, n0, n1, nullptr, 0, st)))
    return rc;
  HIPCHK(hipMemcpyAsync(pin_out, dc, cbytes, hipMemcpyDeviceToHost, st));
  HIPCHK(hipStreamSynchronize(st));
  for (int r = 0; r < m; r++)
    memcpy(c + (size_t)r * ldc + 16 * n0, (const float*)pin_out + (size_t)r * wcols, (size_t)wcols * 4);
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

// The calling thread's drop-in staging for the other sources' drop-ins
// (fgm_model.hip): its stream, a device buffer and a pinned host buffer of
// at least the given sizes (slots of their own, valid until the thread's
// next staging request).
int fgm_stage(size_t dev_bytes, size_t pin_bytes, void** dev, void** pin, hipStream_t* st) {
  int rc = staging(5, dev_bytes, dev);
  if (rc || (rc = pinned(0, pin_bytes, pin))) return rc;
  *st = g_stage.st;
  return FGM_HIP_OK;
}


// ====================================================================== C ABI
// Status helpers for the library's other sources (fgm_model.hip).
int fgm_status_fail(int code, const char* msg) { return fail(code, "%s", msg); }
int fgm_status_hip(hipError_t e, const char* what) { return hip_fail(e, what); }
int fgm_status_device() { return ensure_device(); }

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

int fgm_hip_gemm_plan(int bits, int m, int n, int k, int group, int n0, int n1, int* launches) {
  if (!launches) return fail(FGM_HIP_EINVAL, "gemm_plan: launches is NULL");
  if (bits != 4 && bits != 8) return fail(FGM_HIP_EINVAL, "gemm_plan: bits=%d", bits);
  int rc = check_gemm(m, n, k, n, n0, n1, bits, group);
  if (rc) return rc;
  // stand-in operand addresses: the dry run computes addresses and reads none
  const uintptr_t fake = (uintptr_t)1 << 44;
  GemmProb p = make_prob(m, n, k, (const int8_t*)fake, (const float*)fake, (const void*)fake,
                         (const void*)fake, group, (float*)fake, n, n0, n1, nullptr, 0);
  int count = 0;
  g_plan = &count;
  rc = run_probs(bits, &p, 1, nullptr);
  g_plan = nullptr;
  *launches = count;
  return rc;
}

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

// One fused problem (rows [0, m)) through the prep kernel.
static int run_prep_preop(int preop, const float* src, const float* aux, int lda, float eps, float* pre,
                   float* rot, int8_t* qa, float* qs, int8_t* pa, int m, int k, int hsz,
                   hipStream_t st, const char* what) {
  fgm_hip_prep_desc d{src, lda, rot, qa, qs, pa, m, k, hsz, 0, m};
  if (m < 0) return fail(FGM_HIP_EINVAL, "%s: m=%d", what, m);
  int rc = check_prep(d);
  if (rc || m == 0) return rc;
  if (preop == PREP_GELU_MUL && !aux) return fail(FGM_HIP_EINVAL, "%s: up is NULL", what);
  if ((rc = ensure_device())) return rc;
  PrepBatch b{};
  PrepProb p{src, rot, qa, qs, pa, lda, m, k, hsz, 0, m, fwht_scale(hsz), 0};
  p.preop = preop;
  p.aux = aux;
  p.pre = pre;
  p.eps = eps;
  b.p[0] = p;
  b.count = 1;
  hipError_t e = fgm_launch_prep(b, st);
  if (e != hipSuccess) return hip_fail(e, what);
  return FGM_HIP_OK;
}

int fgm_hip_prep_rmsnorm_dev(const float* x, int lda, const float* w, float eps, float* xn,
                             float* rot, int8_t* qa, float* qs, int8_t* pa, int m, int k, int hsz,
                             void* stream) {
  return run_prep_preop(PREP_RMSNORM, x, w, lda, eps, xn, rot, qa, qs, pa, m, k, hsz,
                        (hipStream_t)stream, "prep_rmsnorm");
}

int fgm_hip_prep_gelu_mul_dev(const float* gate, const float* up, int lda, float* act, float* rot,
                              int8_t* qa, float* qs, int8_t* pa, int m, int k, int hsz,
                              void* stream) {
  return run_prep_preop(PREP_GELU_MUL, gate, up, lda, 0.0f, act, rot, qa, qs, pa, m, k, hsz,
                        (hipStream_t)stream, "prep_gelu_mul");
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
size_t fgm_hip_weight_cache_bytes(int replaced) {
  std::shared_lock<std::shared_mutex> lk(g_wcache.mu);
  size_t t = 0;
  if (replaced) {
    for (CachedBuf* r : g_wcache.retired) t += r->bytes;
  } else {
    for (auto& kv : g_wcache.map) t += kv.second->bytes;
  }
  return t;
}

void fgm_hip_weight_cache_clear(void) {
  std::unique_lock<std::shared_mutex> lk(g_wcache.mu);
  // callers clear the cache when no drop-in call is in flight; the device is
  // synchronised so that no queued kernel still reads a freed copy
  (void)hipDeviceSynchronize();
  for (auto& kv : g_wcache.map) {
    (void)hipFree(kv.second->dev);
    delete kv.second;
  }
  for (CachedBuf* r : g_wcache.retired) {
    (void)hipFree(r->dev);
    delete r;
  }
  g_wcache.map.clear();
  g_wcache.retired.clear();
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
  // One staging layout on both sides, rows [r0, ...) only:
  //   in : src rows [n][k] f32, then the qa rows [r1, qa_end) the pack reads
  //   out: rot [n][k] f32 | qa [qa_end - r0][k] | qs [n] f32 | pa [blk_end - r0][k]
  const size_t o_src = 0, o_qin = up256((size_t)n * k * 4);
  const size_t inb = o_qin + (size_t)(qa_end - r1) * k;
  const size_t o_rot = 0, o_qa = up256((size_t)n * k * 4), o_qs = o_qa + up256((size_t)(qa_end - r0) * k),
               o_pa = o_qs + up256((size_t)n * 4), outb = o_pa + (size_t)(blk_end - r0) * k;
  void *din, *dout, *pin_in, *pin_out;
  if ((rc = staging(0, inb, &din)) || (rc = staging(1, outb, &dout)) || (rc = pinned(0, inb, &pin_in)) ||
      (rc = pinned(1, outb, &pin_out)))
    return rc;
  hipStream_t st = g_stage.st;
  for (int r = 0; r < n; r++)
    memcpy((float*)((char*)pin_in + o_src) + (size_t)r * k, src + (size_t)(r0 + r) * lda, (size_t)k * 4);
  if (qa_end > r1) memcpy((char*)pin_in + o_qin, qa + (size_t)r1 * k, (size_t)(qa_end - r1) * k);
  HIPCHK(hipMemcpyAsync(din, pin_in, inb, hipMemcpyHostToDevice, st));
  char* dq = (char*)dout + o_qa;
  if (qa_end > r1)  // the rows the pack copies from qa, in place in the output image
    HIPCHK(hipMemcpyAsync(dq + (size_t)n * k, (char*)din + o_qin, (size_t)(qa_end - r1) * k,
                          hipMemcpyDeviceToDevice, st));
  // device images hold rows [r0, ...) only; offset the bases so row indices stay absolute
  const float* bsrc = (const float*)((char*)din + o_src) - (size_t)r0 * k;
  float* brot = (float*)((char*)dout + o_rot) - (size_t)r0 * k;
  int8_t* bqa = (int8_t*)dq - (size_t)r0 * k;
  float* bqs = (float*)((char*)dout + o_qs) - r0;
  int8_t* bpa = (int8_t*)((char*)dout + o_pa) - (size_t)r0 * k;  // r0 % 16 == 0: tile blocks start at r0
  if ((rc = fgm_hip_prep_rows_dev(bsrc, k, brot, bqa, bqs, bpa, m, k, hsz, r0, r1, st))) return rc;
  HIPCHK(hipMemcpyAsync(pin_out, dout, outb, hipMemcpyDeviceToHost, st));
  HIPCHK(hipStreamSynchronize(st));
  const char* po = (const char*)pin_out;
  memcpy(rot + (size_t)r0 * k, po + o_rot, (size_t)n * k * 4);
  memcpy(qa + (size_t)r0 * k, po + o_qa, (size_t)n * k);
  memcpy(qs + r0, po + o_qs, (size_t)n * 4);
  memcpy(pa + (size_t)r0 * k, po + o_pa, (size_t)(blk_end - r0) * k);
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
  // ops.c:138-139, on the host with the host's libm
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

// ------------------------------------------------------ int8-KV attention
// Validates the sequences, fills the row bookkeeping and the grid of `a`
// (scratch pointers excepted); *max_n, *max_span receive the longest range
// and the longest range-or-ring of any row.
static int attn_plan(AttnArgs& a, int* max_n, int* max_span) {
  if (a.nh <= 0 || a.kvh <= 0 || a.nh % a.kvh)
    return fail(FGM_HIP_EINVAL, "attend: n_heads=%d is not a multiple of kv_heads=%d", a.nh, a.kvh);
  if (a.nh / a.kvh > 16) return fail(FGM_HIP_EINVAL, "attend: %d query heads per kv head > 16", a.nh / a.kvh);
  if (a.hd < 64 || a.hd > 512 || a.hd % 64)
    return fail(FGM_HIP_EINVAL, "attend: head_dim=%d must be a multiple of 64 in [64, 512]", a.hd);
  if (a.h0 < 0 || a.h1 > a.nh || a.h0 > a.h1)
    return fail(FGM_HIP_EINVAL, "attend: head range [%d,%d) outside [0,%d)", a.h0, a.h1, a.nh);
  if (a.window < 0) return fail(FGM_HIP_EINVAL, "attend: window=%d", a.window);
  if (a.nseq < 0 || a.nseq > FGM_ATTN_MAX_SEQ)
    return fail(FGM_HIP_EINVAL, "attend: %d sequences (at most %d per call)", a.nseq, FGM_ATTN_MAX_SEQ);
  if (!a.out || !a.q) return fail(FGM_HIP_EINVAL, "attend: out or q is NULL");
  int m = 0, mn = 0, ms = 1, p1max = 1, steps_max = 1;
  long long tiles = 0;
  for (int i = 0; i < a.nseq; i++) {
    AttnSeq& s = a.seq[i];
    if (s.nrows < 0) return fail(FGM_HIP_EINVAL, "attend: sequence %d has %d rows", i, s.nrows);
    if (s.nrows && (!s.kc || !s.ks || !s.vc || !s.vs))
      return fail(FGM_HIP_EINVAL, "attend: sequence %d has a NULL cache pointer", i);
    if (s.k_len <= 0 || s.ring < 0 || s.ring > s.k_len)
      return fail(FGM_HIP_EINVAL, "attend: sequence %d: k_len=%d ring=%d", i, s.k_len, s.ring);
    s.row0 = m;
    m += s.nrows;
    for (int j = 0; j < s.nrows; j++) {
      const AttnSpan sp = attn_span(s.pos0 + j + 1, s.lo, a.window, s.ring);
      if (sp.st < 0 || sp.n < 0)
        return fail(FGM_HIP_EINVAL, "attend: sequence %d row %d: range [%d,%d)", i, j, sp.st, sp.en);
      if (!s.ring && sp.en > s.k_len)
        return fail(FGM_HIP_EINVAL, "attend: sequence %d row %d: position %d outside a cache of %d",
                    i, j, sp.en - 1, s.k_len);
      if (s.ring && sp.n > s.ring)
        return fail(FGM_HIP_EINVAL, "attend: sequence %d row %d: %d positions exceed the ring of %d",
                    i, j, sp.n, s.ring);
      if (sp.n > FGM_ATTN_MAX_SPAN)
        return fail(FGM_HIP_EINVAL, "attend: %d positions in one row (at most %d)", sp.n, FGM_ATTN_MAX_SPAN);
      mn = std::max(mn, sp.n);
      ms = std::max(ms, std::max(sp.n, s.ring));
      tiles += (sp.n + 15) / 16;
      steps_max = std::max(steps_max, sp.dom_steps);
    }
  }
  // positions per score workgroup: two 16-position tiles per wave while the
  // launch is small (about 512 workgroups), more once it has thousands
  const int tpw = (int)std::min<long long>(16, std::max<long long>(2, tiles / (4 * 512)));
  a.p1_chunk = 64 * tpw;
  p1max = std::max(1, (mn + a.p1_chunk - 1) / a.p1_chunk);
  a.m = m;
  a.p1_chunks = p1max;
  // P.V: the row's 64-slot steps split into at most attn_pv_chunks chunks
  const int chunks = m ? attn_pv_chunks(m, a.kvh, a.hd) : 1;
  a.p3_spw = std::max(1, (steps_max + 4 * chunks - 1) / (4 * chunks));
  *max_n = mn;
  *max_span = ms;
  return FGM_HIP_OK;
}

static int attn_run(AttnArgs& a, void* scratch, size_t scratch_bytes, hipStream_t st) {
  int max_n, max_span, rc;
  if ((rc = attn_plan(a, &max_n, &max_span))) return rc;
  if (a.m == 0 || a.h0 == a.h1) return FGM_HIP_OK;
  const size_t need = fgm_attn_layout(nullptr, nullptr, a.m, a.nh, a.kvh, a.hd, max_span);
  if (!scratch || scratch_bytes < need)
    return fail(FGM_HIP_EINVAL, "attend: scratch of %zu bytes, this call needs %zu", scratch_bytes, need);
  if (((uintptr_t)scratch) & 255) return fail(FGM_HIP_EINVAL, "attend: scratch must be 256-byte aligned");
  fgm_attn_layout(&a, scratch, a.m, a.nh, a.kvh, a.hd, max_span);
  hipError_t e = fgm_launch_attn(a, max_n, st);
  return e == hipSuccess ? FGM_HIP_OK : hip_fail(e, "attention launch");
}

size_t fgm_hip_attend_scratch_bytes(int m, int n_heads, int kv_heads, int head_dim, int max_span) {
  if (m <= 0 || n_heads <= 0 || kv_heads <= 0 || n_heads % kv_heads || head_dim <= 0) return 0;
  return fgm_attn_layout(nullptr, nullptr, m, n_heads, kv_heads, head_dim, std::max(max_span, 1));
}

int fgm_hip_attend_dev(float* out, const float* q, const fgm_hip_attn_seq* seqs, int nseq,
                       int n_heads, int kv_heads, int head_dim, int window, void* scratch,
                       size_t scratch_bytes, void* stream) {
  int rc = ensure_device();
  if (rc) return rc;
  if (nseq < 0 || nseq > FGM_ATTN_MAX_SEQ || (nseq && !seqs))
    return fail(FGM_HIP_EINVAL, "attend: bad sequence array (count %d, at most %d)", nseq, FGM_ATTN_MAX_SEQ);
  AttnArgs a{};
  for (int i = 0; i < nseq; i++) {
    const fgm_hip_attn_seq& s = seqs[i];
    a.seq[i] = AttnSeq{s.kc, s.ks, s.vc, s.vs, s.k_len, s.ring, s.pos, 0, s.rows, 0};
  }
  a.nseq = nseq, a.nh = n_heads, a.kvh = kv_heads, a.hd = head_dim, a.window = window;
  a.h0 = 0, a.h1 = n_heads, a.out = out, a.q = q;
  return attn_run(a, scratch, scratch_bytes, (hipStream_t)stream);
}

int fgm_hip_attend_heads_dev(float* out, const float* q, const int8_t* kc, const float* ks,
                             const int8_t* vc, const float* vs, int n_heads, int kv_heads,
                             int head_dim, int start, int end, int h0, int h1, int ring, int cap,
                             void* scratch, size_t scratch_bytes, void* stream) {
  int rc = ensure_device();
  if (rc) return rc;
  if (start < 0 || end < start)
    return fail(FGM_HIP_EINVAL, "attend_heads: range [%d,%d)", start, end);
  AttnArgs a{};
  a.seq[0] = AttnSeq{kc, ks, vc, vs, cap, ring, end - 1, start, 1, 0};
  a.nseq = 1, a.nh = n_heads, a.kvh = kv_heads, a.hd = head_dim, a.window = 0;
  a.h0 = h0, a.h1 = h1, a.out = out, a.q = q;
  return attn_run(a, scratch, scratch_bytes, (hipStream_t)stream);
}

int fgm_hip_store_v_t_dev(int8_t* vt, const int8_t* src, int n, int slot, void* stream) {
  int rc = ensure_device();
  if (rc) return rc;
  if (n < 0 || slot < 0) return fail(FGM_HIP_EINVAL, "store_v_t: n=%d slot=%d", n, slot);
  if (n && (!vt || !src)) return fail(FGM_HIP_EINVAL, "store_v_t: NULL buffer");
  hipError_t e = fgm_launch_store_v_t(vt, src, n, slot, (hipStream_t)stream);
  return e == hipSuccess ? FGM_HIP_OK : hip_fail(e, "store_v_t launch");
}

int fgm_hip_kv_store_dev(const float* k, const float* v, int m, int row_len, int8_t* kc, float* ks,
                         int8_t* vt, float* vs, int cap, int pos, int ring, void* stream) {
  int rc = ensure_device();
  if (rc) return rc;
  if (m < 0 || row_len < 0 || pos < 0 || ring < 0 || cap < 0)
    return fail(FGM_HIP_EINVAL, "kv_store: m=%d row_len=%d cap=%d pos=%d ring=%d", m, row_len, cap, pos, ring);
  if (ring ? ring > cap : (long long)pos + m > cap)
    return fail(FGM_HIP_EINVAL, "kv_store: positions [%d,%d) do not fit a cache of %d slots (ring %d)", pos,
                pos + m, cap, ring);
  if (row_len > 8192) return fail(FGM_HIP_EINVAL, "kv_store: row_len=%d > 8192", row_len);
  if (ring && m > ring) return fail(FGM_HIP_EINVAL, "kv_store: %d rows overwrite each other in a ring of %d", m, ring);
  if (m && (!k || !v || !kc || !ks || !vt || !vs)) return fail(FGM_HIP_EINVAL, "kv_store: NULL buffer");
  hipError_t e = fgm_launch_kv_store(k, v, m, row_len, kc, ks, vt, vs, pos, ring, (hipStream_t)stream);
  return e == hipSuccess ? FGM_HIP_OK : hip_fail(e, "kv_store launch");
}

// drop-ins: the caches move to the device per call (they are the caller's
// mutable host buffers); `scratch` is the reference's host scratch and is
// not touched.
static int dropin_attend(float* out, const float* q, const int8_t* kc, const float* ks,
                         const int8_t* vc, const float* vs, int n_heads, int kv_heads, int head_dim,
                         int start, int end, int h0, int h1, int ring, int cap) {
  int rc = ensure_device();
  if (rc) return rc;
  if (n_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || cap <= 0 || h1 <= h0) {
    AttnArgs a{};
    a.nh = n_heads, a.kvh = kv_heads, a.hd = head_dim, a.h0 = h0, a.h1 = h1;
    int mn, ms;
    a.out = out, a.q = q;
    return attn_plan(a, &mn, &ms);  // reports the invalid argument, or nothing to do
  }
  const size_t kvd = (size_t)kv_heads * head_dim;
  const size_t kb = (size_t)cap * kvd, vb = (size_t)(cap + 3) / 4 * 4 * kvd, ob = (size_t)n_heads * head_dim * 4;
  const int span = std::max(std::max(end - start, ring), 1);
  const size_t sb = fgm_hip_attend_scratch_bytes(1, n_heads, kv_heads, head_dim, span);
  void *dq, *dkc, *dks, *dvc, *dvs, *dout, *dsc;
  if ((rc = staging(0, ob, &dq)) || (rc = staging(1, kb, &dkc)) || (rc = staging(2, (size_t)cap * 4, &dks)) ||
      (rc = staging(3, vb, &dvc)) || (rc = staging(4, (size_t)cap * 4, &dvs)) || (rc = staging(5, ob, &dout)) ||
      (rc = staging(6, sb, &dsc)))
    return rc;
  hipStream_t st = g_stage.st;
  HIPCHK(hipMemcpyAsync(dq, q, ob, hipMemcpyHostToDevice, st));
  HIPCHK(hipMemcpyAsync(dkc, kc, kb, hipMemcpyHostToDevice, st));
  HIPCHK(hipMemcpyAsync(dks, ks, (size_t)cap * 4, hipMemcpyHostToDevice, st));
  HIPCHK(hipMemcpyAsync(dvc, vc, vb, hipMemcpyHostToDevice, st));
  HIPCHK(hipMemcpyAsync(dvs, vs, (size_t)cap * 4, hipMemcpyHostToDevice, st));
  if ((rc = fgm_hip_attend_heads_dev((float*)dout, (const float*)dq, (const int8_t*)dkc, (const float*)dks,
                                     (const int8_t*)dvc, (const float*)dvs, n_heads, kv_heads, head_dim,
                                     start, end, h0, h1, ring, cap, dsc, sb, st)))
    return rc;
  const size_t o0 = (size_t)h0 * head_dim, on = (size_t)(h1 - h0) * head_dim;
  HIPCHK(hipMemcpyAsync(out + o0, (float*)dout + o0, on * 4, hipMemcpyDeviceToHost, st));
  HIPCHK(hipStreamSynchronize(st));
  return FGM_HIP_OK;
}

void fgm_attend_q8_heads_hip(float* out, const float* q, const int8_t* kc, const float* ks,
                             const int8_t* vc, const float* vs, int n_heads, int kv_heads,
                             int head_dim, int start, int end, float* scratch, int h0, int h1,
                             int ring, int cap) {
  (void)scratch;
  // an empty or reversed range gives zeros, as the reference's loops do
  DROPIN(dropin_attend(out, q, kc, ks, vc, vs, n_heads, kv_heads, head_dim, start, std::max(end, start),
                       h0, h1, ring, cap),
         "fgm_attend_q8_heads_hip");
}

void fgm_attend_q8_hip(float* out, const float* q, const int8_t* kc, const float* ks, const int8_t* vc,
                       const float* vs, int n_heads, int kv_heads, int head_dim, int start, int end,
                       float* scratch) {
  (void)scratch;
  DROPIN(dropin_attend(out, q, kc, ks, vc, vs, n_heads, kv_heads, head_dim, start, std::max(end, start), 0,
                       n_heads, 0, std::max(end, 1)),
         "fgm_attend_q8_hip");
}

void fgm_attend_q8_row_hip(float* out, const float* q, const int8_t* kc, const float* ks,
                           const int8_t* vc, const float* vs, int n_heads, int kv_heads, int head_dim,
                           int start, int end, float* scratch, int ring, int cap) {
  (void)scratch;
  // ops.c:734-744: an empty range zeroes every head (the device path gives
  // zeros for an empty range); kv_heads != 1 takes the per-head path; the
  // head-batched path computes at most eight heads (ops.c:749)
  const int h1 = (end - start <= 0 || kv_heads != 1) ? n_heads : std::min(n_heads, 8);
  DROPIN(dropin_attend(out, q, kc, ks, vc, vs, n_heads, kv_heads, head_dim, start,
                       std::max(end, start), 0, h1, ring, cap),
         "fgm_attend_q8_row_hip");
}

static int dropin_store_v_t(int8_t* vt, const int8_t* src, int n, int slot) {
  int rc = ensure_device();
  if (rc || n <= 0) return rc;
  if (slot < 0) return fail(FGM_HIP_EINVAL, "store_v_t: slot=%d", slot);
  // the n * 4 bytes of slot's four-slot group
  int8_t* grp = vt + (size_t)(slot >> 2) * n * 4;
  void *dg, *ds;
  if ((rc = staging(0, (size_t)n * 4, &dg)) || (rc = staging(1, (size_t)n, &ds))) return rc;
  hipStream_t st = g_stage.st;
  HIPCHK(hipMemcpyAsync(dg, grp, (size_t)n * 4, hipMemcpyHostToDevice, st));
  HIPCHK(hipMemcpyAsync(ds, src, (size_t)n, hipMemcpyHostToDevice, st));
  if ((rc = fgm_hip_store_v_t_dev((int8_t*)dg, (const int8_t*)ds, n, slot & 3, st))) return rc;
  HIPCHK(hipMemcpyAsync(grp, dg, (size_t)n * 4, hipMemcpyDeviceToHost, st));
  HIPCHK(hipStreamSynchronize(st));
  return FGM_HIP_OK;
}

void fgm_store_v_t_hip(int8_t* vt, const int8_t* src, int n, int slot) {
  DROPIN(dropin_store_v_t(vt, src, n, slot), "fgm_store_v_t_hip");
}

// The reference keeps this flag for an A/B switch that its kernels no longer
// read (ops.c:53-54); accepted and ignored.
void fgm_set_scalar_wfill_hip(int on) { (void)on; }

int fgm_rowbatch_scratch_hip(int n_heads, int cap, int head_dim) {
  return n_heads * cap + (cap + 3) / 2 + 2 * head_dim + 64;
}

}  // extern "C"

