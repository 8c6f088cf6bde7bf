// fgm_model.hip -- the .fgm model file on the GPU: reader, device residency,
// typed tensor access, the int4 / int8 dual-weight selection, the embedding
// gathers and the reference's pool jobs on the HIP backend.
//
// Mirrors crates/fgm-core/src/model.rs:1-220 (file layout, Model::open /
// linear / dual / gather), forward.rs:26-89 (DualW, WeightSel, FGM_WEIGHTS),
// forward.rs:128-158 (Gemm::run) and pool.rs:20-79,285-332 (the jobs) on the
// layout written by convert/fgm.py:1-16:
//   [0, 8)   magic "FASTGEM1"
//   [8, 12)  u32 little-endian header length
//   [12, ..) header JSON {config, tensors: {name: {dtype, shape, offset,
//            nbytes, meta}}, meta}, then 64-byte-aligned tensor blobs at
//            absolute file offsets.
// The file is mapped read-only; with device residency its whole tensor body
// is copied to HBM once (one allocation, offsets preserved), so every later
// GEMM reads weights from HBM with no host traffic.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/fgm_hip.h"
#include "fgm_common.h"
#include "fgm_kernels.h"

// status helpers of fgm_api.hip
int fgm_status_fail(int code, const char* msg);
int fgm_status_hip(hipError_t e, const char* what);
int fgm_status_device();

namespace {
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return fgm_status_fail(code, buf);
}
int hip_fail(hipError_t e, const char* what) { return fgm_status_hip(e, what); }
int ensure_device() { return fgm_status_device(); }
}  // namespace

namespace {

// ------------------------------------------------------------ JSON reader
// Enough JSON for the header: objects, arrays, strings (with escapes),
// numbers, true / false / null.
struct Json {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double num = 0.0;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;

  const Json* get(const char* key) const {
    if (kind != Obj) return nullptr;
    for (const auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

struct JsonParser {
  const char* p;
  const char* end;
  std::string err;

  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
  }
  bool lit(const char* s) {
    const size_t n = strlen(s);
    if ((size_t)(end - p) < n || memcmp(p, s, n)) return false;
    p += n;
    return true;
  }
  static void utf8(std::string& o, uint32_t c) {
    if (c < 0x80) {
      o += (char)c;
    } else if (c < 0x800) {
      o += (char)(0xC0 | (c >> 6));
      o += (char)(0x80 | (c & 63));
    } else if (c < 0x10000) {
      o += (char)(0xE0 | (c >> 12));
      o += (char)(0x80 | ((c >> 6) & 63));
      o += (char)(0x80 | (c & 63));
    } else {
      o += (char)(0xF0 | (c >> 18));
      o += (char)(0x80 | ((c >> 12) & 63));
      o += (char)(0x80 | ((c >> 6) & 63));
      o += (char)(0x80 | (c & 63));
    }
  }
  bool hex4(uint32_t* v) {
    if (end - p < 4) return false;
    uint32_t x = 0;
    for (int i = 0; i < 4; i++) {
      const char c = p[i];
      x <<= 4;
      if (c >= '0' && c <= '9') x |= c - '0';
      else if (c >= 'a' && c <= 'f') x |= c - 'a' + 10;
      else if (c >= 'A' && c <= 'F') x |= c - 'A' + 10;
      else return false;
    }
    p += 4;
    *v = x;
    return true;
  }
  bool string(std::string& o) {
    if (p >= end || *p != '"') return false;
    p++;
    while (p < end && *p != '"') {
      if (*p == '\\') {
        if (++p >= end) return false;
        const char c = *p++;
        switch (c) {
          case '"': o += '"'; break;
          case '\\': o += '\\'; break;
          case '/': o += '/'; break;
          case 'b': o += '\b'; break;
          case 'f': o += '\f'; break;
          case 'n': o += '\n'; break;
          case 'r': o += '\r'; break;
          case 't': o += '\t'; break;
          case 'u': {
            uint32_t u;
            if (!hex4(&u)) return false;
            if (u >= 0xD800 && u < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
              p += 2;
              uint32_t lo;
              if (!hex4(&lo)) return false;
              u = 0x10000 + ((u - 0xD800) << 10) + (lo - 0xDC00);
            }
            utf8(o, u);
            break;
          }
          default: return false;
        }
      } else {
        o += *p++;
      }
    }
    if (p >= end) return false;
    p++;
    return true;
  }
  bool value(Json& v, int depth) {
    if (depth > 64) return false;
    ws();
    if (p >= end) return false;
    const char c = *p;
    if (c == '{') {
      p++;
      v.kind = Json::Obj;
      ws();
      if (p < end && *p == '}') return p++, true;
      for (;;) {
        ws();
        std::string key;
        if (!string(key)) return false;
        ws();
        if (p >= end || *p != ':') return false;
        p++;
        v.obj.emplace_back(std::move(key), Json());
        if (!value(v.obj.back().second, depth + 1)) return false;
        ws();
        if (p < end && *p == ',') { p++; continue; }
        if (p < end && *p == '}') return p++, true;
        return false;
      }
    }
    if (c == '[') {
      p++;
      v.kind = Json::Arr;
      ws();
      if (p < end && *p == ']') return p++, true;
      for (;;) {
        v.arr.emplace_back();
        if (!value(v.arr.back(), depth + 1)) return false;
        ws();
        if (p < end && *p == ',') { p++; continue; }
        if (p < end && *p == ']') return p++, true;
        return false;
      }
    }
    if (c == '"') {
      v.kind = Json::Str;
      return string(v.str);
    }
    if (lit("true")) return v.kind = Json::Bool, v.b = true, true;
    if (lit("false")) return v.kind = Json::Bool, v.b = false, true;
    if (lit("null")) return v.kind = Json::Null, true;
    char* q = nullptr;
    std::string tmp;
    const char* s = p;
    while (s < end && (isdigit((unsigned char)*s) || *s == '-' || *s == '+' || *s == '.' || *s == 'e' || *s == 'E'))
      tmp += *s++;
    if (tmp.empty()) return false;
    v.num = strtod(tmp.c_str(), &q);
    if (q != tmp.c_str() + tmp.size()) return false;
    v.kind = Json::Num;
    p = s;
    return true;
  }
};

bool json_parse(const char* s, size_t n, Json& out) {
  JsonParser jp{s, s + n, {}};
  if (!jp.value(out, 0)) return false;
  jp.ws();
  return jp.p == jp.end;
}

int64_t json_int(const Json* v, int64_t dflt) {
  return (v && v->kind == Json::Num) ? (int64_t)v->num : dflt;
}

struct Tensor {
  std::string dtype;
  std::vector<int64_t> shape;
  size_t offset = 0, nbytes = 0;
  int hadamard = 0, group = -1;  // meta; group -1 = absent
};

}  // namespace

// ---------------------------------------------------------------- the model
struct fgm_hip_model {
  int fd = -1;
  void* map = nullptr;
  size_t size = 0;
  std::string config_json, meta_json;
  std::map<std::string, Tensor> tensors;
  size_t body_lo = 0, body_hi = 0;  // byte range of the tensor blobs
  void* dev = nullptr;               // device copy of [body_lo, body_hi)
  int device = -1;

  const uint8_t* host(const Tensor& t) const { return (const uint8_t*)map + t.offset; }
  const uint8_t* devp(const Tensor& t) const {
    return dev ? (const uint8_t*)dev + (t.offset - body_lo) : nullptr;
  }
  ~fgm_hip_model() {
    if (dev) (void)hipFree(dev);
    if (map) munmap(map, size);
    if (fd >= 0) close(fd);
  }
};

namespace {

// Serialise a parsed value back to compact JSON (the config and meta are
// handed to callers as text).
void json_dump(const Json& v, std::string& o) {
  char buf[64];
  switch (v.kind) {
    case Json::Null: o += "null"; break;
    case Json::Bool: o += v.b ? "true" : "false"; break;
    case Json::Num:
      if (v.num == std::floor(v.num) && std::fabs(v.num) < 9.0e15) snprintf(buf, sizeof buf, "%lld", (long long)v.num);
      else snprintf(buf, sizeof buf, "%.17g", v.num);
      o += buf;
      break;
    case Json::Str:
      o += '"';
      for (char c : v.str) {
        if (c == '"' || c == '\\') { o += '\\'; o += c; }
        else if ((unsigned char)c < 0x20) { snprintf(buf, sizeof buf, "\\u%04x", (unsigned char)c); o += buf; }
        else o += c;
      }
      o += '"';
      break;
    case Json::Arr:
      o += '[';
      for (size_t i = 0; i < v.arr.size(); i++) {
        if (i) o += ',';
        json_dump(v.arr[i], o);
      }
      o += ']';
      break;
    case Json::Obj:
      o += '{';
      for (size_t i = 0; i < v.obj.size(); i++) {
        if (i) o += ',';
        Json k;
        k.kind = Json::Str;
        k.str = v.obj[i].first;
        json_dump(k, o);
        o += ':';
        json_dump(v.obj[i].second, o);
      }
      o += '}';
      break;
  }
}

// The tensor body from the file to HBM through two pinned 8 MiB buffers:
// pread fills one (no page faults on the mapping) while the DMA engine
// drains the other.
int upload_body(void* dev, int fd, size_t file_off, size_t n) {
  constexpr size_t CH = (size_t)8 << 20;
  void* pin[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  hipStream_t st = nullptr;
  hipError_t e = hipSuccess;
  int rc = FGM_HIP_OK;
  if ((e = hipStreamCreate(&st)) != hipSuccess) return hip_fail(e, "model: upload stream");
  for (int i = 0; i < 2 && e == hipSuccess; i++) {
    if ((e = hipHostMalloc(&pin[i], CH, hipHostMallocDefault)) == hipSuccess) e = hipEventCreate(&done[i]);
  }
  for (size_t off = 0, c = 0; e == hipSuccess && off < n; off += CH, c ^= 1) {
    const size_t len = n - off < CH ? n - off : CH;
    if ((e = hipEventSynchronize(done[c])) != hipSuccess) break;  // the buffer's last copy is done
    for (size_t got = 0; got < len;) {
      const ssize_t r = pread(fd, (uint8_t*)pin[c] + got, len - got, (off_t)(file_off + off + got));
      if (r <= 0) {
        rc = fail(FGM_HIP_EINVAL, "model: read failed at offset %zu", file_off + off + got);
        break;
      }
      got += (size_t)r;
    }
    if (rc) break;
    if ((e = hipMemcpyAsync((uint8_t*)dev + off, pin[c], len, hipMemcpyHostToDevice, st)) != hipSuccess) break;
    e = hipEventRecord(done[c], st);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  else (void)hipStreamSynchronize(st);
  if (e != hipSuccess && !rc) rc = hip_fail(e, "model: upload");
  for (int i = 0; i < 2; i++) {
    if (done[i]) (void)hipEventDestroy(done[i]);
    if (pin[i]) (void)hipHostFree(pin[i]);
  }
  (void)hipStreamDestroy(st);
  return rc;
}

int open_model(const char* path, int resident, fgm_hip_model** out) {
  std::unique_ptr<fgm_hip_model> m(new fgm_hip_model());
  m->fd = open(path, O_RDONLY);
  if (m->fd < 0) return fail(FGM_HIP_EINVAL, "model: cannot open %s", path);
  struct stat st;
  if (fstat(m->fd, &st) || st.st_size < 12) return fail(FGM_HIP_EINVAL, "model: %s is not a .fgm file", path);
  m->size = (size_t)st.st_size;
  m->map = mmap(nullptr, m->size, PROT_READ, MAP_PRIVATE, m->fd, 0);
  if (m->map == MAP_FAILED) {
    m->map = nullptr;
    return fail(FGM_HIP_EINVAL, "model: cannot map %s", path);
  }
  const uint8_t* b = (const uint8_t*)m->map;
  if (memcmp(b, "FASTGEM1", 8)) return fail(FGM_HIP_EINVAL, "model: %s is not a .fgm file (magic)", path);
  const uint32_t hlen = (uint32_t)b[8] | (uint32_t)b[9] << 8 | (uint32_t)b[10] << 16 | (uint32_t)b[11] << 24;
  if ((size_t)hlen > m->size - 12) return fail(FGM_HIP_EINVAL, "model: header of %u bytes past the end", hlen);
  Json h;
  if (!json_parse((const char*)b + 12, hlen, h) || h.kind != Json::Obj)
    return fail(FGM_HIP_EINVAL, "model: the header is not valid JSON");
  const Json* cfg = h.get("config");
  const Json* ts = h.get("tensors");
  if (!cfg || cfg->kind != Json::Obj || !ts || ts->kind != Json::Obj)
    return fail(FGM_HIP_EINVAL, "model: header lacks config or tensors");
  json_dump(*cfg, m->config_json);
  if (const Json* mt = h.get("meta")) json_dump(*mt, m->meta_json);
  else m->meta_json = "{}";
  m->body_lo = m->size, m->body_hi = 0;
  for (const auto& kv : ts->obj) {
    const Json& e = kv.second;
    const Json* dt = e.get("dtype");
    const Json* sh = e.get("shape");
    const Json* off = e.get("offset");
    const Json* nb = e.get("nbytes");
    if (!dt || dt->kind != Json::Str || !sh || sh->kind != Json::Arr || !off || off->kind != Json::Num ||
        !nb || nb->kind != Json::Num)
      return fail(FGM_HIP_EINVAL, "model: tensor %s has a malformed entry", kv.first.c_str());
    Tensor t;
    t.dtype = dt->str;
    for (const Json& d : sh->arr) t.shape.push_back(json_int(&d, -1));
    t.offset = (size_t)off->num;
    t.nbytes = (size_t)nb->num;
    if (t.offset > m->size || t.nbytes > m->size - t.offset)
      return fail(FGM_HIP_EINVAL, "model: tensor %s lies past the end of the file", kv.first.c_str());
    if (const Json* meta = e.get("meta")) {
      t.hadamard = (int)json_int(meta->get("hadamard"), 0);
      t.group = (int)json_int(meta->get("group"), -1);
    }
    if (t.nbytes) {
      m->body_lo = std::min(m->body_lo, t.offset);
      m->body_hi = std::max(m->body_hi, t.offset + t.nbytes);
    }
    m->tensors[kv.first] = std::move(t);
  }
  if (m->body_hi < m->body_lo) m->body_lo = m->body_hi = 0;
  if (resident && m->body_hi > m->body_lo) {
    int rc = ensure_device();
    if (rc) return rc;
    hipError_t e = hipGetDevice(&m->device);
    if (e != hipSuccess) return hip_fail(e, "model: hipGetDevice");
    const size_t n = m->body_hi - m->body_lo;
    if ((e = hipMalloc(&m->dev, n)) != hipSuccess) {
      m->dev = nullptr;
      return hip_fail(e, "model: device allocation");
    }
    if ((rc = upload_body(m->dev, m->fd, m->body_lo, n))) return rc;
  }
  *out = m.release();
  return FGM_HIP_OK;
}

const Tensor* find(const fgm_hip_model* m, const char* name) {
  if (!m || !name) return nullptr;
  auto it = m->tensors.find(name);
  return it == m->tensors.end() ? nullptr : &it->second;
}

// Model::linear (model.rs:167-192): dtype q4g (f16 scales at <name>.scale,
// meta.group default 64) or q8c (f32 scales, group 0); meta.hadamard default 0.
int linear_of(const fgm_hip_model* m, const char* name, fgm_hip_linear* o) {
  const Tensor* t = find(m, name);
  if (!t) return fail(FGM_HIP_EINVAL, "model: missing tensor %s", name ? name : "(null)");
  if (t->shape.size() != 2) return fail(FGM_HIP_EINVAL, "model: %s is not two-dimensional", name);
  int bits;
  if (t->dtype == "q4g") bits = 4;
  else if (t->dtype == "q8c") bits = 8;
  else return fail(FGM_HIP_EINVAL, "model: tensor %s has non-linear dtype %s", name, t->dtype.c_str());
  const std::string sname = std::string(name) + ".scale";
  const Tensor* s = find(m, sname.c_str());
  if (!s) return fail(FGM_HIP_EINVAL, "model: missing tensor %s", sname.c_str());
  // the GEMM reads n * k (int8) or n * k / 2 (int4) weight bytes and the
  // scales' n (f32) or (k / group) * n (f16) entries: a short or malformed
  // tensor is refused here rather than read past its end on the device
  const int64_t n = t->shape[0], k = t->shape[1];
  const int group = bits == 4 ? (t->group >= 0 ? t->group : 64) : 0;
  if (n <= 0 || k <= 0 || n % 16 || k % 64 || n > 0x7fffffff || k > 0x7fffffff)
    return fail(FGM_HIP_EINVAL, "model: %s has shape [%lld, %lld] (n %% 16 == 0, k %% 64 == 0 required)", name,
                (long long)n, (long long)k);
  if (bits == 4 && (group <= 0 || group % 64 || k % group))
    return fail(FGM_HIP_EINVAL, "model: %s has group %d (a multiple of 64 dividing k=%lld required)", name, group,
                (long long)k);
  const uint64_t wbytes = bits == 8 ? (uint64_t)n * k : (uint64_t)n * k / 2;
  const uint64_t sbytes = bits == 8 ? (uint64_t)n * 4 : (uint64_t)(k / group) * n * 2;
  if (t->nbytes < wbytes)
    return fail(FGM_HIP_EINVAL, "model: %s holds %zu bytes, its shape needs %llu", name, t->nbytes,
                (unsigned long long)wbytes);
  if (s->nbytes < sbytes)
    return fail(FGM_HIP_EINVAL, "model: %s holds %zu bytes, %s needs %llu", sname.c_str(), s->nbytes, name,
                (unsigned long long)sbytes);
  memset(o, 0, sizeof *o);
  o->bits = bits;
  o->n = (int)n;
  o->k = (int)k;
  o->group = group;
  o->hadamard = t->hadamard;
  o->b_host = m->host(*t);
  o->b_scale_host = m->host(*s);
  o->b = m->devp(*t);
  o->b_scale = m->devp(*s);
  return FGM_HIP_OK;
}

// ------------------------------------------------------------- gather kernels
// fgm_gather_q8r (ops.c:208-217): out = (float)q * sc[row]
__global__ void gather_q8r_kernel(float* out, const int8_t* tbl, const float* sc, const int* rows,
                                  int row0, int k) {
  const int r = rows ? rows[blockIdx.y] : row0;
  const float s = sc[r];
  const int8_t* p = tbl + (size_t)r * k;
  float* o = out + (size_t)blockIdx.y * k;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < k; i += gridDim.x * blockDim.x)
    o[i] = (float)p[i] * s;
}

// fgm_gather_q4r (ops.c:228-251): group 64, per 64-block packed[i] holds
// q[i] (low nibble) and q[i + 32] (high nibble), two's complement; scales f16
// [rows][k / 64].
__global__ void gather_q4r_kernel(float* out, const uint8_t* tbl, const uint16_t* sc, const int* rows,
                                  int row0, int k) {
  const int r = rows ? rows[blockIdx.y] : row0;
  const uint8_t* p = tbl + (size_t)r * (k / 2);
  const uint16_t* rs = sc + (size_t)r * (k / 64);
  float* o = out + (size_t)blockIdx.y * k;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < k; i += gridDim.x * blockDim.x) {
    const int blk = i >> 6, j = i & 63;
    const uint8_t byte = p[blk * 32 + (j & 31)];
    const int nib = j < 32 ? (byte & 15) : (byte >> 4);
    const int q = (nib ^ 8) - 8;
    o[i] = (float)q * f16_bits_to_f32(rs[blk]);
  }
}

int gather_launch(const std::string& dtype, float* out, const void* tbl, const void* sc, const int* rows,
                  int row0, int m, int k, hipStream_t st) {
  if (m <= 0 || k <= 0) return FGM_HIP_OK;
  const dim3 grid((k + 255) / 256 < 64 ? (k + 255) / 256 : 64, m);
  if (dtype == "q8r") {
    hipLaunchKernelGGL(gather_q8r_kernel, grid, dim3(256), 0, st, out, (const int8_t*)tbl, (const float*)sc, rows,
                       row0, k);
  } else if (dtype == "q4r") {
    if (k % 64) return fail(FGM_HIP_EINVAL, "gather_q4r: k=%d is not a multiple of 64", k);
    hipLaunchKernelGGL(gather_q4r_kernel, grid, dim3(256), 0, st, out, (const uint8_t*)tbl, (const uint16_t*)sc,
                       rows, row0, k);
  } else {
    return fail(FGM_HIP_EINVAL, "gather: dtype %s is not a gather table", dtype.c_str());
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? FGM_HIP_OK : hip_fail(e, "gather launch");
}

}  // namespace

extern "C" {

fgm_hip_model* fgm_hip_model_open(const char* path, int device_resident) {
  fgm_hip_model* m = nullptr;
  if (!path) {
    fail(FGM_HIP_EINVAL, "model: path is NULL");
    return nullptr;
  }
  return open_model(path, device_resident, &m) == FGM_HIP_OK ? m : nullptr;
}

void fgm_hip_model_close(fgm_hip_model* m) { delete m; }

int fgm_hip_model_has(const fgm_hip_model* m, const char* name) { return find(m, name) ? 1 : 0; }

const char* fgm_hip_model_config(const fgm_hip_model* m) { return m ? m->config_json.c_str() : nullptr; }

const char* fgm_hip_model_meta(const fgm_hip_model* m) { return m ? m->meta_json.c_str() : nullptr; }

size_t fgm_hip_model_total_bytes(const fgm_hip_model* m) {
  size_t s = 0;
  if (m)
    for (const auto& kv : m->tensors) s += kv.second.nbytes;
  return s;
}

int fgm_hip_model_tensor_count(const fgm_hip_model* m) { return m ? (int)m->tensors.size() : 0; }

const char* fgm_hip_model_tensor_name(const fgm_hip_model* m, int i) {
  if (!m || i < 0 || i >= (int)m->tensors.size()) return nullptr;
  auto it = m->tensors.begin();
  std::advance(it, i);
  return it->first.c_str();
}

int fgm_hip_model_tensor(const fgm_hip_model* m, const char* name, fgm_hip_tensor* out) {
  const Tensor* t = find(m, name);
  if (!t) return fail(FGM_HIP_EINVAL, "model: missing tensor %s", name ? name : "(null)");
  if (!out) return fail(FGM_HIP_EINVAL, "model: out is NULL");
  memset(out, 0, sizeof *out);
  snprintf(out->dtype, sizeof out->dtype, "%s", t->dtype.c_str());
  out->ndim = (int)std::min<size_t>(t->shape.size(), 4);
  for (int i = 0; i < out->ndim; i++) out->shape[i] = t->shape[i];
  out->offset = t->offset;
  out->nbytes = t->nbytes;
  out->host = m->host(*t);
  out->dev = m->devp(*t);
  out->hadamard = t->hadamard;
  out->group = t->group;
  return FGM_HIP_OK;
}

int fgm_hip_model_linear(const fgm_hip_model* m, const char* name, fgm_hip_linear* out) {
  if (!out) return fail(FGM_HIP_EINVAL, "model: out is NULL");
  return linear_of(m, name, out);
}

int fgm_hip_weight_sel(const char* value, int* threshold) {
  int t = 16;
  int sel = FGM_HIP_SEL_ABOVE;
  if (value && !strcmp(value, "int4")) {
    sel = FGM_HIP_SEL_LO;
  } else if (value && !strcmp(value, "int8")) {
    sel = FGM_HIP_SEL_HI;
  } else if (value && !strncmp(value, "auto:", 5)) {
    // Rust's usize parse (forward.rs:64): an optional '+', then decimal
    // digits, value below 2^64; anything else falls back to 16.  Thresholds
    // past INT_MAX behave alike (no row count reaches them).
    const char* d = value + 5;
    if (*d == '+') d++;
    bool ok = *d != 0;
    unsigned __int128 v = 0;
    for (const char* c = d; *c && ok; c++) {
      if (*c < '0' || *c > '9') ok = false;
      else if ((v = v * 10 + (unsigned)(*c - '0')) > (unsigned __int128)UINT64_MAX) ok = false;
    }
    t = ok ? (int)(v > 0x7fffffff ? 0x7fffffff : (unsigned)v) : 16;
  }
  if (threshold) *threshold = t;
  return sel;
}

int fgm_hip_model_dual(const fgm_hip_model* m, const char* name, int rows, int sel, int threshold,
                       fgm_hip_linear* out) {
  if (!out || !name) return fail(FGM_HIP_EINVAL, "model: out or name is NULL");
  const std::string alt = std::string(name) + ".i8";
  const bool hi = find(m, alt.c_str()) != nullptr;
  const bool use_hi = hi && (sel == FGM_HIP_SEL_HI || (sel == FGM_HIP_SEL_ABOVE && rows >= threshold));
  return linear_of(m, use_hi ? alt.c_str() : name, out);
}

int fgm_hip_model_gather_dev(const fgm_hip_model* m, const char* name, const int* rows, int count,
                             float* out, void* stream) {
  int rc = ensure_device();
  if (rc) return rc;
  const Tensor* t = find(m, name);
  if (!t) return fail(FGM_HIP_EINVAL, "model: missing tensor %s", name ? name : "(null)");
  const std::string sname = std::string(name) + ".scale";
  const Tensor* s = find(m, sname.c_str());
  if (!s) return fail(FGM_HIP_EINVAL, "model: missing tensor %s", sname.c_str());
  if (!m->dev) return fail(FGM_HIP_EINVAL, "model: opened without device residency");
  if (t->shape.size() != 2 || count < 0 || (count && (!rows || !out)))
    return fail(FGM_HIP_EINVAL, "gather: bad arguments for %s", name);
  return gather_launch(t->dtype, out, m->devp(*t), m->devp(*s), rows, 0, count, (int)t->shape[1],
                       (hipStream_t)stream);
}

int fgm_hip_gather_dev(int bits, const void* tbl, const void* sc, const int* rows, int count, int k, float* out,
                       void* stream) {
  int rc = ensure_device();
  if (rc) return rc;
  if (bits != 4 && bits != 8) return fail(FGM_HIP_EINVAL, "gather: bits=%d", bits);
  if (count < 0 || k < 0 || (count && (!tbl || !sc || !rows || !out)))
    return fail(FGM_HIP_EINVAL, "gather: bad arguments");
  return gather_launch(bits == 8 ? "q8r" : "q4r", out, tbl, sc, rows, 0, count, k, (hipStream_t)stream);
}

// drop-ins: the table row and its scales move to the device, the row comes back
static int dropin_gather(int bits, float* out, const void* tbl, const void* sc, int row, int k) {
  int rc = ensure_device();
  if (rc || k <= 0) return rc;
  if (row < 0) return fail(FGM_HIP_EINVAL, "gather: row=%d", row);
  if (bits == 4 && k % 64) return fail(FGM_HIP_EINVAL, "gather_q4r: k=%d is not a multiple of 64", k);
  const size_t rb = bits == 8 ? (size_t)k : (size_t)k / 2;
  const size_t sb = bits == 8 ? 4 : (size_t)(k / 64) * 2;
  const uint8_t* trow = (const uint8_t*)tbl + (size_t)row * rb;
  const uint8_t* srow = (const uint8_t*)sc + (size_t)row * sb;
  // in: [row | scales] through pinned memory, out: the k floats, one copy
  // each way on the thread's staging stream, no allocation per call
  const size_t so = (rb + 255) & ~(size_t)255, oo = (so + sb + 255) & ~(size_t)255;
  const size_t pinb = oo > (size_t)k * 4 ? oo : (size_t)k * 4;
  void *dbuf = nullptr, *pin = nullptr;
  hipStream_t st = nullptr;
  if ((rc = fgm_stage(oo + (size_t)k * 4, pinb, &dbuf, &pin, &st))) return rc;
  memcpy(pin, trow, rb);
  memcpy((char*)pin + so, srow, sb);
  hipError_t e;
  if ((e = hipMemcpyAsync(dbuf, pin, so + sb, hipMemcpyHostToDevice, st)) != hipSuccess)
    return hip_fail(e, "gather: upload");
  // the staged row is row 0 of a one-row table
  float* dout = (float*)((char*)dbuf + oo);
  rc = gather_launch(bits == 8 ? "q8r" : "q4r", dout, dbuf, (char*)dbuf + so, nullptr, 0, 1, k, st);
  if (rc) return rc;
  if ((e = hipMemcpyAsync(pin, dout, (size_t)k * 4, hipMemcpyDeviceToHost, st)) != hipSuccess ||
      (e = hipStreamSynchronize(st)) != hipSuccess)
    return hip_fail(e, "gather: download");
  memcpy(out, pin, (size_t)k * 4);
  return FGM_HIP_OK;
}

// ------------------------------------------------------- the pool's jobs
int fgm_hip_pool_gemm_dev(const fgm_hip_gemm_job* j, void* stream) {
  if (!j) return fail(FGM_HIP_EINVAL, "pool gemm: job is NULL");
  if (j->bits == 4)
    return fgm_hip_gemm_q4g_dev(j->m, j->n, j->kdim, j->a, j->a_scale, j->bq, j->s4, j->group ? j->group : 64, j->c,
                                j->ldc, 0, j->n / 16, stream);
  if (j->bits == 8)
    return fgm_hip_gemm_q8c_dev(j->m, j->n, j->kdim, j->a, j->a_scale, j->b8, j->s8, j->c, j->ldc, 0, j->n / 16,
                                stream);
  return fail(FGM_HIP_EINVAL, "pool gemm: bits=%d", j->bits);
}

int fgm_hip_pool_prep_dev(const fgm_hip_prep_job* j, void* stream) {
  if (!j) return fail(FGM_HIP_EINVAL, "pool prep: job is NULL");
  return fgm_hip_prep_rows_dev(j->src, j->lda, j->rot, j->qa, j->qs, j->pa, j->m, j->k, j->hsz, 0, j->m, stream);
}

size_t fgm_hip_linear_scratch_bytes(int m, int k) {
  if (m <= 0 || k <= 0) return 0;
  return 256 + (size_t)(m + 63) / 64 * 256 + (size_t)(m + 15) / 16 * 16 * (size_t)k;
}

int fgm_hip_linear_run_dev(const fgm_hip_linear* w, const float* a, int m, int lda, float* out, void* scratch,
                           size_t scratch_bytes, void* stream) {
  if (!w || !w->b || !w->b_scale) return fail(FGM_HIP_EINVAL, "linear: no device weights (open the model resident)");
  if (m <= 0) return FGM_HIP_OK;
  const size_t need = fgm_hip_linear_scratch_bytes(m, w->k);
  if (!scratch || scratch_bytes < need)
    return fail(FGM_HIP_EINVAL, "linear: scratch of %zu bytes, %zu needed", scratch_bytes, need);
  // qs [m] f32, then the packed activation, both 256-byte aligned
  const uintptr_t base = ((uintptr_t)scratch + 255) & ~(uintptr_t)255;
  float* qs = (float*)base;
  int8_t* pa = (int8_t*)(base + (size_t)(m + 63) / 64 * 256);
  int rc = fgm_hip_prep_rows_dev(a, lda, nullptr, nullptr, qs, pa, m, w->k, w->hadamard, 0, m, stream);
  if (rc) return rc;
  fgm_hip_gemm_job j{};
  j.m = m, j.n = w->n, j.kdim = w->k, j.a = pa, j.a_scale = qs, j.bits = w->bits;
  j.group = w->group ? w->group : 64;
  j.c = out, j.ldc = w->n;
  if (w->bits == 4) j.bq = (const uint8_t*)w->b, j.s4 = (const uint16_t*)w->b_scale;
  else j.b8 = (const int8_t*)w->b, j.s8 = (const float*)w->b_scale;
  return fgm_hip_pool_gemm_dev(&j, stream);
}

// ------------------------------------------------- the allocation-free run
// fgm_hip_linear_run_dev with its scratch (row scales + packed activation) in
// a file-scope device array instead of a caller buffer, for callers that must
// not allocate (graph capture, serving loops).  Each GPU holds its own copy
// of the array for the life of the process; its device address is looked up
// once per device and kept, since the array's name is only a host-side
// stand-in in host code.  Every call on a GPU shares that GPU's array, so
// calls that overlap on one GPU (different streams, concurrent graphs) race.
// Nothing in the array has to start at zero: the prep writes every row scale
// and every packed-A byte the GEMM reads, pad rows included.
constexpr size_t FGM_NOALLOC_SCRATCH_BYTES = (size_t)8 << 20;
static __device__ __align__(256) char scratch[FGM_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int FGM_NOALLOC_MAX_DEVICES = 64;
static std::mutex g_noalloc_mu;
static void* g_noalloc_ptr[FGM_NOALLOC_MAX_DEVICES];

// this device's copy of `scratch` (nullptr and a status on failure)
static int noalloc_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "linear (no-alloc): hipGetDevice");
  if (dev < 0 || dev >= FGM_NOALLOC_MAX_DEVICES)
    return fail(FGM_HIP_EINVAL, "linear (no-alloc): device %d beyond %d", dev, FGM_NOALLOC_MAX_DEVICES);
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if (!g_noalloc_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "linear (no-alloc): scratch address");
    g_noalloc_ptr[dev] = p;
  }
  *out = g_noalloc_ptr[dev];
  return FGM_HIP_OK;
}
}  // namespace

size_t fgm_hip_linear_noalloc_max_bytes(void) { return FGM_NOALLOC_SCRATCH_BYTES; }

int fgm_hip_linear_run_noalloc_dev(const fgm_hip_linear* w, const float* a, int m, int lda, float* out,
                                   void* stream) {
  if (!w || !w->b || !w->b_scale) return fail(FGM_HIP_EINVAL, "linear: no device weights (open the model resident)");
  if (m <= 0) return FGM_HIP_OK;
  const size_t need = fgm_hip_linear_scratch_bytes(m, w->k);
  if (need > FGM_NOALLOC_SCRATCH_BYTES)
    return fail(FGM_HIP_EINVAL, "linear (no-alloc): m=%d k=%d needs %zu scratch bytes, the limit is %zu", m, w->k,
                need, FGM_NOALLOC_SCRATCH_BYTES);
  int rc = ensure_device();
  if (rc) return rc;
  void* p = nullptr;
  if ((rc = noalloc_scratch(&p))) return rc;
  return fgm_hip_linear_run_dev(w, a, m, lda, out, p, FGM_NOALLOC_SCRATCH_BYTES, stream);
}

void fgm_gather_q8r_hip(float* out, const int8_t* tbl, const float* sc, int row, int k) {
  if (dropin_gather(8, out, tbl, sc, row, k) != FGM_HIP_OK) {
    fprintf(stderr, "fastgemma_amd: fgm_gather_q8r_hip: %s\n", fgm_hip_last_error());
    abort();
  }
}

void fgm_gather_q4r_hip(float* out, const uint8_t* tbl, const uint16_t* sc, int row, int k) {
  if (dropin_gather(4, out, tbl, sc, row, k) != FGM_HIP_OK) {
    fprintf(stderr, "fastgemma_amd: fgm_gather_q4r_hip: %s\n", fgm_hip_last_error());
    abort();
  }
}

}  // extern "C"
