// The engine's packed weight file (.qw) on MI355X: parse, validate, and upload into one resident hipMalloc
// region; plus the small runtime surface a host needs around the ops (streams, device memory, copies).
//
// File format (tools/convert.py:13-17, 49-89 writes it; engine/src/weights.mm:16-79 reads it):
//   "QWTS" | u32 version | u64 header_len | JSON header | zero pad to 16 KiB | tensor data
//   header = {"tensors": {name: {"dtype": "bf16"|"f32"|"f16"|"i8", "shape": [...], "offset": o,
//             "nbytes": n}}, "meta": {...}}; offsets are relative to the data start, 16 KiB aligned.
// The reference maps the file and wraps each name-prefix segment in a no-copy Metal buffer (unified
// memory). A discrete GPU needs the bytes in HBM: the whole data region goes into ONE device allocation
// (dit_q8.qw is ~13 GB, a small fraction of 288 GB), so every tensor keeps its file offset and a tensor's
// device address is base + offset. The copy streams through two pinned staging buffers: host threads fill
// one from the mapping while the DMA engine drains the other.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "kh_internal.h"

namespace {

constexpr size_t kAlign = 16384;  // tensor and data-start alignment of the format (convert.py ALIGN)

// ---- minimal JSON reader (objects, arrays, strings, numbers, literals) ----
struct JVal {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  bool integral = false;
  int64_t i = 0;
  double d = 0;
  std::string s;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
  const char *begin = nullptr, *end = nullptr;  // source span
  const JVal* get(const char* key) const {
    for (auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

struct JParser {
  const char *p, *e;
  std::string why;
  void ws() {
    while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++;
  }
  bool fail(const char* m) {
    if (why.empty()) why = m;
    return false;
  }
  static void put_utf8(std::string& out, uint32_t c) {
    if (c < 0x80) {
      out += (char)c;
    } else if (c < 0x800) {
      out += (char)(0xC0 | (c >> 6));
      out += (char)(0x80 | (c & 63));
    } else if (c < 0x10000) {
      out += (char)(0xE0 | (c >> 12));
      out += (char)(0x80 | ((c >> 6) & 63));
      out += (char)(0x80 | (c & 63));
    } else {
      out += (char)(0xF0 | (c >> 18));
      out += (char)(0x80 | ((c >> 12) & 63));
      out += (char)(0x80 | ((c >> 6) & 63));
      out += (char)(0x80 | (c & 63));
    }
  }
  bool hex4(uint32_t& c) {
    if (e - p < 4) return fail("truncated \\u escape");
    c = 0;
    for (int k = 0; k < 4; k++) {
      const char h = *p++;
      c <<= 4;
      if (h >= '0' && h <= '9') c |= h - '0';
      else if (h >= 'a' && h <= 'f') c |= h - 'a' + 10;
      else if (h >= 'A' && h <= 'F') c |= h - 'A' + 10;
      else return fail("bad \\u escape");
    }
    return true;
  }
  bool str(std::string& out) {
    if (p >= e || *p != '"') return fail("expected string");
    p++;
    while (p < e && *p != '"') {
      char c = *p++;
      if ((unsigned char)c < 0x20) return fail("control character in string");
      if (c != '\\') {
        out += c;
        continue;
      }
      if (p >= e) return fail("truncated escape");
      c = *p++;
      switch (c) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          uint32_t c1;
          if (!hex4(c1)) return false;
          if (c1 >= 0xD800 && c1 < 0xDC00 && e - p >= 6 && p[0] == '\\' && p[1] == 'u') {
            p += 2;
            uint32_t c2;
            if (!hex4(c2)) return false;
            if (c2 < 0xDC00 || c2 >= 0xE000) return fail("bad surrogate pair");
            c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
          }
          put_utf8(out, c1);
          break;
        }
        default: return fail("bad escape");
      }
    }
    if (p >= e) return fail("unterminated string");
    p++;
    return true;
  }
  bool num(JVal& v) {
    const char* s = p;
    if (p < e && *p == '-') p++;
    bool frac = false;
    while (p < e && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-')) {
      if (*p == '.' || *p == 'e' || *p == 'E') frac = true;
      p++;
    }
    if (p == s) return fail("expected value");
    const std::string t(s, p);
    char* endp = nullptr;
    v.kind = JVal::NUM;
    v.d = strtod(t.c_str(), &endp);
    if (*endp) return fail("bad number");
    if (!frac) {
      errno = 0;
      v.i = strtoll(t.c_str(), &endp, 10);
      if (errno || *endp) return fail("integer out of range");
      v.integral = true;
    }
    return true;
  }
  bool lit(const char* w, size_t n) {
    if ((size_t)(e - p) < n || memcmp(p, w, n)) return fail("bad literal");
    p += n;
    return true;
  }
  bool value(JVal& v, int depth) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (p >= e) return fail("unexpected end of header");
    v.begin = p;
    bool ok;
    switch (*p) {
      case '{': {
        v.kind = JVal::OBJ;
        p++;
        ws();
        ok = true;
        if (p < e && *p == '}') {
          p++;
          break;
        }
        for (;;) {
          ws();
          std::string k;
          if (!str(k)) return false;
          ws();
          if (p >= e || *p != ':') return fail("expected ':'");
          p++;
          v.obj.emplace_back(std::move(k), JVal());
          if (!value(v.obj.back().second, depth + 1)) return false;
          ws();
          if (p < e && *p == ',') {
            p++;
            continue;
          }
          if (p < e && *p == '}') {
            p++;
            break;
          }
          return fail("expected ',' or '}'");
        }
        break;
      }
      case '[': {
        v.kind = JVal::ARR;
        p++;
        ws();
        ok = true;
        if (p < e && *p == ']') {
          p++;
          break;
        }
        for (;;) {
          v.arr.emplace_back();
          if (!value(v.arr.back(), depth + 1)) return false;
          ws();
          if (p < e && *p == ',') {
            p++;
            continue;
          }
          if (p < e && *p == ']') {
            p++;
            break;
          }
          return fail("expected ',' or ']'");
        }
        break;
      }
      case '"':
        v.kind = JVal::STR;
        ok = str(v.s);
        break;
      case 't':
        v.kind = JVal::BOOL;
        v.b = true;
        ok = lit("true", 4);
        break;
      case 'f':
        v.kind = JVal::BOOL;
        ok = lit("false", 5);
        break;
      case 'n':
        ok = lit("null", 4);
        break;
      default:
        ok = num(v);
    }
    v.end = p;
    return ok;
  }
};

struct QwTensor {
  std::string name;
  int dtype;
  int ndim;
  int64_t shape[KH_QW_MAX_DIMS];
  size_t offset, nbytes;
};

int dtype_code(const std::string& s, size_t& esz) {
  if (s == "f32") return esz = 4, KH_F32;
  if (s == "f16") return esz = 2, KH_F16;
  if (s == "bf16") return esz = 2, KH_BF16;
  if (s == "i8") return esz = 1, KH_I8;
  return -1;
}

}  // namespace

struct kh_qw {
  std::string path;
  void* base = nullptr;  // read-only mapping of the whole file
  size_t map_size = 0, file_size = 0, data_start = 0, data_used = 0;
  uint32_t version = 0;
  std::string meta;
  std::vector<QwTensor> tensors;  // sorted by name
  std::unordered_map<std::string, int> index;
  char* dev = nullptr;  // resident copy of [data_start, data_start + data_used)
  int dev_id = -1;
};

namespace {

void fill(const kh_qw* f, int i, kh_qw_tensor* out) {
  const QwTensor& t = f->tensors[i];
  out->name = t.name.c_str();
  out->dtype = t.dtype;
  out->ndim = t.ndim;
  for (int d = 0; d < KH_QW_MAX_DIMS; d++) out->shape[d] = d < t.ndim ? t.shape[d] : 0;
  out->offset = t.offset;
  out->nbytes = t.nbytes;
  out->host = (const char*)f->base + f->data_start + t.offset;
  out->dev = f->dev ? f->dev + t.offset : nullptr;
}

int parse(kh_qw* f, kh::Err& e) {
  const char* p = (const char*)f->base;
  if (f->file_size < 16 || memcmp(p, "QWTS", 4) != 0) return e.fail("qw %s: bad magic", f->path.c_str());
  uint64_t hlen;
  memcpy(&f->version, p + 4, 4);
  memcpy(&hlen, p + 8, 8);
  if (hlen > f->file_size - 16) return e.fail("qw %s: header length %llu past the end", f->path.c_str(),
                                              (unsigned long long)hlen);
  f->data_start = (16 + hlen + kAlign - 1) / kAlign * kAlign;
  const size_t data_size = f->file_size > f->data_start ? f->file_size - f->data_start : 0;
  JParser jp{p + 16, p + 16 + hlen, {}};
  JVal root;
  if (!jp.value(root, 0)) return e.fail("qw %s: header JSON: %s", f->path.c_str(), jp.why.c_str());
  if (root.kind != JVal::OBJ) return e.fail("qw %s: header is not an object", f->path.c_str());
  if (const JVal* m = root.get("meta")) f->meta.assign(m->begin, m->end);
  else f->meta = "{}";
  const JVal* ts = root.get("tensors");
  if (!ts || ts->kind != JVal::OBJ) return e.fail("qw %s: no \"tensors\" object", f->path.c_str());
  for (auto& kv : ts->obj) {
    const JVal& d = kv.second;
    const char* n = kv.first.c_str();
    const JVal *dt = d.get("dtype"), *sh = d.get("shape"), *off = d.get("offset"), *nb = d.get("nbytes");
    if (d.kind != JVal::OBJ || !dt || !sh || !off || !nb || dt->kind != JVal::STR || sh->kind != JVal::ARR ||
        off->kind != JVal::NUM || !off->integral || nb->kind != JVal::NUM || !nb->integral)
      return e.fail("qw %s: malformed entry for tensor %s", f->path.c_str(), n);
    QwTensor t;
    t.name = kv.first;
    size_t esz = 0;
    t.dtype = dtype_code(dt->s, esz);
    if (t.dtype < 0) return e.fail("qw %s: tensor %s: unknown dtype \"%s\"", f->path.c_str(), n, dt->s.c_str());
    if (sh->arr.size() > KH_QW_MAX_DIMS) return e.fail("qw %s: tensor %s: more than %d dims", f->path.c_str(), n,
                                                       KH_QW_MAX_DIMS);
    t.ndim = (int)sh->arr.size();
    unsigned __int128 count = 1;
    for (int i = 0; i < t.ndim; i++) {
      const JVal& s = sh->arr[i];
      if (s.kind != JVal::NUM || !s.integral || s.i < 0) return e.fail("qw %s: tensor %s: bad shape", f->path.c_str(), n);
      t.shape[i] = s.i;
      count *= (uint64_t)s.i;
    }
    if (off->i < 0 || nb->i < 0) return e.fail("qw %s: tensor %s: negative offset / size", f->path.c_str(), n);
    t.offset = (size_t)off->i;
    t.nbytes = (size_t)nb->i;
    if (count * esz != (unsigned __int128)t.nbytes)
      return e.fail("qw %s: tensor %s: nbytes %zu != shape x %zu-byte elements", f->path.c_str(), n, t.nbytes, esz);
    if (t.offset > data_size || t.nbytes > data_size - t.offset)
      return e.fail("qw %s: tensor %s: bytes [%zu, %zu) past the end of the data (%zu)", f->path.c_str(), n, t.offset,
                    t.offset + t.nbytes, data_size);
    f->data_used = std::max(f->data_used, t.offset + t.nbytes);
    f->tensors.push_back(std::move(t));
  }
  std::sort(f->tensors.begin(), f->tensors.end(), [](const QwTensor& a, const QwTensor& b) { return a.name < b.name; });
  for (size_t i = 0; i < f->tensors.size(); i++) {
    if (!f->index.emplace(f->tensors[i].name, (int)i).second)
      return e.fail("qw %s: tensor %s listed twice", f->path.c_str(), f->tensors[i].name.c_str());
  }
  return KH_OK;
}

// host -> device through two pinned staging buffers; `threads` host threads fill a chunk in parallel
int upload_region(const char* src, char* dst, size_t n, hipStream_t st, kh::Err& e) {
  constexpr size_t CH = (size_t)64 << 20;
  const int threads = (int)std::max(1u, std::min(8u, std::thread::hardware_concurrency()));
  char* stage[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  int rc = KH_OK;
  hipError_t r = hipSuccess;
  for (int i = 0; i < 2 && r == hipSuccess; i++) {
    r = hipHostMalloc((void**)&stage[i], CH, hipHostMallocDefault);
    if (r == hipSuccess) r = hipEventCreateWithFlags(&done[i], hipEventDisableTiming);
  }
  if (r != hipSuccess) rc = e.hip(r, "qw upload: staging buffers");
  for (size_t off = 0, k = 0; rc == KH_OK && off < n; off += CH, k++) {
    const size_t len = std::min(CH, n - off);
    char* buf = stage[k & 1];
    if (k >= 2 && (r = hipEventSynchronize(done[k & 1])) != hipSuccess) {  // this buffer's previous copy
      rc = e.hip(r, "qw upload: wait");
      break;
    }
    const size_t part = (len + threads - 1) / threads;
    std::vector<std::thread> pool;
    for (int t = 1; t < threads; t++) {
      const size_t a = std::min(len, t * part), b = std::min(len, a + part);
      if (a < b) pool.emplace_back([=] { memcpy(buf + a, src + off + a, b - a); });
    }
    memcpy(buf, src + off, std::min(len, part));
    for (auto& th : pool) th.join();
    if ((r = hipMemcpyAsync(dst + off, buf, len, hipMemcpyHostToDevice, st)) != hipSuccess ||
        (r = hipEventRecord(done[k & 1], st)) != hipSuccess)
      rc = e.hip(r, "qw upload: copy");
  }
  if ((r = hipStreamSynchronize(st)) != hipSuccess && rc == KH_OK) rc = e.hip(r, "qw upload: sync");
  for (int i = 0; i < 2; i++) {
    if (done[i]) (void)hipEventDestroy(done[i]);
    if (stage[i]) (void)hipHostFree(stage[i]);
  }
  return rc;
}

}  // namespace

extern "C" {

kh_qw* kh_qw_open(const char* path, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  if (!path) return e.fail("qw: null path"), nullptr;
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return e.fail("qw: cannot open %s: %s", path, strerror(errno)), nullptr;
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size <= 0) {
    close(fd);
    return e.fail("qw: cannot stat %s (or empty)", path), nullptr;
  }
  kh_qw* f = new kh_qw;
  f->path = path;
  f->file_size = (size_t)st.st_size;
  const size_t page = (size_t)sysconf(_SC_PAGESIZE);
  f->map_size = (f->file_size + page - 1) / page * page;
  f->base = mmap(nullptr, f->map_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (f->base == MAP_FAILED) {
    f->base = nullptr;
    e.fail("qw: mmap of %s failed", path);
    delete f;
    return nullptr;
  }
  if (parse(f, e) != KH_OK) {
    kh_qw_close(f);
    return nullptr;
  }
  return f;
}

void kh_qw_close(kh_qw* f) {
  if (!f) return;
  if (f->dev) {
    int cur = -1;
    (void)hipGetDevice(&cur);
    (void)hipSetDevice(f->dev_id);
    (void)hipFree(f->dev);
    if (cur >= 0) (void)hipSetDevice(cur);
  }
  if (f->base) munmap(f->base, f->map_size);
  delete f;
}

int kh_qw_count(const kh_qw* f) { return f ? (int)f->tensors.size() : 0; }

unsigned kh_qw_version(const kh_qw* f) { return f ? f->version : 0; }

const char* kh_qw_meta(const kh_qw* f) { return f ? f->meta.c_str() : nullptr; }

int kh_qw_at(const kh_qw* f, int i, kh_qw_tensor* out) {
  if (!f || !out || i < 0 || i >= (int)f->tensors.size()) return KH_EINVAL;
  fill(f, i, out);
  return KH_OK;
}

int kh_qw_find(const kh_qw* f, const char* name, kh_qw_tensor* out) {
  if (!f || !name || !out) return KH_EINVAL;
  auto it = f->index.find(name);
  if (it == f->index.end()) return KH_EINVAL;
  fill(f, it->second, out);
  return KH_OK;
}

int kh_qw_upload(kh_qw* f, kh_stream stream, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  if (!f) return e.fail("qw upload: null file");
  if (f->dev) return KH_OK;
  hipError_t r = hipGetDevice(&f->dev_id);
  if (r != hipSuccess) return e.hip(r, "qw upload: no device");
  const size_t n = std::max<size_t>(f->data_used, 256);
  if ((r = hipMalloc((void**)&f->dev, n)) != hipSuccess) {
    f->dev = nullptr;
    return e.hip(r, "qw upload: hipMalloc");
  }
  madvise(f->base, f->map_size, MADV_SEQUENTIAL);
  const int rc = upload_region((const char*)f->base + f->data_start, f->dev, f->data_used, (hipStream_t)stream, e);
  if (rc != KH_OK) {
    (void)hipFree(f->dev);
    f->dev = nullptr;
  }
  return rc;
}

// ---- runtime surface: streams, device memory, copies ----
int kh_stream_create(kh_stream* out, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  if (!out) return e.fail("stream_create: null output");
  hipStream_t s = nullptr;
  const hipError_t r = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (r != hipSuccess) return e.hip(r, "hipStreamCreate");
  *out = (kh_stream)s;
  return KH_OK;
}

int kh_stream_destroy(kh_stream s) { return hipStreamDestroy((hipStream_t)s) == hipSuccess ? KH_OK : KH_EHIP; }

int kh_stream_sync(kh_stream s, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  const hipError_t r = hipStreamSynchronize((hipStream_t)s);
  return r == hipSuccess ? KH_OK : e.hip(r, "hipStreamSynchronize");
}

int kh_alloc(void** out, size_t bytes, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  if (!out) return e.fail("alloc: null output");
  *out = nullptr;
  const hipError_t r = hipMalloc(out, std::max<size_t>(bytes, 1));
  if (r != hipSuccess) {
    *out = nullptr;
    return e.hip(r, "hipMalloc");
  }
  return KH_OK;
}

int kh_free(void* p) { return hipFree(p) == hipSuccess ? KH_OK : KH_EHIP; }

int kh_upload(kh_stream s, void* dst, const void* src, size_t bytes, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  if (bytes && (!dst || !src)) return e.fail("upload: null pointer");
  hipError_t r = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)s);
  if (r == hipSuccess) r = hipStreamSynchronize((hipStream_t)s);
  return r == hipSuccess ? KH_OK : e.hip(r, "upload");
}

int kh_download(kh_stream s, void* dst, const void* src, size_t bytes, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  if (bytes && (!dst || !src)) return e.fail("download: null pointer");
  hipError_t r = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)s);
  if (r == hipSuccess) r = hipStreamSynchronize((hipStream_t)s);
  return r == hipSuccess ? KH_OK : e.hip(r, "download");
}

int kh_copy(kh_stream s, void* dst, const void* src, size_t bytes, char* err, int errlen) {
  kh::Err e{err, errlen};
  e.clear();
  if (bytes && (!dst || !src)) return e.fail("copy: null pointer");
  const uintptr_t d = (uintptr_t)dst, a = (uintptr_t)src;
  if (bytes && d < a + bytes && a < d + bytes && d != a) return e.fail("copy: overlapping ranges");
  const hipError_t r = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)s);
  return r == hipSuccess ? KH_OK : e.hip(r, "copy");
}

}  // extern "C"
