// safetensors.cpp -- reader for the safetensors files MLX checkpoints ship in
// (MLX 4-bit layout: u32-packed `.weight`, bf16/f16 `.scales`/`.biases`),
// the sharded-checkpoint index, and the quantized-key remapping of the
// reference loader (crates/higgs-models/src/lib.rs:574-723).
//
// Format: an 8-byte little-endian header length N, N bytes of JSON
//   { "<name>": {"dtype": "BF16", "shape": [..], "data_offsets": [begin, end]},
//     ..., "__metadata__": {..} }
// then the byte buffer; offsets are relative to the buffer start.
//
// The file is memory-mapped read-only. Device uploads go through two pinned
// staging buffers (hipHostMalloc) so the copy out of the page cache overlaps
// the DMA of the previous chunk; nothing is registered with the runtime.
#include <fcntl.h>
#include <hip/hip_runtime_api.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "../../include/higgs_hip.h"
#include "hgk_host.h"

namespace hgk {
namespace {

// ---------------------------------------------------------------- JSON
// A small recursive-descent JSON reader: enough for safetensors headers and
// model.safetensors.index.json (objects, arrays, strings with escapes,
// numbers, true/false/null). Numbers are kept as text and converted on use.
struct Json {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  std::string s;  // string value, or a number's text
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;

  const Json* get(const std::string& key) const {
    for (const auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

class JsonParser {
 public:
  JsonParser(const char* p, size_t n) : p_(p), end_(p + n) {}

  bool parse(Json* out, std::string* err) {
    if (!value(out, 0)) {
      *err = err_.empty() ? "malformed JSON" : err_;
      return false;
    }
    ws();
    if (p_ != end_) {
      *err = "trailing characters after JSON value";
      return false;
    }
    return true;
  }

 private:
  const char* p_;
  const char* end_;
  std::string err_;

  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool lit(const char* w) {
    const size_t n = std::strlen(w);
    if ((size_t)(end_ - p_) < n || std::memcmp(p_, w, n) != 0) return false;
    p_ += n;
    return true;
  }
  static void utf8(uint32_t cp, std::string* s) {
    if (cp < 0x80) {
      s->push_back((char)cp);
    } else if (cp < 0x800) {
      s->push_back((char)(0xC0 | (cp >> 6)));
      s->push_back((char)(0x80 | (cp & 0x3F)));
    } else if (cp < 0x10000) {
      s->push_back((char)(0xE0 | (cp >> 12)));
      s->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
      s->push_back((char)(0x80 | (cp & 0x3F)));
    } else {
      s->push_back((char)(0xF0 | (cp >> 18)));
      s->push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
      s->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
      s->push_back((char)(0x80 | (cp & 0x3F)));
    }
  }
  bool hex4(uint32_t* v) {
    if (end_ - p_ < 4) return false;
    *v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p_++;
      *v <<= 4;
      if (c >= '0' && c <= '9') *v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') *v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') *v |= (uint32_t)(c - 'A' + 10);
      else return false;
    }
    return true;
  }
  bool string(std::string* s) {
    if (p_ >= end_ || *p_ != '"') return false;
    ++p_;
    while (p_ < end_ && *p_ != '"') {
      const unsigned char c = (unsigned char)*p_;
      if (c < 0x20) return false;
      if (c != '\\') {
        s->push_back((char)c);
        ++p_;
        continue;
      }
      if (++p_ >= end_) return false;
      const char e = *p_++;
      switch (e) {
        case '"': s->push_back('"'); break;
        case '\\': s->push_back('\\'); break;
        case '/': s->push_back('/'); break;
        case 'b': s->push_back('\b'); break;
        case 'f': s->push_back('\f'); break;
        case 'n': s->push_back('\n'); break;
        case 'r': s->push_back('\r'); break;
        case 't': s->push_back('\t'); break;
        case 'u': {
          uint32_t cp;
          if (!hex4(&cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
            uint32_t lo;
            if (!lit("\\u") || !hex4(&lo) || lo < 0xDC00 || lo >= 0xE000) return false;
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(cp, s);
          break;
        }
        default: return false;
      }
    }
    if (p_ >= end_) return false;
    ++p_;
    return true;
  }
  bool number(std::string* s) {
    const char* b = p_;
    if (p_ < end_ && *p_ == '-') ++p_;
    if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return false;
    while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' ||
                         *p_ == '+' || *p_ == '-'))
      ++p_;
    s->assign(b, p_);
    return true;
  }
  bool value(Json* v, int depth) {
    if (depth > 64) {
      err_ = "JSON nested too deeply";
      return false;
    }
    ws();
    if (p_ >= end_) return false;
    const char c = *p_;
    if (c == '{') {
      v->kind = Json::Obj;
      ++p_;
      ws();
      if (p_ < end_ && *p_ == '}') {
        ++p_;
        return true;
      }
      for (;;) {
        ws();
        std::string key;
        if (!string(&key)) return false;
        ws();
        if (p_ >= end_ || *p_ != ':') return false;
        ++p_;
        Json child;
        if (!value(&child, depth + 1)) return false;
        v->obj.emplace_back(std::move(key), std::move(child));
        ws();
        if (p_ < end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < end_ && *p_ == '}') {
          ++p_;
          return true;
        }
        return false;
      }
    }
    if (c == '[') {
      v->kind = Json::Arr;
      ++p_;
      ws();
      if (p_ < end_ && *p_ == ']') {
        ++p_;
        return true;
      }
      for (;;) {
        Json child;
        if (!value(&child, depth + 1)) return false;
        v->arr.push_back(std::move(child));
        ws();
        if (p_ < end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < end_ && *p_ == ']') {
          ++p_;
          return true;
        }
        return false;
      }
    }
    if (c == '"') {
      v->kind = Json::Str;
      return string(&v->s);
    }
    if (lit("true")) { v->kind = Json::Bool; v->b = true; return true; }
    if (lit("false")) { v->kind = Json::Bool; v->b = false; return true; }
    if (lit("null")) { v->kind = Json::Null; return true; }
    v->kind = Json::Num;
    return number(&v->s);
  }
};

// A JSON number that is a non-negative integer below 2^63.
bool as_u63(const Json& j, int64_t* out) {
  if (j.kind != Json::Num || j.s.empty()) return false;
  uint64_t v = 0;
  for (char c : j.s) {
    if (c < '0' || c > '9') return false;
    if (v > (UINT64_C(1) << 62) / 5) return false;  // keeps v * 10 + 9 below 2^63
    v = v * 10 + (uint64_t)(c - '0');
  }
  *out = (int64_t)v;
  return true;
}

// ---------------------------------------------------------------- dtypes
struct DtypeInfo {
  const char* name;
  int code;   // hgk dtype code, or -1 for a type the kernels do not take
  int bytes;  // element size
};
const DtypeInfo kDtypes[] = {
    {"F32", HGK_F32, 4}, {"BF16", HGK_BF16, 2}, {"F16", HGK_F16, 2}, {"U32", HGK_U32, 4},
    {"I32", HGK_I32, 4}, {"F64", -1, 8},        {"I64", -1, 8},      {"U64", -1, 8},
    {"I16", -1, 2},      {"U16", -1, 2},        {"I8", -1, 1},       {"U8", -1, 1},
    {"BOOL", -1, 1},     {"F8_E4M3", -1, 1},    {"F8_E5M2", -1, 1},
};

const DtypeInfo* dtype_info(const std::string& s) {
  for (const auto& d : kDtypes)
    if (s == d.name) return &d;
  return nullptr;
}

}  // namespace

struct StTensor {
  std::string name;
  std::string dtype_name;
  int dtype = -1;
  int64_t itemsize = 0;
  std::vector<int64_t> shape;
  int64_t begin = 0, end = 0;  // byte offsets into the data buffer
};

}  // namespace hgk

struct hgk_st_file {
  std::string path;
  int fd = -1;
  const unsigned char* map = nullptr;
  size_t size = 0;
  const unsigned char* data = nullptr;  // start of the byte buffer
  size_t data_size = 0;
  std::vector<hgk::StTensor> tensors;   // in header order
  std::map<std::string, int64_t> index;
  std::vector<std::pair<std::string, std::string>> metadata;
};

namespace hgk {
namespace {

void st_free(hgk_st_file* f) {
  if (!f) return;
  if (f->map) munmap((void*)f->map, f->size);
  if (f->fd >= 0) close(f->fd);
  delete f;
}

int st_parse(hgk_st_file* f) {
  const char* fn = "hgk_st_open";
  if (f->size < 8) return fail(HGK_ERR_ARG, "%s: %s is too small for a safetensors header", fn, f->path.c_str());
  uint64_t n = 0;
  for (int i = 7; i >= 0; --i) n = (n << 8) | f->map[i];
  if (n > f->size - 8)
    return fail(HGK_ERR_ARG, "%s: %s: header length %llu exceeds the file", fn, f->path.c_str(),
                (unsigned long long)n);
  Json root;
  std::string err;
  JsonParser jp(reinterpret_cast<const char*>(f->map + 8), (size_t)n);
  if (!jp.parse(&root, &err) || root.kind != Json::Obj)
    return fail(HGK_ERR_ARG, "%s: %s: header is not a JSON object (%s)", fn, f->path.c_str(),
                err.empty() ? "not an object" : err.c_str());
  f->data = f->map + 8 + n;
  f->data_size = f->size - 8 - (size_t)n;
  for (const auto& kv : root.obj) {
    if (kv.first == "__metadata__") {
      if (kv.second.kind != Json::Obj)
        return fail(HGK_ERR_ARG, "%s: %s: __metadata__ is not an object", fn, f->path.c_str());
      for (const auto& m : kv.second.obj)
        f->metadata.emplace_back(m.first, m.second.kind == Json::Str ? m.second.s : std::string());
      continue;
    }
    const Json& t = kv.second;
    const Json* dt = t.get("dtype");
    const Json* sh = t.get("shape");
    const Json* off = t.get("data_offsets");
    if (t.kind != Json::Obj || !dt || dt->kind != Json::Str || !sh || sh->kind != Json::Arr || !off ||
        off->kind != Json::Arr || off->arr.size() != 2)
      return fail(HGK_ERR_ARG, "%s: %s: tensor '%s' lacks dtype/shape/data_offsets", fn,
                  f->path.c_str(), kv.first.c_str());
    StTensor st;
    st.name = kv.first;
    st.dtype_name = dt->s;
    const DtypeInfo* di = dtype_info(dt->s);
    if (!di)
      return fail(HGK_ERR_ARG, "%s: %s: tensor '%s' has unknown dtype '%s'", fn, f->path.c_str(),
                  kv.first.c_str(), dt->s.c_str());
    st.dtype = di->code;
    st.itemsize = di->bytes;
    int64_t numel = 1;
    for (const auto& d : sh->arr) {
      int64_t v;
      if (!as_u63(d, &v))
        return fail(HGK_ERR_ARG, "%s: %s: tensor '%s' has a bad shape", fn, f->path.c_str(),
                    kv.first.c_str());
      if (v != 0 && numel > INT64_MAX / v)
        return fail(HGK_ERR_ARG, "%s: %s: tensor '%s' is too large", fn, f->path.c_str(), kv.first.c_str());
      numel *= v;
      st.shape.push_back(v);
    }
    if (st.shape.size() > 8)
      return fail(HGK_ERR_UNSUPPORTED, "%s: %s: tensor '%s' has more than 8 dimensions", fn,
                  f->path.c_str(), kv.first.c_str());
    if (!as_u63(off->arr[0], &st.begin) || !as_u63(off->arr[1], &st.end) || st.begin > st.end ||
        (uint64_t)st.end > f->data_size)
      return fail(HGK_ERR_ARG, "%s: %s: tensor '%s' has data offsets outside the buffer", fn,
                  f->path.c_str(), kv.first.c_str());
    if (numel > INT64_MAX / st.itemsize || st.end - st.begin != numel * st.itemsize)
      return fail(HGK_ERR_ARG, "%s: %s: tensor '%s' holds %lld bytes, its shape needs %lld", fn,
                  f->path.c_str(), kv.first.c_str(), (long long)(st.end - st.begin),
                  (long long)(numel * st.itemsize));
    if (!f->index.emplace(st.name, (int64_t)f->tensors.size()).second)
      return fail(HGK_ERR_ARG, "%s: %s: tensor '%s' appears twice", fn, f->path.c_str(), kv.first.c_str());
    f->tensors.push_back(std::move(st));
  }
  // the buffer is covered by the tensors without overlaps (as the format requires)
  std::vector<std::pair<int64_t, int64_t>> spans;
  for (const auto& t : f->tensors) spans.emplace_back(t.begin, t.end);
  std::sort(spans.begin(), spans.end());
  int64_t pos = 0;
  for (const auto& sp : spans) {
    if (sp.first != pos)
      return fail(HGK_ERR_ARG, "%s: %s: tensor data %s at byte %lld", fn, f->path.c_str(),
                  sp.first < pos ? "overlaps" : "leaves a gap", (long long)sp.first);
    pos = sp.second;
  }
  if ((uint64_t)pos != f->data_size)
    return fail(HGK_ERR_ARG, "%s: %s: %llu trailing bytes after the last tensor", fn,
                f->path.c_str(), (unsigned long long)(f->data_size - (uint64_t)pos));
  return HGK_OK;
}

const StTensor* st_at(const hgk_st_file* f, int64_t i, const char* fn) {
  if (!f) {
    fail(HGK_ERR_ARG, "%s: null file", fn);
    return nullptr;
  }
  if (i < 0 || i >= (int64_t)f->tensors.size()) {
    fail(HGK_ERR_ARG, "%s: index %lld out of range (%zu tensors)", fn, (long long)i, f->tensors.size());
    return nullptr;
  }
  return &f->tensors[(size_t)i];
}

// Two pinned staging buffers per process, allocated on first use and kept
// (pinned allocations are expensive); uploads hold the mutex for their
// duration, so concurrent uploads from several threads are serialised.
constexpr size_t kStage = size_t(32) << 20;
std::mutex g_stage_mu;
void* g_stage[2] = {nullptr, nullptr};
hipEvent_t g_stage_ev[2] = {nullptr, nullptr};

bool exists(const std::string& p) {
  struct stat sb;
  return ::stat(p.c_str(), &sb) == 0;
}

}  // namespace
}  // namespace hgk

using namespace hgk;

extern "C" int hgk_st_open(const char* path, hgk_st_file** out) {
  clear_error();
  if (!path || !out) return fail(HGK_ERR_ARG, "hgk_st_open: null argument");
  *out = nullptr;
  std::unique_ptr<hgk_st_file, void (*)(hgk_st_file*)> f(new hgk_st_file(), st_free);
  f->path = path;
  f->fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (f->fd < 0) return fail(HGK_ERR_ARG, "hgk_st_open: cannot open %s: %s", path, std::strerror(errno));
  struct stat sb;
  if (fstat(f->fd, &sb) != 0) return fail(HGK_ERR_ARG, "hgk_st_open: cannot stat %s", path);
  f->size = (size_t)sb.st_size;
  if (f->size > 0) {
    void* m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
    if (m == MAP_FAILED) return fail(HGK_ERR_ARG, "hgk_st_open: cannot map %s: %s", path, std::strerror(errno));
    f->map = static_cast<const unsigned char*>(m);
  }
  const int st = st_parse(f.get());
  if (st) return st;
  *out = f.release();
  return HGK_OK;
}

extern "C" void hgk_st_close(hgk_st_file* f) { st_free(f); }

extern "C" int64_t hgk_st_count(const hgk_st_file* f) { return f ? (int64_t)f->tensors.size() : -1; }

extern "C" int hgk_st_find(const hgk_st_file* f, const char* name, int64_t* index) {
  clear_error();
  if (!f || !name || !index) return fail(HGK_ERR_ARG, "hgk_st_find: null argument");
  const auto it = f->index.find(name);
  if (it == f->index.end()) return fail(HGK_ERR_ARG, "hgk_st_find: no tensor '%s' in %s", name, f->path.c_str());
  *index = it->second;
  return HGK_OK;
}

extern "C" int hgk_st_tensor(const hgk_st_file* f, int64_t index, const char** name,
                             const char** dtype_name, int* dtype, int* ndim, int64_t shape[8],
                             int64_t* nbytes) {
  clear_error();
  const StTensor* t = st_at(f, index, "hgk_st_tensor");
  if (!t) return HGK_ERR_ARG;
  if (name) *name = t->name.c_str();
  if (dtype_name) *dtype_name = t->dtype_name.c_str();
  if (dtype) *dtype = t->dtype;
  if (ndim) *ndim = (int)t->shape.size();
  if (shape)
    for (size_t i = 0; i < t->shape.size(); ++i) shape[i] = t->shape[i];
  if (nbytes) *nbytes = t->end - t->begin;
  return HGK_OK;
}

extern "C" int hgk_st_copy_to_host(const hgk_st_file* f, int64_t index, void* dst, int64_t dst_bytes) {
  clear_error();
  const StTensor* t = st_at(f, index, "hgk_st_copy_to_host");
  if (!t) return HGK_ERR_ARG;
  const int64_t n = t->end - t->begin;
  if (!dst && n > 0) return fail(HGK_ERR_ARG, "hgk_st_copy_to_host: null destination");
  if (dst_bytes < n)
    return fail(HGK_ERR_ARG, "hgk_st_copy_to_host: '%s' needs %lld bytes, %lld given", t->name.c_str(),
                (long long)n, (long long)dst_bytes);
  if (n) std::memcpy(dst, f->data + t->begin, (size_t)n);
  return HGK_OK;
}

extern "C" int hgk_st_upload(const hgk_st_file* f, int64_t index, void* dst, int64_t dst_bytes,
                             void* stream) {
  clear_error();
  const char* fn = "hgk_st_upload";
  const StTensor* t = st_at(f, index, fn);
  if (!t) return HGK_ERR_ARG;
  const int64_t n = t->end - t->begin;
  if (!dst && n > 0) return fail(HGK_ERR_ARG, "%s: null destination", fn);
  if (dst_bytes < n)
    return fail(HGK_ERR_ARG, "%s: '%s' needs %lld bytes, %lld given", fn, t->name.c_str(),
                (long long)n, (long long)dst_bytes);
  if (n == 0) return HGK_OK;
  const hipStream_t s = as_stream(stream);
  std::lock_guard<std::mutex> lock(g_stage_mu);
  for (int i = 0; i < 2; ++i) {
    if (!g_stage[i]) {
      if (hipHostMalloc(&g_stage[i], kStage, hipHostMallocDefault) != hipSuccess) {
        g_stage[i] = nullptr;
        return fail(HGK_ERR_HIP, "%s: cannot allocate %zu MiB of pinned staging memory", fn, kStage >> 20);
      }
    }
    if (!g_stage_ev[i] && hipEventCreateWithFlags(&g_stage_ev[i], hipEventDisableTiming) != hipSuccess) {
      g_stage_ev[i] = nullptr;
      return fail(HGK_ERR_HIP, "%s: hipEventCreate failed", fn);
    }
  }
  // chunk k is staged in buffer k % 2; before refilling a buffer, wait for
  // the copy that last read it
  const unsigned char* src = f->data + t->begin;
  bool used[2] = {false, false};
  // On an error part-way, copies already queued may still read the staging
  // buffers, which the next call refills: wait for the whole stream before
  // returning, so no exit leaves a copy in flight.
  auto drain_fail = [&](const char* what) {
    (void)hipStreamSynchronize(s);
    return fail(HGK_ERR_HIP, "%s: %s for '%s'", fn, what, t->name.c_str());
  };
  for (int64_t off = 0, k = 0; off < n; off += (int64_t)kStage, ++k) {
    const int bi = (int)(k & 1);
    const size_t len = (size_t)std::min<int64_t>((int64_t)kStage, n - off);
    if (used[bi] && hipEventSynchronize(g_stage_ev[bi]) != hipSuccess)
      return drain_fail("hipEventSynchronize failed");
    std::memcpy(g_stage[bi], src + off, len);
    if (hipMemcpyAsync(static_cast<char*>(dst) + off, g_stage[bi], len, hipMemcpyDefault, s) != hipSuccess)
      return drain_fail("hipMemcpyAsync failed");
    if (hipEventRecord(g_stage_ev[bi], s) != hipSuccess) return drain_fail("hipEventRecord failed");
    used[bi] = true;
  }
  // the staging buffers are reused by the next call: wait for the last copies
  for (int i = 0; i < 2; ++i)
    if (used[i] && hipEventSynchronize(g_stage_ev[i]) != hipSuccess)
      return drain_fail("hipEventSynchronize failed");
  return HGK_OK;
}

extern "C" int hgk_st_collect_files(const char* model_dir, char* out, int64_t cap, int64_t* needed) {
  clear_error();
  const char* fn = "hgk_st_collect_files";
  if (!model_dir) return fail(HGK_ERR_ARG, "%s: null model_dir", fn);
  const std::string dir = model_dir;
  const std::string index_path = dir + "/model.safetensors.index.json";
  std::vector<std::string> files;
  if (exists(index_path)) {
    int fd = ::open(index_path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(HGK_ERR_ARG, "%s: cannot open %s", fn, index_path.c_str());
    std::string text;
    char buf[65536];
    for (;;) {
      const ssize_t r = ::read(fd, buf, sizeof buf);
      if (r < 0) {
        close(fd);
        return fail(HGK_ERR_ARG, "%s: cannot read %s", fn, index_path.c_str());
      }
      if (r == 0) break;
      text.append(buf, (size_t)r);
    }
    close(fd);
    Json root;
    std::string err;
    JsonParser jp(text.data(), text.size());
    if (!jp.parse(&root, &err) || root.kind != Json::Obj)
      return fail(HGK_ERR_ARG, "%s: %s is not a JSON object (%s)", fn, index_path.c_str(), err.c_str());
    const Json* wm = root.get("weight_map");
    if (!wm || wm->kind != Json::Obj)
      return fail(HGK_ERR_ARG, "%s: %s has no weight_map object", fn, index_path.c_str());
    std::set<std::string> uniq;
    for (const auto& kv : wm->obj) {
      if (kv.second.kind != Json::Str)
        return fail(HGK_ERR_ARG, "%s: weight_map['%s'] is not a file name", fn, kv.first.c_str());
      if (kv.second.s.find('/') != std::string::npos || kv.second.s == ".." || kv.second.s.empty())
        return fail(HGK_ERR_ARG, "%s: weight_map['%s'] = '%s' is not a file in the model directory",
                    fn, kv.first.c_str(), kv.second.s.c_str());
      uniq.insert(kv.second.s);
    }
    for (const auto& s : uniq) files.push_back(dir + "/" + s);
  } else if (exists(dir + "/model.safetensors")) {
    files.push_back(dir + "/model.safetensors");
  } else {
    return fail(HGK_ERR_ARG, "%s: MissingWeight: no safetensors files found in %s", fn, dir.c_str());
  }
  std::string joined;
  for (const auto& s : files) {
    joined += s;
    joined += '\n';
  }
  if (needed) *needed = (int64_t)joined.size() + 1;
  if (!out || cap < (int64_t)joined.size() + 1)
    return out ? fail(HGK_ERR_ARG, "%s: output buffer holds %lld bytes, %zu needed", fn,
                      (long long)cap, joined.size() + 1)
               : HGK_OK;
  std::memcpy(out, joined.c_str(), joined.size() + 1);
  return HGK_OK;
}

extern "C" int hgk_remap_quantized_key(const char* key, char* out, int64_t cap) {
  clear_error();
  if (!key || !out) return fail(HGK_ERR_ARG, "hgk_remap_quantized_key: null argument");
  const std::string k = key;
  static const char* const kSuffix[] = {".weight", ".scales", ".biases", ".bias"};
  for (const char* sfx : kSuffix) {
    const size_t n = std::strlen(sfx);
    if (k.size() >= n && k.compare(k.size() - n, n, sfx) == 0) {
      const std::string r = k.substr(0, k.size() - n) + ".inner" + sfx;
      if ((int64_t)r.size() + 1 > cap)
        return fail(HGK_ERR_ARG, "hgk_remap_quantized_key: output buffer too small");
      std::memcpy(out, r.c_str(), r.size() + 1);
      return HGK_OK;
    }
  }
  if (cap > 0) out[0] = '\0';
  return HGK_ERR_UNSUPPORTED;  // no quantized form for this key
}
