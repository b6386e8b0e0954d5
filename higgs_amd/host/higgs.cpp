// higgs.cpp -- the C++ host API (higgs.hpp) over the C ABI of libhiggs_hip.so.
// Shape handling, result allocation and error reporting live here; every op's
// arithmetic runs in the HIP kernels behind the C ABI.
#include "higgs.hpp"

#include <cmath>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <sstream>

namespace higgs {

// ------------------------------------------------------------------ dtypes
std::size_t size_of(Dtype dt) {
  switch (dt) {
    case Dtype::Bfloat16:
    case Dtype::Float16:
      return 2;
    case Dtype::Float32:
    case Dtype::Uint32:
    case Dtype::Int32:
      return 4;
  }
  throw Exception::custom("unknown dtype");
}

const char* name_of(Dtype dt) {
  switch (dt) {
    case Dtype::Float32: return "Float32";
    case Dtype::Bfloat16: return "Bfloat16";
    case Dtype::Float16: return "Float16";
    case Dtype::Uint32: return "Uint32";
    case Dtype::Int32: return "Int32";
  }
  return "?";
}

bool is_floating(Dtype dt) {
  return dt == Dtype::Float32 || dt == Dtype::Bfloat16 || dt == Dtype::Float16;
}

Dtype promote(Dtype a, Dtype b) { return a == b ? a : Dtype::Float32; }

std::string format_shape(const Shape& s) {
  std::ostringstream o;
  o << '[';
  for (std::size_t i = 0; i < s.size(); ++i) o << (i ? ", " : "") << s[i];
  o << ']';
  return o.str();
}

namespace {

// Round-to-nearest-even conversions for host uploads and readback.
uint16_t f32_to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

float bf16_to_f32(uint16_t b) {
  uint32_t u = static_cast<uint32_t>(b) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

uint16_t f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return static_cast<uint16_t>(sign | 0x7e00u);
  if (ax >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);  // >= 65520 -> inf
  if (ax < 0x38800000u) {  // below 2^-14: the f16 value is round(|f| * 2^24) ulps
    float af;
    std::memcpy(&af, &ax, 4);
    return static_cast<uint16_t>(sign | static_cast<uint32_t>(std::nearbyint(af * 16777216.0f)));
  }
  uint32_t r = ax + 0xfffu + ((ax >> 13) & 1u);  // round at bit 13, ties to even
  r -= 0x38000000u;                              // exponent bias 127 -> 15
  return static_cast<uint16_t>(sign | (r >> 13));
}

float f16_to_f32(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  float v;
  if (e == 0) {
    v = std::ldexp(static_cast<float>(m), -24);
    uint32_t u;
    std::memcpy(&u, &v, 4);
    u |= sign;
    std::memcpy(&v, &u, 4);
    return v;
  }
  uint32_t u = e == 31 ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
  std::memcpy(&v, &u, 4);
  return v;
}

thread_local Stream t_current;

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess)
    throw Exception(HGK_ERR_HIP, std::string(what) + " failed: " + hipGetErrorString(e));
}

using Operands = std::initializer_list<std::pair<const char*, const Array*>>;

std::string operands_text(Operands ops) {
  std::ostringstream o;
  o << '[';
  bool first = true;
  for (const auto& p : ops) {
    if (!p.second) continue;
    o << (first ? "" : " ") << p.first << '=' << p.second->describe();
    first = false;
  }
  o << ']';
  return o.str();
}

[[noreturn]] void fail(const char* op, const std::string& msg, Operands ops) {
  throw Exception::custom(std::string(op) + " failed: " + msg + " " + operands_text(ops));
}

void check(int status, const char* op, Operands ops) {
  if (status == HGK_OK) return;
  const char* m = hgk_last_error();
  throw Exception(status, std::string(op) + " failed: " + (m ? m : "") + " " + operands_text(ops));
}

void* stream_arg() { return reinterpret_cast<void*>(Stream::task_local_or_default().get()); }

struct Rows {
  int64_t rows, n, row_stride;
};

// x viewed as [rows, n] with unit stride along n and one stride between rows.
bool as_rows(const Array& x, Rows* r) {
  if (x.ndim() == 0) return false;
  const Shape& s = x.shape();
  const Shape& st = x.strides();
  const int nd = x.ndim();
  const int64_t n = s[nd - 1];
  if (n > 1 && st[nd - 1] != 1) return false;
  if (nd == 1) {
    *r = {1, n, n};
    return true;
  }
  // leading axes collapse when each one's stride is the next one's span
  int64_t rows = 1, rs = 0;
  bool have = false;
  for (int i = nd - 2; i >= 0; --i) {
    if (s[i] == 1) continue;
    if (!have) {
      rs = st[i];
      have = true;
    } else if (st[i] != rows * rs) {
      return false;
    }
    rows *= s[i];
  }
  if (!have) rs = n;
  *r = {rows, n, rs};
  return true;
}

Rows rows_of(const Array& x, const char* op, Operands ops) {
  Rows r;
  if (!as_rows(x, &r))
    fail(op, "operand is not expressible as rows with a unit-stride last axis", ops);
  return r;
}

}  // namespace

// ------------------------------------------------------------------ Stream
Stream Stream::create() {
  hipStream_t s = nullptr;
  hip_check(hipStreamCreate(&s), "hipStreamCreate");
  Stream out(s);
  out.owner_ = std::shared_ptr<void>(s, [](void* p) { (void)hipStreamDestroy(static_cast<hipStream_t>(p)); });
  return out;
}

Stream Stream::task_local_or_default() { return t_current; }

void Stream::synchronize() const { check(hgk_sync(reinterpret_cast<void*>(s_)), "synchronize", {}); }

StreamScope::StreamScope(const Stream& s) : prev_(t_current) { t_current = s; }
StreamScope::~StreamScope() { t_current = prev_; }

// ------------------------------------------------------------------ Buffer
namespace detail {
// A stream-ordered device allocation. It holds the Stream it was allocated on
// (with that stream's owner, so the stream outlives the allocation) and every
// other stream that has used it; the free is ordered after the work already
// queued on each of those streams, so memory read by an op on another stream
// is not handed out again while that op may still run.
struct Buffer {
  void* ptr = nullptr;
  std::size_t bytes = 0;
  Stream stream;
  std::mutex mu;
  std::vector<Stream> users;  // streams other than `stream` that used the buffer
  Buffer(std::size_t n, const Stream& s) : bytes(n), stream(s) {
    if (n) hip_check(hipMallocAsync(&ptr, n, s.get()), "hipMallocAsync");
  }
  void note_use(const Stream& s) {
    if (s.get() == stream.get()) return;
    std::lock_guard<std::mutex> g(mu);
    for (const Stream& u : users)
      if (u.get() == s.get()) return;
    users.push_back(s);
  }
  ~Buffer() {
    if (!ptr) return;
    for (const Stream& u : users) {
      hipEvent_t ev = nullptr;
      bool ordered = false;
      if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) == hipSuccess) {
        ordered = hipEventRecord(ev, u.get()) == hipSuccess &&
                  hipStreamWaitEvent(stream.get(), ev, 0) == hipSuccess;
        (void)hipEventDestroy(ev);
      }
      if (!ordered) (void)hipStreamSynchronize(u.get());
    }
    (void)hipFreeAsync(ptr, stream.get());
  }
  Buffer(const Buffer&) = delete;
  Buffer& operator=(const Buffer&) = delete;
};
}  // namespace detail

// ------------------------------------------------------------------ Array
static Shape row_major(const Shape& shape) {
  Shape st(shape.size());
  int64_t acc = 1;
  for (int i = static_cast<int>(shape.size()) - 1; i >= 0; --i) {
    st[i] = acc;
    acc *= shape[i];
  }
  return st;
}

static int64_t numel(const Shape& s) {
  int64_t n = 1;
  for (int64_t d : s) {
    if (d < 0) throw Exception::custom("negative dimension in shape " + format_shape(s));
    n *= d;
  }
  return n;
}

Array Array::empty(const Shape& shape, Dtype dt) {
  Array a;
  a.shape_ = shape;
  a.strides_ = row_major(shape);
  a.dtype_ = dt;
  a.buf_ = std::make_shared<detail::Buffer>(static_cast<std::size_t>(numel(shape)) * size_of(dt),
                                            Stream::task_local_or_default());
  return a;
}

static Array upload(const void* host, std::size_t bytes, const Shape& shape, Dtype dt) {
  Array a = Array::empty(shape, dt);
  if (bytes) {
    hipStream_t s = Stream::task_local_or_default().get();
    hip_check(hipMemcpyAsync(a.data(), host, bytes, hipMemcpyHostToDevice, s), "hipMemcpyAsync");
    hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
  }
  return a;
}

static void check_count(std::size_t n, const Shape& shape) {
  if (static_cast<int64_t>(n) != numel(shape))
    throw Exception::custom("from_slice: " + std::to_string(n) + " values for shape " +
                            format_shape(shape));
}

Array Array::from_slice(const float* data, std::size_t n, const Shape& shape, Dtype dt) {
  check_count(n, shape);
  if (dt == Dtype::Float32) return upload(data, n * 4, shape, dt);
  if (dt != Dtype::Bfloat16 && dt != Dtype::Float16)
    throw Exception::custom(std::string("from_slice: float data cannot become ") + name_of(dt));
  std::vector<uint16_t> bits(n);
  for (std::size_t i = 0; i < n; ++i)
    bits[i] = dt == Dtype::Bfloat16 ? f32_to_bf16(data[i]) : f32_to_f16(data[i]);
  return upload(bits.data(), n * 2, shape, dt);
}

Array Array::from_slice(const int32_t* data, std::size_t n, const Shape& shape) {
  check_count(n, shape);
  return upload(data, n * 4, shape, Dtype::Int32);
}

Array Array::from_slice(const uint32_t* data, std::size_t n, const Shape& shape) {
  check_count(n, shape);
  return upload(data, n * 4, shape, Dtype::Uint32);
}

Array Array::from_bits(const uint16_t* bits, std::size_t n, const Shape& shape, Dtype dt) {
  check_count(n, shape);
  if (size_of(dt) != 2) throw Exception::custom("from_bits: needs a 16-bit dtype");
  return upload(bits, n * 2, shape, dt);
}

int64_t Array::dim(int axis) const {
  const int nd = ndim();
  const int a = axis < 0 ? axis + nd : axis;
  if (a < 0 || a >= nd)
    throw Exception::custom("axis " + std::to_string(axis) + " out of range for " + describe());
  return shape_[a];
}

int64_t Array::size() const { return numel(shape_); }

bool Array::is_contiguous() const { return strides_ == row_major(shape_) || size() <= 1; }

void* Array::data() const {
  if (!buf_ || !buf_->ptr) return nullptr;
  // every device access goes through here, on the calling thread's stream
  buf_->note_use(Stream::task_local_or_default());
  return static_cast<char*>(buf_->ptr) + offset_ * static_cast<int64_t>(itemsize());
}

Array Array::transpose(const std::vector<int>& axes) const {
  if (static_cast<int>(axes.size()) != ndim())
    throw Exception::custom("transpose: axes do not match " + describe());
  Array v = *this;
  std::vector<bool> seen(axes.size(), false);
  for (std::size_t i = 0; i < axes.size(); ++i) {
    const int a = axes[i] < 0 ? axes[i] + ndim() : axes[i];
    if (a < 0 || a >= ndim() || seen[a]) throw Exception::custom("transpose: bad axes");
    seen[a] = true;
    v.shape_[i] = shape_[a];
    v.strides_[i] = strides_[a];
  }
  return v;
}

Array Array::slice(int axis, int64_t start, int64_t stop) const {
  const int a = axis < 0 ? axis + ndim() : axis;
  if (a < 0 || a >= ndim() || start < 0 || stop < start || stop > shape_[a])
    throw Exception::custom("slice out of range for " + describe());
  Array v = *this;
  v.offset_ += start * strides_[a];
  v.shape_[a] = stop - start;
  return v;
}

// Strides for viewing (dims, strides) as `nd` without a copy, when each run of
// old axes that merges into (or splits across) new axes is itself row-major.
static bool view_strides(const Shape& dims, const Shape& strides, const Shape& nd, Shape* ns) {
  Shape od, os;
  for (std::size_t i = 0; i < dims.size(); ++i)
    if (dims[i] != 1) {
      od.push_back(dims[i]);
      os.push_back(strides[i]);
    }
  const int on = static_cast<int>(od.size()), nn = static_cast<int>(nd.size());
  ns->assign(nn, 1);
  int oi = 0, oj = 1, ni = 0, nj = 1;
  while (ni < nn && oi < on) {
    int64_t np = nd[ni], op = od[oi];
    while (np != op) {
      if (np < op) np *= nd[nj++];
      else op *= od[oj++];
    }
    for (int k = oi; k < oj - 1; ++k)
      if (os[k] != od[k + 1] * os[k + 1]) return false;
    (*ns)[nj - 1] = os[oj - 1];
    for (int k = nj - 1; k > ni; --k) (*ns)[k - 1] = (*ns)[k] * nd[k];
    ni = nj++;
    oi = oj++;
  }
  return true;
}

Array Array::reshape(const Shape& shape) const {
  if (numel(shape) != size())
    throw Exception::custom("reshape: " + format_shape(shape) + " does not match " + describe());
  Array v = *this;
  v.shape_ = shape;
  if (size() == 0 || is_contiguous()) {
    v.strides_ = row_major(shape);
  } else if (!view_strides(shape_, strides_, shape, &v.strides_)) {
    throw Exception::custom("reshape: " + describe() + " cannot be viewed as " +
                            format_shape(shape) + " without a copy");
  }
  return v;
}

std::string Array::describe() const { return format_shape(shape_) + "/" + name_of(dtype_); }

void Array::gather_host(void* out) const {
  const int64_t n = size();
  if (n == 0) return;
  // the span of buffer elements the view touches
  int64_t hi = 0;
  for (int i = 0; i < ndim(); ++i) {
    if (strides_[i] < 0) throw Exception::custom("readback: negative strides are not supported");
    hi += (shape_[i] - 1) * strides_[i];
  }
  const std::size_t isz = itemsize();
  std::vector<unsigned char> span(static_cast<std::size_t>(hi + 1) * isz);
  hipStream_t s = Stream::task_local_or_default().get();
  hip_check(hipMemcpyAsync(span.data(), data(), span.size(), hipMemcpyDeviceToHost, s),
            "hipMemcpyAsync");
  hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
  std::vector<int64_t> idx(ndim(), 0);
  unsigned char* o = static_cast<unsigned char*>(out);
  for (int64_t e = 0; e < n; ++e) {
    int64_t off = 0;
    for (int i = 0; i < ndim(); ++i) off += idx[i] * strides_[i];
    std::memcpy(o + e * isz, span.data() + off * isz, isz);
    for (int i = ndim() - 1; i >= 0; --i) {
      if (++idx[i] < shape_[i]) break;
      idx[i] = 0;
    }
  }
}

std::vector<float> Array::to_f32() const {
  const int64_t n = size();
  std::vector<float> out(n);
  if (dtype_ == Dtype::Float32) {
    gather_host(out.data());
    return out;
  }
  if (size_of(dtype_) == 2) {
    std::vector<uint16_t> b(n);
    gather_host(b.data());
    for (int64_t i = 0; i < n; ++i)
      out[i] = dtype_ == Dtype::Bfloat16 ? bf16_to_f32(b[i]) : f16_to_f32(b[i]);
    return out;
  }
  std::vector<uint32_t> w(n);
  gather_host(w.data());
  for (int64_t i = 0; i < n; ++i)
    out[i] = dtype_ == Dtype::Int32 ? static_cast<float>(static_cast<int32_t>(w[i]))
                                    : static_cast<float>(w[i]);
  return out;
}

std::vector<uint16_t> Array::to_bits() const {
  if (size_of(dtype_) != 2) throw Exception::custom("to_bits: needs a 16-bit dtype");
  std::vector<uint16_t> b(size());
  gather_host(b.data());
  return b;
}

std::vector<uint32_t> Array::to_u32() const {
  if (size_of(dtype_) != 4) throw Exception::custom("to_u32: needs a 32-bit dtype");
  std::vector<uint32_t> w(size());
  gather_host(w.data());
  return w;
}

float Array::item() const {
  if (size() != 1) throw Exception::custom("item: array has " + std::to_string(size()) + " elements");
  return to_f32()[0];
}

// ------------------------------------------------------------------ RoPE tables
std::vector<float> rope_inv_freq(float base, int dims, const std::vector<float>* freqs) {
  if (dims < 2 || dims % 2) throw Exception::custom("rope_inv_freq: dims must be even and >= 2");
  if (freqs && static_cast<int>(freqs->size()) != dims / 2)
    throw Exception::custom("rope_inv_freq: freqs must hold dims/2 values");
  std::vector<float> inv(dims / 2);
  check(hgk_rope_inv_freq(base, dims, freqs ? freqs->data() : nullptr, inv.data()),
        "rope_inv_freq", {});
  return inv;
}

std::vector<float> llama3_rope_freqs(float base, int dims, float factor, float low_freq_factor,
                                     float high_freq_factor, float original_max_position) {
  if (dims < 2 || dims % 2) throw Exception::custom("llama3_rope_freqs: dims must be even and >= 2");
  std::vector<float> f(dims / 2);
  check(hgk_llama3_rope_freqs(base, dims, factor, low_freq_factor, high_freq_factor,
                              original_max_position, f.data()),
        "llama3_rope_freqs", {});
  return f;
}

// ------------------------------------------------------------------ norms
static Array rms_norm_impl(const char* op, const Array& x, const Array* w, float eps,
                           bool plus_one) {
  const Rows r = rows_of(x, op, {{"x", &x}, {"w", w}});
  if (w && (w->ndim() != 1 || w->dim(0) != r.n))
    fail(op, "weight must be 1-D with the size of x's last axis", {{"x", &x}, {"w", w}});
  const Dtype wd = w ? w->dtype() : x.dtype();
  const Dtype w_eff = w ? (plus_one ? Dtype::Float32 : wd) : x.dtype();
  const Dtype od = promote(x.dtype(), w_eff);
  Array y = Array::empty(x.shape(), od);
  if (x.size() == 0) return y;
  check(hgk_rms_norm(x.data(), static_cast<int>(x.dtype()), r.row_stride, w ? w->data() : nullptr,
                     static_cast<int>(wd), plus_one ? 1 : 0, eps, y.data(), static_cast<int>(od),
                     r.n, r.rows, r.n, stream_arg()),
        op, {{"x", &x}, {"w", w}});
  return y;
}

Array fast::rms_norm(const Array& x, const Array& weight, float eps) {
  return rms_norm_impl("rms_norm", x, &weight, eps, false);
}

Array nn::RmsNorm::forward(const Array& x) const {
  return rms_norm_impl("rms_norm", x, &weight, eps, plus_one);
}

std::pair<Array, Array> add_rms_norm(const Array& x, const Array& r, const nn::RmsNorm& norm) {
  const char* op = "add_rms_norm";
  Operands ops = {{"x", &x}, {"r", &r}, {"w", &norm.weight}};
  if (x.shape() != r.shape() || x.dtype() != r.dtype())
    fail(op, "x and r must match in shape and dtype", ops);
  const Rows xr = rows_of(x, op, ops);
  const Rows rr = rows_of(r, op, ops);
  if (norm.weight.ndim() != 1 || norm.weight.dim(0) != xr.n)
    fail(op, "weight must be 1-D with the size of x's last axis", ops);
  const Dtype wd = norm.weight.dtype();
  const Dtype od = promote(x.dtype(), norm.plus_one ? Dtype::Float32 : wd);
  Array h = Array::empty(x.shape(), x.dtype());
  Array y = Array::empty(x.shape(), od);
  if (x.size() == 0) return {h, y};
  check(hgk_add_rms_norm(static_cast<int>(x.dtype()), x.data(), xr.row_stride, r.data(),
                         rr.row_stride, norm.weight.data(), static_cast<int>(wd),
                         norm.plus_one ? 1 : 0, norm.eps, h.data(), xr.n, y.data(),
                         static_cast<int>(od), xr.n, xr.rows, xr.n, stream_arg()),
        op, ops);
  return {h, y};
}

Array gated_rms_norm(const Array& y, const Array& z, const nn::RmsNorm& norm) {
  const char* op = "gated_rms_norm";
  Operands ops = {{"y", &y}, {"z", &z}, {"w", &norm.weight}};
  if (norm.plus_one) fail(op, "a (1 + w) weight is not supported here", ops);
  const Rows r = rows_of(y, op, ops);
  if (z.dtype() != y.dtype()) fail(op, "z must have y's dtype", ops);
  if (norm.weight.ndim() != 1 || norm.weight.dim(0) != r.n)
    fail(op, "weight must be 1-D with the size of y's last axis", ops);
  // z as plain rows, or as (groups, rows in group) when it is a strided
  // slice such as the z part of in_proj_qkvz
  int64_t zs = 0, zg = 0, zgs = 0;
  Rows zr;
  if (as_rows(z, &zr) && zr.rows == r.rows && zr.n == r.n) {
    zs = zr.row_stride;
  } else {
    const int nd = z.ndim();
    const Shape& s = z.shape();
    const Shape& st = z.strides();
    bool ok = nd >= 3 && s[nd - 1] == r.n && (r.n == 1 || st[nd - 1] == 1);
    int64_t groups = 1;
    for (int i = nd - 4; ok && i >= 0; --i)
      if (s[i] != 1 && st[i] != s[i + 1] * st[i + 1]) ok = false;
    for (int i = 0; ok && i < nd - 2; ++i) groups *= s[i];
    if (!ok || groups * s[nd - 2] != r.rows)
      fail(op, "z is not expressible as (groups, rows, n) over y's rows", ops);
    zs = st[nd - 2];
    zg = s[nd - 2];
    zgs = st[nd - 3];
  }
  const Dtype od = promote(y.dtype(), norm.weight.dtype());
  Array out = Array::empty(y.shape(), od);
  if (y.size() == 0) return out;
  check(hgk_gated_rms_norm(static_cast<int>(y.dtype()), y.data(), r.row_stride, z.data(), zs, zg,
                           zgs, norm.weight.data(), static_cast<int>(norm.weight.dtype()), norm.eps,
                           out.data(), static_cast<int>(od), r.n, r.rows, r.n, stream_arg()),
        op, ops);
  return out;
}

// ------------------------------------------------------------------ RoPE
namespace {
struct HeadView {
  int64_t B, L, H, D;
  int64_t st[3];  // strides of (b, l, h)
};

// x [..., L, D] as (B, L, H, D): 3-D x is [N, L, D] with H = 1; 4-D and up
// is [..., H, L, D] with the axes before H collapsed into B.
bool head_view(const Array& x, HeadView* v) {
  const int nd = x.ndim();
  if (nd < 3) return false;
  const Shape& s = x.shape();
  const Shape& st = x.strides();
  if (s[nd - 1] > 1 && st[nd - 1] != 1) return false;
  v->D = s[nd - 1];
  v->L = s[nd - 2];
  if (nd == 3) {
    *v = {s[0], s[1], 1, s[2], {st[0], st[1], 0}};
    return true;
  }
  int64_t B = 1;
  for (int i = 0; i < nd - 3; ++i) {
    if (i + 1 < nd - 3 && s[i] != 1 && st[i] != s[i + 1] * st[i + 1]) return false;
    B *= s[i];
  }
  *v = {B, s[nd - 2], s[nd - 3], s[nd - 1], {st[nd - 4], st[nd - 2], st[nd - 3]}};
  return true;
}

Array rope_impl(const char* op, const Array& x, int dims, bool traditional,
                std::optional<float> base, float scale, int offset, const Array* offsets,
                const std::vector<float>* freqs) {
  Operands ops = {{"x", &x}, {"offsets", offsets}};
  if (base.has_value() == (freqs != nullptr))
    fail(op, "exactly one of base and freqs must be given", ops);
  if (freqs && static_cast<int>(freqs->size()) != dims / 2)
    fail(op, "freqs must hold dims/2 values", ops);
  HeadView xv;
  if (!head_view(x, &xv)) fail(op, "x must be [..., L, D] with a unit-stride last axis", ops);
  if (offsets) {
    if (x.ndim() != 4) fail(op, "per-sequence offsets need x as [B, H, L, D]", ops);
    if (offsets->dtype() != Dtype::Int32 || offsets->size() != xv.B || !offsets->is_contiguous())
      fail(op, "offsets must be a contiguous Int32 array with one value per sequence", ops);
  }
  Array y = Array::empty(x.shape(), x.dtype());
  if (x.size() == 0) return y;
  HeadView yv;
  head_view(y, &yv);
  check(hgk_rope(static_cast<int>(x.dtype()), x.data(), xv.st, y.data(), yv.st, xv.B, xv.L, xv.H,
                 xv.D, dims, traditional ? 1 : 0, base.value_or(0.0f), scale,
                 freqs ? freqs->data() : nullptr, offset, offsets ? static_cast<const int32_t*>(offsets->data()) : nullptr,
                 stream_arg()),
        op, ops);
  return y;
}

const std::vector<float>* rope_freqs(const nn::Rope& r) { return r.freqs.empty() ? nullptr : &r.freqs; }
std::optional<float> rope_base(const nn::Rope& r) {
  return r.freqs.empty() ? r.base : std::optional<float>();
}
}  // namespace

Array fast::rope(const Array& x, int dims, bool traditional, std::optional<float> base, float scale,
                 int offset, const std::vector<float>* freqs) {
  return rope_impl("rope", x, dims, traditional, base, scale, offset, nullptr, freqs);
}

Array fast::rope_batched(const Array& x, int dims, bool traditional, std::optional<float> base,
                         float scale, const Array& offsets, const std::vector<float>* freqs) {
  return rope_impl("rope", x, dims, traditional, base, scale, 0, &offsets, freqs);
}

Array nn::Rope::forward(const Array& x, int offset) const { return apply_rope(x, *this, offset); }

Array apply_rope(const Array& x, const nn::Rope& rope, int offset) {
  return rope_impl("rope", x, rope.dimensions, rope.traditional, rope_base(rope), rope.scale, offset,
                   nullptr, rope_freqs(rope));
}

Array apply_rope_batched(const Array& x, const nn::Rope& rope, const Array& offsets) {
  return rope_impl("rope", x, rope.dimensions, rope.traditional, rope_base(rope), rope.scale, 0,
                   &offsets, rope_freqs(rope));
}

std::pair<Array, Array> qk_norm_rope(const Array& q, const Array& k, const nn::RmsNorm* q_norm,
                                     const nn::RmsNorm* k_norm, const nn::Rope& rope, int offset,
                                     const Array* offsets) {
  const char* op = "qk_norm_rope";
  const Array* qw = q_norm ? &q_norm->weight : nullptr;
  const Array* kw = k_norm ? &k_norm->weight : nullptr;
  Operands ops = {{"q", &q}, {"k", &k}, {"q_norm", qw}, {"k_norm", kw}, {"offsets", offsets}};
  if (q.ndim() != 4 || k.ndim() != 4) fail(op, "q and k must be [B, L, H, D]", ops);
  if (q.dtype() != k.dtype()) fail(op, "q and k must share a dtype", ops);
  const int64_t B = q.dim(0), L = q.dim(1), Hq = q.dim(2), D = q.dim(3), Hk = k.dim(2);
  if (k.dim(0) != B || k.dim(1) != L || k.dim(3) != D) fail(op, "q and k shapes disagree", ops);
  if ((q_norm && q_norm->plus_one) || (k_norm && k_norm->plus_one))
    fail(op, "a (1 + w) head norm is not supported here", ops);
  if ((q_norm && k_norm && q_norm->eps != k_norm->eps))
    fail(op, "q_norm and k_norm must share eps", ops);
  const float eps = q_norm ? q_norm->eps : (k_norm ? k_norm->eps : 1e-6f);
  const Dtype wd = qw ? qw->dtype() : (kw ? kw->dtype() : q.dtype());
  if (qw && kw && qw->dtype() != kw->dtype()) fail(op, "q_norm and k_norm dtypes differ", ops);
  if (offsets && (offsets->dtype() != Dtype::Int32 || offsets->size() != B ||
                  !offsets->is_contiguous()))
    fail(op, "offsets must be a contiguous Int32 array with one value per sequence", ops);
  const std::vector<float>* freqs = rope_freqs(rope);
  const std::optional<float> base = rope_base(rope);
  if (!freqs && !base) fail(op, "rope needs a base or a frequency table", ops);
  Array qo = Array::empty({B, Hq, L, D}, q.dtype());
  Array ko = Array::empty({B, Hk, L, D}, k.dtype());
  if (q.size() == 0 && k.size() == 0) return {qo, ko};
  const int64_t qs[3] = {q.strides()[0], q.strides()[1], q.strides()[2]};
  const int64_t ks[3] = {k.strides()[0], k.strides()[1], k.strides()[2]};
  const int64_t qos[3] = {Hq * L * D, D, L * D};
  const int64_t kos[3] = {Hk * L * D, D, L * D};
  if (D > 1 && (q.strides()[3] != 1 || k.strides()[3] != 1))
    fail(op, "q and k need a unit-stride head_dim", ops);
  check(hgk_qk_norm_rope(static_cast<int>(q.dtype()), q.data(), qs, qo.data(), qos, Hq,
                         qw ? qw->data() : nullptr, k.data(), ks, ko.data(), kos, Hk,
                         kw ? kw->data() : nullptr, static_cast<int>(wd), eps, B, L, D,
                         rope.dimensions, base.value_or(0.0f), rope.scale,
                         freqs ? freqs->data() : nullptr, offset,
                         offsets ? static_cast<const int32_t*>(offsets->data()) : nullptr,
                         stream_arg()),
        op, ops);
  return {qo, ko};
}

// ------------------------------------------------------------------ GLU
static Array glu_impl(const char* op, int act, const Array& gate, const Array& up) {
  Operands ops = {{"gate", &gate}, {"up", &up}};
  if (gate.shape() != up.shape() || gate.dtype() != up.dtype())
    fail(op, "gate and up must match in shape and dtype", ops);
  const Rows g = rows_of(gate, op, ops);
  const Rows u = rows_of(up, op, ops);
  Array out = Array::empty(gate.shape(), gate.dtype());
  if (gate.size() == 0) return out;
  check(hgk_glu(act, static_cast<int>(gate.dtype()), gate.data(), g.row_stride, up.data(),
                u.row_stride, out.data(), static_cast<int>(gate.dtype()), g.n, g.rows, g.n,
                stream_arg()),
        op, ops);
  return out;
}

Array swiglu(const Array& gate, const Array& x) { return glu_impl("swiglu", HGK_ACT_SILU, gate, x); }
Array nn::silu_mul(const Array& gate, const Array& up) {
  return glu_impl("silu_mul", HGK_ACT_SILU, gate, up);
}
Array nn::gelu_approximate_mul(const Array& gate, const Array& up) {
  return glu_impl("gelu_approximate_mul", HGK_ACT_GELU_TANH, gate, up);
}

// ------------------------------------------------------------------ embedding
int64_t nn::QuantizedEmbedding::hidden() const {
  if (weight.ndim() != 2 || bits <= 0) return 0;
  return weight.dim(1) * 32 / bits;
}

static void qembed_check(const char* op, const nn::QuantizedEmbedding& e, const Array& ids) {
  Operands ops = {{"ids", &ids}, {"w", &e.weight}, {"scales", &e.scales}, {"biases", &e.biases}};
  if (e.weight.ndim() != 2 || e.weight.dtype() != Dtype::Uint32 || !e.weight.is_contiguous())
    fail(op, "weight must be contiguous Uint32 [vocab, hidden*bits/32]", ops);
  if (ids.dtype() != Dtype::Int32 && ids.dtype() != Dtype::Uint32)
    fail(op, "ids must be Int32 or Uint32", ops);
  if (!ids.is_contiguous()) fail(op, "ids must be contiguous", ops);
  if (e.scales.dtype() != e.biases.dtype() || e.scales.shape() != e.biases.shape())
    fail(op, "scales and biases must match", ops);
  const int64_t V = e.weight.dim(0), H = e.hidden();
  if (e.scales.ndim() != 2 || e.scales.dim(0) != V || e.group_size <= 0 ||
      e.scales.dim(1) * e.group_size != H || !e.scales.is_contiguous() || !e.biases.is_contiguous())
    fail(op, "scales/biases must be contiguous [vocab, hidden/group_size]", ops);
}

static Array qembed_impl(const nn::QuantizedEmbedding& e, const Array& ids, float scale) {
  const char* op = "quantized_embedding";
  Operands ops = {{"ids", &ids}, {"w", &e.weight}, {"scales", &e.scales}, {"biases", &e.biases}};
  qembed_check(op, e, ids);
  const int64_t V = e.weight.dim(0), H = e.hidden();
  Shape os = ids.shape();
  os.push_back(H);
  Array out = Array::empty(os, e.scales.dtype());
  if (ids.size() == 0) return out;
  check(hgk_quantized_embedding(ids.data(), static_cast<int>(ids.dtype()), ids.size(),
                                static_cast<const uint32_t*>(e.weight.data()), e.scales.data(),
                                e.biases.data(), static_cast<int>(e.scales.dtype()), V, H,
                                e.group_size, e.bits, scale, out.data(), H, stream_arg()),
        op, ops);
  return out;
}

std::pair<Array, Array> nn::QuantizedEmbedding::forward_rms_norm(const Array& ids,
                                                                 const RmsNorm& norm,
                                                                 float scale) const {
  const char* op = "quantized_embedding_rms_norm";
  Operands ops = {{"ids", &ids}, {"w", &weight}, {"scales", &scales}, {"biases", &biases},
                  {"norm", &norm.weight}};
  qembed_check(op, *this, ids);
  const int64_t V = weight.dim(0), H = hidden();
  if (norm.weight.ndim() != 1 || norm.weight.dim(0) != H || !norm.weight.is_contiguous())
    fail(op, "norm weight must be contiguous with hidden elements", ops);
  const Dtype od = promote(scales.dtype(), norm.plus_one ? Dtype::Float32 : norm.weight.dtype());
  Shape os = ids.shape();
  os.push_back(H);
  Array h = Array::empty(os, scales.dtype());
  Array y = Array::empty(os, od);
  if (ids.size() == 0) return {h, y};
  check(hgk_quantized_embedding_rms_norm(
            ids.data(), static_cast<int>(ids.dtype()), ids.size(),
            static_cast<const uint32_t*>(weight.data()), scales.data(), biases.data(),
            static_cast<int>(scales.dtype()), V, H, group_size, bits, scale, h.data(), H,
            norm.weight.data(), static_cast<int>(norm.weight.dtype()), norm.plus_one ? 1 : 0,
            norm.eps, y.data(), static_cast<int>(od), H, stream_arg()),
        op, ops);
  return {h, y};
}

Array nn::QuantizedEmbedding::forward(const Array& ids) const { return qembed_impl(*this, ids, 0.0f); }
Array nn::QuantizedEmbedding::forward_scaled(const Array& ids, float scale) const {
  return qembed_impl(*this, ids, scale);
}


// ------------------------------------------------------------------ gather_qmm
Array gather_qmm(const Array& x, const Array& w, const Array& scales, const Array& biases,
                 const Array& rhs_indices, bool transpose, int group_size, int bits,
                 int64_t x_row_div, const Array* lhs_indices) {
  const char* op = "gather_qmm";
  Operands ops = {{"x", &x}, {"w", &w}, {"scales", &scales}, {"biases", &biases},
                  {"idx", &rhs_indices}, {"lhs", lhs_indices}};
  if (!transpose) fail(op, "only transpose = true (weights stored [N, K]) is implemented", ops);
  if (x.ndim() != 2 || (x.dim(1) > 1 && x.strides()[1] != 1))
    fail(op, "x must be [rows, K] with a unit-stride last axis", ops);
  if (w.ndim() != 3 || w.dtype() != Dtype::Uint32 || !w.is_contiguous() || scales.ndim() != 3 ||
      scales.shape() != biases.shape() || !scales.is_contiguous() || !biases.is_contiguous() ||
      scales.dtype() != biases.dtype())
    fail(op, "w must be contiguous Uint32 [E, N, K/8]; scales/biases [E, N, K/group] of one dtype",
         ops);
  if (!rhs_indices.is_contiguous() || (lhs_indices && !lhs_indices->is_contiguous()))
    fail(op, "indices must be contiguous", ops);
  const int64_t P = rhs_indices.size(), E = w.dim(0), N = w.dim(1), K = x.dim(1);
  if (w.dim(2) * 32 / bits != K) fail(op, "w's packed width does not match x's K", ops);
  Array y = Array::empty({P, N}, x.dtype());
  if (P == 0) return y;
  check(hgk_gather_qmm(static_cast<int>(x.dtype()), x.data(), x.dim(0), x.strides()[0], x_row_div,
                       lhs_indices ? static_cast<const int32_t*>(lhs_indices->data()) : nullptr,
                       static_cast<const uint32_t*>(w.data()), scales.data(), biases.data(),
                       static_cast<int>(scales.dtype()), E, N, K, group_size, bits,
                       rhs_indices.data(), static_cast<int>(rhs_indices.dtype()), P, y.data(), N,
                       stream_arg()),
        op, ops);
  return y;
}

Array quantized_matmul(const Array& x, const Array& w, const Array& scales, const Array& biases,
                       bool transpose, int group_size, int bits) {
  const char* op = "quantized_matmul";
  Operands ops = {{"x", &x}, {"w", &w}, {"scales", &scales}, {"biases", &biases}};
  if (!transpose) fail(op, "only transpose = true (weights stored [N, K]) is implemented", ops);
  if (x.ndim() < 1) fail(op, "x must have at least one axis", ops);
  if (w.ndim() != 2 || w.dtype() != Dtype::Uint32 || !w.is_contiguous() || scales.ndim() != 2 ||
      scales.shape() != biases.shape() || !scales.is_contiguous() || !biases.is_contiguous() ||
      scales.dtype() != biases.dtype())
    fail(op, "w must be contiguous Uint32 [N, K/8]; scales/biases [N, K/group] of one dtype", ops);
  const int64_t K = x.dim(-1), N = w.dim(0);
  if (bits <= 0 || w.dim(1) * 32 / bits != K) fail(op, "w's packed width does not match x's K", ops);
  Shape lead(x.shape().begin(), x.shape().end() - 1);
  int64_t M = 1;
  for (int64_t d : lead) M *= d;
  // rows of x: [M, K] with a unit-stride last axis (a 2-d strided view is
  // taken as it is; more leading axes must merge without a copy)
  if (K > 1 && x.strides().back() != 1) fail(op, "x's last axis must have unit stride", ops);
  Array x2 = x.ndim() == 2 ? x : x.reshape({M, K});
  Shape oshape = lead;
  oshape.push_back(N);
  Array y = Array::empty(oshape, x.dtype());
  if (M == 0) return y;
  check(hgk_quantized_matmul(static_cast<int>(x.dtype()), x2.data(), M, x2.strides()[0],
                             static_cast<const uint32_t*>(w.data()), scales.data(), biases.data(),
                             static_cast<int>(scales.dtype()), N, K, group_size, bits, y.data(), N,
                             stream_arg()),
        op, ops);
  return y;
}

Array nn::QLinear::forward(const Array& x) const {
  return quantized_matmul(x, weight, scales, biases, true, group_size, bits);
}

Array nn::SwitchMlpWeights::forward_gather(const Array& x, const Array& indices) const {
  if (x.ndim() != 2 || indices.ndim() != 2 || indices.dim(0) != x.dim(0))
    throw Exception::custom("forward_gather input must be [T, D] with indices [T, top_k] " +
                            operands_text({{"x", &x}, {"indices", &indices}}));
  const int64_t T = x.dim(0), top_k = indices.dim(1);
  const Array idx = indices.reshape({T * top_k});
  // gate, up and the SwiGLU in one launch where a fused kernel applies (same
  // weights' shapes, bf16: the decode GEMV at few pairs per expert, the
  // grouped kernel's fused form at many); otherwise the reference's three
  // calls
  Array act;
  bool fused = false;
  const Array& gw = gate_proj.weight;
  // (one scales dtype reaches the kernel for both projections, so every
  // scale and bias must share it)
  const Dtype sdt = gate_proj.scales.dtype();
  const bool same = gw.shape() == up_proj.weight.shape() &&
                    gate_proj.scales.shape() == up_proj.scales.shape() &&
                    gate_proj.biases.dtype() == sdt && up_proj.scales.dtype() == sdt &&
                    up_proj.biases.dtype() == sdt &&
                    gate_proj.group_size == up_proj.group_size && gate_proj.bits == up_proj.bits;
  if (same && gw.ndim() == 3 && x.dtype() == Dtype::Bfloat16 && x.strides()[1] == 1 &&
      gw.is_contiguous() && up_proj.weight.is_contiguous() && gate_proj.scales.is_contiguous() &&
      gate_proj.biases.is_contiguous() && up_proj.scales.is_contiguous() &&
      up_proj.biases.is_contiguous() && idx.is_contiguous()) {
    const int64_t E = gw.dim(0), N = gw.dim(1), K = x.dim(1), P = T * top_k;
    act = Array::empty({P, N}, x.dtype());
    const int st = hgk_gather_qmm_swiglu(
        static_cast<int>(x.dtype()), x.data(), T, x.strides()[0], top_k, nullptr,
        static_cast<const uint32_t*>(gw.data()), gate_proj.scales.data(), gate_proj.biases.data(),
        static_cast<const uint32_t*>(up_proj.weight.data()), up_proj.scales.data(),
        up_proj.biases.data(), static_cast<int>(gate_proj.scales.dtype()), E, N, K,
        gate_proj.group_size, gate_proj.bits, idx.data(), static_cast<int>(idx.dtype()), P,
        act.data(), N, stream_arg());
    if (st != HGK_ERR_UNSUPPORTED) check(st, "forward_gather", {{"x", &x}, {"indices", &indices}});
    fused = st == HGK_OK;
  }
  if (!fused) {
    const Array g = gather_qmm(x, gate_proj.weight, gate_proj.scales, gate_proj.biases, idx, true,
                               gate_proj.group_size, gate_proj.bits, top_k);
    const Array u = gather_qmm(x, up_proj.weight, up_proj.scales, up_proj.biases, idx, true,
                               up_proj.group_size, up_proj.bits, top_k);
    act = swiglu(g, u);
  }
  const Array d = gather_qmm(act, down_proj.weight, down_proj.scales, down_proj.biases, idx, true,
                             down_proj.group_size, down_proj.bits, 1);
  return d.reshape({T, top_k, d.dim(1)});
}

// ------------------------------------------------------------------ gated delta
std::pair<Array, Array> gated_delta(const Array& q, const Array& k, const Array& v,
                                    const Array& a_log, const Array& a, const Array& dt_bias,
                                    const Array& b, const Array* state_in, const Array* q_norm_w,
                                    const Array* k_norm_w, float eps) {
  const char* op = "gated_delta";
  Operands ops = {{"q", &q},   {"k", &k}, {"v", &v},         {"a_log", &a_log},
                  {"a", &a},   {"dt_bias", &dt_bias},        {"b", &b},
                  {"state", state_in}, {"q_norm_w", q_norm_w}, {"k_norm_w", k_norm_w}};
  if (q.ndim() != 4 || k.shape() != q.shape() || v.ndim() != 4 || a.ndim() != 3 ||
      b.shape() != a.shape())
    fail(op, "q, k must be [B, T, Hk, Dk], v [B, T, Hv, Dv], a and b [B, T, Hv]", ops);
  const int64_t B = q.dim(0), T = q.dim(1), Hk = q.dim(2), Dk = q.dim(3);
  const int64_t Hv = v.dim(2), Dv = v.dim(3);
  if (v.dim(0) != B || v.dim(1) != T || a.dim(0) != B || a.dim(1) != T || a.dim(2) != Hv)
    fail(op, "batch, steps or v heads disagree", ops);
  for (const Array* t : {&q, &k, &v, &a, &b})
    if (!t->is_contiguous() || t->dtype() != q.dtype())
      fail(op, "q, k, v, a, b must be contiguous and share a dtype", ops);
  if (a_log.size() != Hv || dt_bias.size() != Hv || a_log.dtype() != dt_bias.dtype() ||
      !a_log.is_contiguous() || !dt_bias.is_contiguous())
    fail(op, "a_log and dt_bias must be contiguous [Hv] of one dtype", ops);
  if (state_in && (state_in->shape() != Shape({B, Hv, Dv, Dk}) || !state_in->is_contiguous() ||
                   state_in->dtype() != q.dtype()))
    fail(op, "state must be contiguous [B, Hv, Dv, Dk] in q's dtype", ops);
  if ((q_norm_w == nullptr) != (k_norm_w == nullptr)) fail(op, "pass both norm weights or neither", ops);
  if (q_norm_w && (q_norm_w->size() != Dk || k_norm_w->size() != Dk ||
                   q_norm_w->dtype() != q.dtype() || k_norm_w->dtype() != q.dtype() ||
                   !q_norm_w->is_contiguous() || !k_norm_w->is_contiguous()))
    fail(op, "norm weights must be contiguous [Dk] in q's dtype", ops);
  Array y = Array::empty({B, T, Hv, Dv}, q.dtype());
  Array st = Array::empty({B, Hv, Dv, Dk}, q.dtype());
  if (B == 0) return {y, st};
  check(hgk_gated_delta(static_cast<int>(q.dtype()), q.data(), k.data(), v.data(), a_log.data(),
                        a.data(), dt_bias.data(), b.data(), static_cast<int>(a_log.dtype()),
                        state_in ? state_in->data() : nullptr,
                        q_norm_w ? q_norm_w->data() : nullptr, k_norm_w ? k_norm_w->data() : nullptr,
                        eps, B, T, Hk, Dk, Hv, Dv, y.data(), st.data(), stream_arg()),
        op, ops);
  return {y, st};
}

std::pair<Array, Array> gdn_qk_norm_weights(int64_t head_k_dim, Dtype dt) {
  const float s = 1.0f / std::sqrt(static_cast<float>(head_k_dim));
  std::vector<float> wq(head_k_dim, s * s), wk(head_k_dim, s);
  return {Array::from_slice(wq, {head_k_dim}, dt), Array::from_slice(wk, {head_k_dim}, dt)};
}

// ------------------------------------------------------------------ checkpoints
namespace io {

std::vector<std::string> collect_safetensors_files(const std::string& model_dir) {
  int64_t need = 0;
  check(hgk_st_collect_files(model_dir.c_str(), nullptr, 0, &need), "collect_safetensors_files", {});
  std::string buf((size_t)need, '\0');
  check(hgk_st_collect_files(model_dir.c_str(), &buf[0], need, &need), "collect_safetensors_files", {});
  std::vector<std::string> out;
  size_t pos = 0;
  for (size_t nl; (nl = buf.find('\n', pos)) != std::string::npos; pos = nl + 1)
    out.push_back(buf.substr(pos, nl - pos));
  return out;
}

std::optional<std::string> remap_quantized_key(const std::string& key) {
  std::string buf(key.size() + 16, '\0');
  const int st = hgk_remap_quantized_key(key.c_str(), &buf[0], (int64_t)buf.size());
  if (st == HGK_ERR_UNSUPPORTED) return std::nullopt;
  check(st, "remap_quantized_key", {});
  return std::string(buf.c_str());
}

SafetensorsFile::SafetensorsFile(const std::string& path) : path_(path) {
  check(hgk_st_open(path.c_str(), &f_), "load_safetensors", {});
}

SafetensorsFile::~SafetensorsFile() { hgk_st_close(f_); }

std::vector<std::string> SafetensorsFile::keys() const {
  std::vector<std::string> out;
  const int64_t n = hgk_st_count(f_);
  for (int64_t i = 0; i < n; ++i) {
    const char* name = nullptr;
    check(hgk_st_tensor(f_, i, &name, nullptr, nullptr, nullptr, nullptr, nullptr), "load_safetensors", {});
    out.emplace_back(name);
  }
  return out;
}

int64_t SafetensorsFile::index(const std::string& name) const {
  int64_t i = -1;
  check(hgk_st_find(f_, name.c_str(), &i), "load_safetensors", {});
  return i;
}

bool SafetensorsFile::contains(const std::string& name) const {
  int64_t i = -1;
  return hgk_st_find(f_, name.c_str(), &i) == HGK_OK;
}

Shape SafetensorsFile::shape(const std::string& name) const {
  int nd = 0;
  int64_t sh[8];
  check(hgk_st_tensor(f_, index(name), nullptr, nullptr, nullptr, &nd, sh, nullptr), "load_safetensors", {});
  return Shape(sh, sh + nd);
}

std::string SafetensorsFile::dtype_name(const std::string& name) const {
  const char* dn = nullptr;
  check(hgk_st_tensor(f_, index(name), nullptr, &dn, nullptr, nullptr, nullptr, nullptr), "load_safetensors", {});
  return dn;
}

Array SafetensorsFile::load(const std::string& name) const {
  const int64_t i = index(name);
  int dt = -1, nd = 0;
  int64_t sh[8], nbytes = 0;
  const char* dn = nullptr;
  check(hgk_st_tensor(f_, i, nullptr, &dn, &dt, &nd, sh, &nbytes), "load_safetensors", {});
  if (dt < 0)
    throw Exception(HGK_ERR_UNSUPPORTED, "load_safetensors failed: '" + name + "' is " + dn +
                                             ", which no kernel here takes [" + path_ + "]");
  Array a = Array::empty(Shape(sh, sh + nd), static_cast<Dtype>(dt));
  check(hgk_st_upload(f_, i, a.data(), nbytes, stream_arg()), "load_safetensors", {});
  return a;
}

size_t load_quantized_safetensors_weights(std::map<std::string, Array>& params,
                                          const std::string& model_dir, bool quantized) {
  size_t loaded = 0;
  for (const auto& path : collect_safetensors_files(model_dir)) {
    SafetensorsFile f(path);
    for (const auto& key : f.keys()) {
      auto it = params.find(key);
      if (it == params.end() && quantized) {
        const auto rk = remap_quantized_key(key);
        if (rk) it = params.find(*rk);
      }
      if (it == params.end()) continue;
      it->second = f.load(key);
      ++loaded;
    }
  }
  return loaded;
}

}  // namespace io
}  // namespace higgs
