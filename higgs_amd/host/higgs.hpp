// higgs.hpp -- C++ host API over the C ABI of libhiggs_hip.so.
//
// The reference (panbanda/higgs, crates/higgs-models) calls these ops through
// mlx-rs from its layer structs. This header keeps those calls' names,
// argument meaning and error behaviour, so a layer forward written against
// mlx-rs reads the same against it:
//
//   fast::rms_norm(x, weight, eps)               mlx_rs::fast::rms_norm
//   nn::RmsNorm{weight, eps}.forward(x)          nn::RmsNorm (transformer.rs:387-392, 407-415)
//   fast::rope(x, dims, traditional, base, scale, offset, freqs)
//                                                mlx_rs::fast::rope
//   apply_rope(x, rope, offset)                  utils.rs:16-26
//   apply_rope_batched(x, rope, offsets)         the per-request rope loop of
//                                                Model::forward_batched (transformer.rs:747-802)
//   qk_norm_rope(q, k, q_norm, k_norm, rope, offset)
//                                                q_norm/k_norm, transpose, apply_rope
//                                                (transformer.rs:264-287)
//   swiglu(gate, x)                              qwen3_next.rs:275-277
//   nn::silu_mul(gate, up)                       nn::silu(gate) * up (transformer.rs:349-353)
//   nn::gelu_approximate_mul(gate, up)           nn::gelu_approximate(gate) * up (gemma2.rs:422-427)
//   gated_rms_norm(y, z, norm)                   swiglu(z, norm(y)) (qwen3_next.rs:1204-1205)
//   add_rms_norm(x, r, norm)                     h = x.add(r); norm(h) (transformer.rs:413-415)
//   nn::QuantizedEmbedding{...}.forward(ids)     nn::QuantizedEmbedding (transformer.rs:494)
//                                                and QEmbedding::forward (qwen3_next.rs:248-257)
//   gather_qmm(x, w, scales, biases, rhs_indices, transpose, group_size, bits)
//                                                qwen3_next.rs:294-363
//   nn::SwitchMlpWeights{...}.forward_gather(x, indices)
//                                                qwen3_next.rs:844-904
//   io::load_quantized_safetensors_weights(params, dir, quantized)
//                                                lib.rs:600-632 (with collect_safetensors_files
//                                                and remap_quantized_key, lib.rs:682-723)
//
// Errors are thrown as higgs::Exception, whose message follows the
// reference's `Exception::custom` convention (qwen3_next.rs:337-361): the
// op name, the library's message, then the operands' shapes and dtypes.
//
// Every op enqueues on the calling thread's current stream
// (Stream::task_local_or_default, after qwen3_next.rs:307) and never
// synchronises; only the host readback helpers (to_f32, to_bits, item) wait.
// Results are allocated stream-ordered (hipMallocAsync) and released with
// hipFreeAsync on the stream they were allocated on.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "higgs_hip.h"

namespace higgs {

// mlx_rs::Dtype names for the types this path uses.
enum class Dtype : int {
  Float32 = HGK_F32,
  Bfloat16 = HGK_BF16,
  Float16 = HGK_F16,
  Uint32 = HGK_U32,
  Int32 = HGK_I32,
};
std::size_t size_of(Dtype dt);
const char* name_of(Dtype dt);      // "Float32", "Bfloat16", ... (Rust Debug form)
bool is_floating(Dtype dt);
Dtype promote(Dtype a, Dtype b);    // MLX float promotion (equal -> same, else Float32)

using Shape = std::vector<int64_t>;
std::string format_shape(const Shape& s);  // "[512, 2048]"

class Exception : public std::runtime_error {
 public:
  Exception(int status, const std::string& msg) : std::runtime_error(msg), status_(status) {}
  // Exception::custom(msg) of mlx-rs: an argument error with a message.
  static Exception custom(const std::string& msg) { return Exception(HGK_ERR_ARG, msg); }
  int status() const { return status_; }

 private:
  int status_;
};

// A HIP stream handle. Default-constructed = the null stream. `create()`
// makes an owning stream at the default priority.
class Stream {
 public:
  Stream() = default;
  explicit Stream(hipStream_t s) : s_(s) {}
  static Stream create();
  // The calling thread's current stream (set with StreamScope), else the
  // null stream.
  static Stream task_local_or_default();
  hipStream_t get() const { return s_; }
  void synchronize() const;

 private:
  hipStream_t s_ = nullptr;
  std::shared_ptr<void> owner_;
};

// Makes `s` the calling thread's current stream for the scope's lifetime.
class StreamScope {
 public:
  explicit StreamScope(const Stream& s);
  ~StreamScope();
  StreamScope(const StreamScope&) = delete;
  StreamScope& operator=(const StreamScope&) = delete;

 private:
  Stream prev_;
};

namespace detail {
struct Buffer;
}

// A device array: shape, element strides and dtype over a shared device
// buffer. Views (transpose, slice, reshape of contiguous data) share the
// buffer; ops write fresh row-major results.
class Array {
 public:
  Array() = default;

  static Array empty(const Shape& shape, Dtype dt);
  // Host values rounded (to nearest even) to `dt` and uploaded.
  static Array from_slice(const float* data, std::size_t n, const Shape& shape,
                          Dtype dt = Dtype::Float32);
  static Array from_slice(const std::vector<float>& v, const Shape& shape,
                          Dtype dt = Dtype::Float32) {
    return from_slice(v.data(), v.size(), shape, dt);
  }
  static Array from_slice(const int32_t* data, std::size_t n, const Shape& shape);
  static Array from_slice(const std::vector<int32_t>& v, const Shape& shape) {
    return from_slice(v.data(), v.size(), shape);
  }
  static Array from_slice(const uint32_t* data, std::size_t n, const Shape& shape);
  static Array from_slice(const std::vector<uint32_t>& v, const Shape& shape) {
    return from_slice(v.data(), v.size(), shape);
  }
  // Raw 16-bit codes (bf16 or f16 bit patterns) uploaded unchanged.
  static Array from_bits(const uint16_t* bits, std::size_t n, const Shape& shape, Dtype dt);

  const Shape& shape() const { return shape_; }
  int64_t dim(int axis) const;  // negative axes count from the end
  const Shape& strides() const { return strides_; }
  int ndim() const { return static_cast<int>(shape_.size()); }
  int64_t size() const;
  Dtype dtype() const { return dtype_; }
  std::size_t itemsize() const { return size_of(dtype_); }
  bool is_contiguous() const;
  // Device address of element [0, ..., 0].
  void* data() const;

  // Views.
  Array transpose(const std::vector<int>& axes) const;
  Array slice(int axis, int64_t start, int64_t stop) const;
  // A view when the new shape only splits or merges row-major runs of axes
  // (always for contiguous arrays); throws where a copy would be needed.
  Array reshape(const Shape& shape) const;

  // Host readback (waits for the current stream). Elements come back in
  // row-major order of the logical shape, whatever the strides.
  std::vector<float> to_f32() const;
  std::vector<uint16_t> to_bits() const;  // 16-bit dtypes only
  std::vector<uint32_t> to_u32() const;   // 32-bit dtypes, raw words
  float item() const;                      // size-1 arrays

  // "[512, 2048]/Bfloat16", the operand form used in error messages.
  std::string describe() const;

 private:
  std::shared_ptr<detail::Buffer> buf_;
  int64_t offset_ = 0;  // elements
  Shape shape_, strides_;
  Dtype dtype_ = Dtype::Float32;
  void gather_host(void* out) const;
};

// Inverse frequencies and llama3 frequency tables, as fast::rope derives them.
std::vector<float> rope_inv_freq(float base, int dims, const std::vector<float>* freqs = nullptr);
std::vector<float> llama3_rope_freqs(float base, int dims, float factor, float low_freq_factor,
                                     float high_freq_factor, float original_max_position);

namespace fast {
// y = weight * round(x * rsqrt(mean(x^2) + eps)) over the last axis. The
// result dtype is the promotion of x's and weight's.
Array rms_norm(const Array& x, const Array& weight, float eps);
// x is [..., L, D] with positions along axis -2 (leading axes flattened).
// Exactly one of `base` and `freqs` is given.
Array rope(const Array& x, int dims, bool traditional, std::optional<float> base, float scale,
           int offset, const std::vector<float>* freqs = nullptr);
// As rope for x [B, H, L, D], with offsets (int32 [B], device) giving each
// sequence its own start position.
Array rope_batched(const Array& x, int dims, bool traditional, std::optional<float> base,
                   float scale, const Array& offsets, const std::vector<float>* freqs = nullptr);
}  // namespace fast

namespace nn {
// nn::RmsNorm. `plus_one` applies Gemma's (1 + weight) in f32, which the
// reference bakes into the weights at load time (gemma2.rs:799-826); the
// result is then Float32, as it is there.
struct RmsNorm {
  Array weight;
  float eps = 1e-5f;
  bool plus_one = false;
  Array forward(const Array& x) const;
};

// nn::Rope's fields (dimensions, traditional, base, scale) plus an optional
// explicit frequency table (the freqs argument of fast::rope,
// deepseek_v2.rs:222-225; llama3 scaling uses it).
struct Rope {
  int dimensions = 0;
  bool traditional = false;
  std::optional<float> base = 10000.0f;
  float scale = 1.0f;
  std::vector<float> freqs;  // empty: derive from base
  Array forward(const Array& x, int offset) const;
};

// nn::QuantizedEmbedding over the MLX affine format: weight Uint32
// [V, H*bits/32], scales and biases [V, H/group_size] (Bfloat16 or Float16).
struct QuantizedEmbedding {
  Array weight, scales, biases;
  int group_size = 64;
  int bits = 4;
  int64_t hidden() const;
  Array forward(const Array& ids) const;
  // forward followed by h * round(scale) (Gemma's sqrt(H) embedding scale,
  // gemma2.rs:587-600) in the same pass.
  Array forward_scaled(const Array& ids, float scale) const;
  // forward_scaled(ids, scale) (scale 0: none) followed by the first block's
  // input norm (transformer.rs:494, 407) in one pass: returns (h, norm(h)).
  std::pair<Array, Array> forward_rms_norm(const Array& ids, const RmsNorm& norm,
                                           float scale = 0.0f) const;
};

Array silu_mul(const Array& gate, const Array& up);
Array gelu_approximate_mul(const Array& gate, const Array& up);

// A quantized linear layer's tensors (qwen3_next.rs:186-210): weight Uint32
// [.., N, K*bits/32], scales/biases [.., N, K/group_size].
struct QLinear {
  Array weight, scales, biases;
  int group_size = 64;
  int bits = 4;
  // QLinear::forward (qwen3_next.rs:210-220): quantized_matmul(x, weight,
  // scales, biases, transpose = true, group_size, bits) over the last axis
  // of x (any leading dims; weight [N, K*bits/32] for this form).
  Array forward(const Array& x) const;
};

// Stacked expert weights of a switch MLP (qwen3_next.rs:824-904).
struct SwitchMlpWeights {
  QLinear gate_proj, up_proj, down_proj;
  // x [T, D], indices [T, top_k] (Int32/Uint32) -> [T, top_k, D]: gate and up
  // gather_qmm, swiglu, down gather_qmm, as forward_gather does (gate, up and
  // swiglu in one launch where a fused kernel applies: the decode GEMV, or
  // the grouped matrix-core kernel's fused form at prefill).
  Array forward_gather(const Array& x, const Array& indices) const;
};
}  // namespace nn

// ops::quantized_matmul(x, w, scales, biases, transpose, group_size, bits)
// (quantized_forward, qwen3_next.rs:174-183): x [..., K] with a unit-stride
// last axis, w [N, K*bits/32] Uint32, scales/biases [N, K/group_size];
// returns [..., N]. Only transpose = true (weights stored [N, K]).
Array quantized_matmul(const Array& x, const Array& w, const Array& scales, const Array& biases,
                       bool transpose, int group_size, int bits);

// gather_qmm(x, w, scales, biases, rhs_indices, transpose = true, group_size,
// bits) with one row of x per (token, expert) pair (qwen3_next.rs:294-363):
// x [R, K]; rhs_indices [P]; pair p reads x row p / x_row_div (or
// lhs_indices[p]). Returns [P, N].
Array gather_qmm(const Array& x, const Array& w, const Array& scales, const Array& biases,
                 const Array& rhs_indices, bool transpose, int group_size, int bits,
                 int64_t x_row_div = 1, const Array* lhs_indices = nullptr);

// gated_delta_kernel_ffi(q, k, v, a_log, a, dt_bias, b, state_in, ...)
// (qwen3_next.rs:559-630): the GatedDeltaNet recurrence over T steps, q/k
// [B, T, Hk, Dk], v [B, T, Hv, Dv], a/b [B, T, Hv], a_log/dt_bias [Hv],
// state_in [B, Hv, Dv, Dk] (nullptr: zeros). With q_norm_w/k_norm_w the
// constant-weight q/k rms_norm in front of it (qwen3_next.rs:1172-1173) runs
// in the same kernel. Returns (y [B, T, Hv, Dv], state_out).
std::pair<Array, Array> gated_delta(const Array& q, const Array& k, const Array& v,
                                    const Array& a_log, const Array& a, const Array& dt_bias,
                                    const Array& b, const Array* state_in,
                                    const Array* q_norm_w = nullptr,
                                    const Array* k_norm_w = nullptr, float eps = 1e-6f);
// Those constant weights: (s * s, s) with s = 1/sqrt(head_k_dim) in f32
// (qwen3_next.rs:1075-1094), cast to dt as at 1165-1169.
std::pair<Array, Array> gdn_qk_norm_weights(int64_t head_k_dim, Dtype dt);

// Checkpoint loading (crates/higgs-models/src/lib.rs:574-723): safetensors
// files in the MLX 4-bit layout, read through the library's reader.
namespace io {
// The checkpoint's files: the shards named by model.safetensors.index.json,
// else model.safetensors; throws (a "MissingWeight" message) when neither exists.
std::vector<std::string> collect_safetensors_files(const std::string& model_dir);
// `x.weight` -> `x.inner.weight` (and .scales, .biases, .bias); nullopt otherwise.
std::optional<std::string> remap_quantized_key(const std::string& key);

class SafetensorsFile {
 public:
  explicit SafetensorsFile(const std::string& path);
  ~SafetensorsFile();
  SafetensorsFile(const SafetensorsFile&) = delete;
  SafetensorsFile& operator=(const SafetensorsFile&) = delete;
  std::vector<std::string> keys() const;  // header order
  bool contains(const std::string& name) const;
  Shape shape(const std::string& name) const;
  std::string dtype_name(const std::string& name) const;  // "BF16", "U32", ...
  // The tensor on the device (current stream; complete on return). Only the
  // dtypes of Dtype load this way.
  Array load(const std::string& name) const;

 private:
  hgk_st_file* f_ = nullptr;
  std::string path_;
  int64_t index(const std::string& name) const;
};

// load_quantized_safetensors_weights: every checkpoint key that names an
// entry of `params` (directly, or after remap_quantized_key when `quantized`)
// replaces that entry. Returns how many were loaded.
size_t load_quantized_safetensors_weights(std::map<std::string, Array>& params,
                                          const std::string& model_dir, bool quantized);
}  // namespace io

Array apply_rope(const Array& x, const nn::Rope& rope, int offset);
Array apply_rope_batched(const Array& x, const nn::Rope& rope, const Array& offsets);
Array swiglu(const Array& gate, const Array& x);
// The block boundary `h = x.add(r); norm.forward(&h)` (transformer.rs:413-415)
// in one pass: returns (h, norm(h)).
std::pair<Array, Array> add_rms_norm(const Array& x, const Array& r, const nn::RmsNorm& norm);
// swiglu(z, norm.forward(y)); z may be a strided view (read in place).
Array gated_rms_norm(const Array& y, const Array& z, const nn::RmsNorm& norm);
// Per-head RMSNorm over head_dim, then RoPE, for q [B, L, Hq, D] and
// k [B, L, Hk, D] in the projection layout (any strides, unit D stride).
// Returns (q, k) as [B, H, L, D]. `offsets` (int32 [B]) overrides `offset`.
std::pair<Array, Array> qk_norm_rope(const Array& q, const Array& k, const nn::RmsNorm* q_norm,
                                     const nn::RmsNorm* k_norm, const nn::Rope& rope,
                                     int offset, const Array* offsets = nullptr);

}  // namespace higgs
