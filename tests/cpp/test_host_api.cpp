// Parity tests of the C++ host API (higgs_amd/host/higgs.hpp) on the GPU,
// written in the shape of the reference's own Rust tests: build inputs with
// Array::from_slice, call the layer-level function, read results back and
// assert. Expected values come from the oracle (oracle/liboracle.so, the CPU
// restatement of MLX's CPU-device ops) on the same seeded inputs, or from the
// reference tests' own constants (qwen3_next.rs:1689-1697, 1927-1961).
//
//   test_host_api            run every test, print one line each, exit 1 on failure
//   test_host_api --list     print the test names (needs no GPU)
//   test_host_api NAME...    run the named tests only
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <map>
#include <string>
#include <tuple>
#include <vector>

#include <unistd.h>

#include "higgs.hpp"

extern "C" {
#include "oracle.h"
}

using higgs::Array;
using higgs::Dtype;
using higgs::Shape;

namespace {

struct Case {
  const char* name;
  std::function<void()> fn;
};
std::vector<Case>& registry() {
  static std::vector<Case> r;
  return r;
}
struct Register {
  Register(const char* n, std::function<void()> f) { registry().push_back({n, std::move(f)}); }
};

#define TEST(name)                                 \
  static void name();                              \
  static Register reg_##name(#name, name);         \
  static void name()

struct Failure {
  std::string msg;
};

#define ASSERT(cond, ...)                                                            \
  do {                                                                               \
    if (!(cond)) {                                                                   \
      char buf_[512];                                                                \
      std::snprintf(buf_, sizeof buf_, __VA_ARGS__);                                 \
      throw Failure{std::string(__FILE__ ":") + std::to_string(__LINE__) + ": " +   \
                    #cond + ": " + buf_};                                            \
    }                                                                                \
  } while (0)

// ---- seeded inputs (the oracle's generators) ----
std::vector<float> normal(uint64_t key, int64_t n, float mean = 0.0f, float sd = 1.0f) {
  std::vector<float> v(n);
  or_fill_normal(key, mean, sd, v.data(), n);
  return v;
}
std::vector<float> uniform(uint64_t key, int64_t n, float lo, float hi) {
  std::vector<float> v(n);
  or_fill_uniform(key, lo, hi, v.data(), n);
  return v;
}
// f32 values as the 16-bit codes of dtype dt (round to nearest even)
std::vector<uint16_t> bits_of(const std::vector<float>& v, int dt) {
  std::vector<uint16_t> b(v.size());
  or_convert_from_f32(dt, v.data(), b.data(), static_cast<int64_t>(v.size()));
  return b;
}
Array dev16(const std::vector<uint16_t>& b, const Shape& s, Dtype dt) {
  return Array::from_bits(b.data(), b.size(), s, dt);
}
int64_t count_mismatch(const std::vector<uint16_t>& a, const std::vector<uint16_t>& b,
                       int64_t* first) {
  int64_t bad = 0;
  *first = -1;
  for (std::size_t i = 0; i < a.size(); ++i)
    if (a[i] != b[i]) {
      if (*first < 0) *first = static_cast<int64_t>(i);
      ++bad;
    }
  return bad;
}

#define ASSERT_BITS_EQ(got, want)                                                          \
  do {                                                                                     \
    ASSERT((got).size() == (want).size(), "size %zu vs %zu", (got).size(), (want).size()); \
    int64_t f_;                                                                            \
    const int64_t bad_ = count_mismatch((got), (want), &f_);                               \
    ASSERT(bad_ == 0, "%lld of %zu differ; first at %lld: 0x%04x vs 0x%04x",               \
           (long long)bad_, (got).size(), (long long)f_, f_ >= 0 ? (got)[f_] : 0,          \
           f_ >= 0 ? (want)[f_] : 0);                                                      \
  } while (0)

// ulp distance between two bf16/f16 codes of the same sign class
int ulp16(uint16_t a, uint16_t b) {
  auto key = [](uint16_t v) { return (v & 0x8000) ? -static_cast<int>(v & 0x7fff) : static_cast<int>(v); };
  return std::abs(key(a) - key(b));
}

// ---------------------------------------------------------------- reference tests
// qwen3_next.rs:1689-1697
TEST(test_swiglu) {
  const float g[] = {1.0f, -1.0f, 0.5f};
  const float x[] = {2.0f, 3.0f, 4.0f};
  Array gate = Array::from_slice(g, 3, {1, 3});
  Array xx = Array::from_slice(x, 3, {1, 3});
  Array result = higgs::swiglu(gate, xx);
  ASSERT(result.shape() == Shape({1, 3}), "shape %s", higgs::format_shape(result.shape()).c_str());
  // silu(1.0) * 2.0 = 0.7311 * 2.0 ~= 1.462
  const float first = result.slice(1, 0, 1).item();
  ASSERT(first > 1.0f, "first = %g", first);
}

// qwen3_next.rs:1927-1961
TEST(test_swiglu_numeric_correctness) {
  auto one = [](float g, float x) {
    return higgs::swiglu(Array::from_slice(&g, 1, {1, 1}), Array::from_slice(&x, 1, {1, 1})).item();
  };
  const float v1 = one(0.0f, 5.0f);
  ASSERT(std::fabs(v1 - 0.0f) < 1e-6f, "silu(0)*5 should be 0, got %g", v1);
  const float v2 = one(1.0f, 1.0f);
  ASSERT(std::fabs(v2 - 0.7310586f) < 1e-4f, "silu(1)*1 should be ~0.7311, got %g", v2);
  const float v3 = one(-1.0f, 2.0f);
  ASSERT(std::fabs(v3 - (-0.5378828f)) < 1e-4f, "silu(-1)*2 should be ~-0.5379, got %g", v3);
}

// ---------------------------------------------------------------- host plumbing
TEST(test_from_slice_rounds_like_the_oracle) {
  std::vector<float> v = normal(11, 4096, 0.0f, 100.0f);
  const float specials[] = {0.0f, -0.0f, 1.0f, 65504.0f, 65519.99f, 65520.0f, 1e-8f, -6.1e-5f,
                            5.96e-8f, 2.98e-8f, 1.00390625f, 1.01171875f, INFINITY, -INFINITY,
                            3.0e38f, 1e-40f};
  v.insert(v.end(), std::begin(specials), std::end(specials));
  for (int dt : {OR_BF16, OR_F16}) {
    const Dtype d = dt == OR_BF16 ? Dtype::Bfloat16 : Dtype::Float16;
    Array a = Array::from_slice(v, {static_cast<int64_t>(v.size())}, d);
    auto got = a.to_bits();
    auto want = bits_of(v, dt);
    ASSERT_BITS_EQ(got, want);
    std::vector<float> back(v.size());
    or_convert_to_f32(dt, want.data(), back.data(), static_cast<int64_t>(v.size()));
    auto f = a.to_f32();
    for (std::size_t i = 0; i < v.size(); ++i)
      ASSERT(std::memcmp(&f[i], &back[i], 4) == 0, "to_f32 mismatch at %zu", i);
  }
}

TEST(test_views_read_back_in_logical_order) {
  std::vector<float> v(2 * 3 * 4);
  for (std::size_t i = 0; i < v.size(); ++i) v[i] = static_cast<float>(i);
  Array a = Array::from_slice(v, {2, 3, 4});
  auto t = a.transpose({2, 0, 1}).to_f32();  // [4, 2, 3]
  for (int k = 0; k < 4; ++k)
    for (int i = 0; i < 2; ++i)
      for (int j = 0; j < 3; ++j)
        ASSERT(t[(k * 2 + i) * 3 + j] == v[(i * 3 + j) * 4 + k], "transpose at %d,%d,%d", k, i, j);
  auto s = a.slice(2, 1, 3).reshape({2, 3, 2, 1}).to_f32();
  ASSERT(s.size() == 12 && s[0] == 1.0f && s[1] == 2.0f && s[2] == 5.0f, "slice/reshape view");
  bool threw = false;
  try {
    a.transpose({1, 0, 2}).reshape({24});
  } catch (const higgs::Exception&) {
    threw = true;
  }
  ASSERT(threw, "a reshape that needs a copy must throw");
}

// ---------------------------------------------------------------- RMSNorm
// nn::RmsNorm on the RMSNorm-alone workload: bf16 [512, 2048], eps 1e-5.
TEST(test_rms_norm_matches_oracle_bf16) {
  const int64_t R = 512, N = 2048;
  auto xb = bits_of(normal(1000, R * N), OR_BF16);
  auto wb = bits_of(normal(1001, N, 1.0f, 0.02f), OR_BF16);
  higgs::nn::RmsNorm norm{dev16(wb, {N}, Dtype::Bfloat16), 1e-5f};
  Array y = norm.forward(dev16(xb, {R, N}, Dtype::Bfloat16));
  ASSERT(y.dtype() == Dtype::Bfloat16, "dtype %s", higgs::name_of(y.dtype()));
  std::vector<uint16_t> want(R * N);
  ASSERT(or_rms_norm(xb.data(), OR_BF16, N, wb.data(), OR_BF16, 0, 1e-5f, want.data(), OR_BF16, N,
                     R, N) == 0, "oracle");
  auto got = y.to_bits();
  ASSERT_BITS_EQ(got, want);
  // fast::rms_norm is the same call
  auto got2 = higgs::fast::rms_norm(dev16(xb, {R, N}, Dtype::Bfloat16), norm.weight, 1e-5f).to_bits();
  ASSERT_BITS_EQ(got2, want);
}

// Gemma's (1 + w) norm: weights shifted in f32 at load time (gemma2.rs:799-826),
// so the result is Float32.
TEST(test_rms_norm_gemma_plus_one_is_float32) {
  const int64_t R = 64, N = 3584;
  auto xb = bits_of(normal(2000, R * N), OR_BF16);
  auto wb = bits_of(normal(2001, N, 0.0f, 0.02f), OR_BF16);
  higgs::nn::RmsNorm norm{dev16(wb, {N}, Dtype::Bfloat16), 1e-6f, true};
  Array y = norm.forward(dev16(xb, {4, 16, N}, Dtype::Bfloat16));
  ASSERT(y.dtype() == Dtype::Float32 && y.shape() == Shape({4, 16, N}), "%s", y.describe().c_str());
  std::vector<float> want(R * N);
  ASSERT(or_rms_norm(xb.data(), OR_BF16, N, wb.data(), OR_BF16, 1, 1e-6f, want.data(), OR_F32, N, R,
                     N) == 0, "oracle");
  auto got = y.to_f32();
  for (int64_t i = 0; i < R * N; ++i)
    ASSERT(std::memcmp(&got[i], &want[i], 4) == 0, "at %lld: %.9g vs %.9g", (long long)i, got[i], want[i]);
}

// Rows read through a row stride (a column slice of a wider buffer).
TEST(test_rms_norm_strided_rows_f16) {
  const int64_t R = 96, W = 1536, N = 1024;
  auto xb = bits_of(normal(3000, R * W), OR_F16);
  auto wb = bits_of(normal(3001, N, 1.0f, 0.02f), OR_F16);
  Array x = dev16(xb, {R, W}, Dtype::Float16).slice(1, 256, 256 + N);
  Array y = higgs::fast::rms_norm(x, dev16(wb, {N}, Dtype::Float16), 1e-6f);
  std::vector<uint16_t> want(R * N);
  ASSERT(or_rms_norm(xb.data() + 256, OR_F16, W, wb.data(), OR_F16, 0, 1e-6f, want.data(), OR_F16, N,
                     R, N) == 0, "oracle");
  auto got = y.to_bits();
  ASSERT_BITS_EQ(got, want);
}

// ---------------------------------------------------------------- RoPE
// Oracle RoPE of x [B, H, L, D] (contiguous) into the same layout.
std::vector<uint16_t> oracle_rope(const std::vector<uint16_t>& xb, int64_t B, int64_t H, int64_t L,
                                  int64_t D, int dims, const std::vector<float>& inv, int offset,
                                  const int32_t* offsets, const uint16_t* norm_w = nullptr) {
  std::vector<uint16_t> y(xb.size());
  const int64_t s[3] = {H * L * D, D, L * D};
  const int rc = or_norm_rope(OR_BF16, xb.data(), s, y.data(), s, B, L, H, D, norm_w, OR_BF16, 1e-6f,
                              dims, inv.data(), 1.0f, offset, offsets);
  if (rc) throw Failure{"oracle rope failed"};
  return y;
}

// apply_rope (utils.rs:16-26) on the post-transpose [B, H, L, D] layout.
TEST(test_apply_rope_default_bf16) {
  const int64_t B = 2, H = 4, L = 16, D = 64;
  auto xb = bits_of(normal(4000, B * H * L * D), OR_BF16);
  higgs::nn::Rope rope;
  rope.dimensions = 64;
  rope.base = 10000.0f;
  Array y = higgs::apply_rope(dev16(xb, {B, H, L, D}, Dtype::Bfloat16), rope, 5);
  std::vector<float> inv(32);
  or_rope_inv_freq(10000.0f, 64, nullptr, inv.data());
  auto want = oracle_rope(xb, B, H, L, D, 64, inv, 5, nullptr);
  auto got = y.to_bits();
  ASSERT_BITS_EQ(got, want);
  // nn::Rope::forward and fast::rope are the same computation
  auto got2 = rope.forward(dev16(xb, {B, H, L, D}, Dtype::Bfloat16), 5).to_bits();
  ASSERT_BITS_EQ(got2, want);
}

// llama3-scaled frequencies passed as fast::rope's freqs (deepseek_v2.rs:222-225).
TEST(test_apply_rope_llama3_freqs) {
  const int64_t B = 1, H = 8, L = 64, D = 64;
  auto freqs = higgs::llama3_rope_freqs(500000.0f, 64, 32.0f, 1.0f, 4.0f, 8192.0f);
  std::vector<float> want_f(32);
  or_llama3_freqs(500000.0f, 64, 32.0f, 1.0f, 4.0f, 8192.0f, want_f.data());
  for (int i = 0; i < 32; ++i)
    ASSERT(std::memcmp(&freqs[i], &want_f[i], 4) == 0, "freq %d: %.9g vs %.9g", i, freqs[i], want_f[i]);
  auto xb = bits_of(normal(4100, B * H * L * D), OR_BF16);
  higgs::nn::Rope rope;
  rope.dimensions = 64;
  rope.freqs = freqs;
  Array y = higgs::apply_rope(dev16(xb, {B, H, L, D}, Dtype::Bfloat16), rope, 1000);
  std::vector<float> inv(32);
  or_rope_inv_freq(0.0f, 64, want_f.data(), inv.data());
  auto want = oracle_rope(xb, B, H, L, D, 64, inv, 1000, nullptr);
  auto got = y.to_bits();
  ASSERT_BITS_EQ(got, want);
}

// Partial rotary (qwen3_next.rs:680-703): dims [64, 256) pass through bit-exactly.
TEST(test_apply_rope_partial_passes_tail_through) {
  const int64_t B = 3, H = 16, L = 1, D = 256;
  auto xb = bits_of(normal(4200, B * H * L * D), OR_BF16);
  higgs::nn::Rope rope;
  rope.dimensions = 64;
  rope.base = 1e7f;
  auto got = higgs::apply_rope(dev16(xb, {B, H, L, D}, Dtype::Bfloat16), rope, 12345).to_bits();
  for (int64_t r = 0; r < B * H * L; ++r)
    for (int64_t d = 64; d < D; ++d)
      ASSERT(got[r * D + d] == xb[r * D + d], "tail changed at row %lld dim %lld", (long long)r, (long long)d);
  std::vector<float> inv(32);
  or_rope_inv_freq(1e7f, 64, nullptr, inv.data());
  auto want = oracle_rope(xb, B, H, L, D, 64, inv, 12345, nullptr);
  ASSERT_BITS_EQ(got, want);
}

// Per-sequence offsets replace forward_batched's per-request rope loop
// (transformer.rs:747-802): one batched call equals the loop, bit for bit.
TEST(test_apply_rope_batched_equals_per_request_loop) {
  const int64_t B = 5, H = 2, L = 1, D = 256;
  auto xb = bits_of(normal(4300, B * H * L * D), OR_BF16);
  const std::vector<int32_t> offs = {1, 100, 32768, 7, 4095};
  higgs::nn::Rope rope;
  rope.dimensions = 64;
  rope.base = 1e7f;
  Array x = dev16(xb, {B, H, L, D}, Dtype::Bfloat16);
  auto batched = higgs::apply_rope_batched(x, rope, Array::from_slice(offs, {B})).to_bits();
  for (int64_t b = 0; b < B; ++b) {
    auto one = higgs::apply_rope(x.slice(0, b, b + 1), rope, offs[b]).to_bits();
    for (int64_t i = 0; i < H * L * D; ++i)
      ASSERT(batched[b * H * L * D + i] == one[i], "sequence %lld element %lld", (long long)b, (long long)i);
  }
  std::vector<float> inv(32);
  or_rope_inv_freq(1e7f, 64, nullptr, inv.data());
  auto want = oracle_rope(xb, B, H, L, D, 64, inv, 0, offs.data());
  ASSERT_BITS_EQ(batched, want);
}

// q_norm / k_norm, transpose and apply_rope (transformer.rs:264-287) in one
// call: q and k in the projection layout [B, L, H, D], results [B, H, L, D].
TEST(test_qk_norm_rope_matches_oracle) {
  const int64_t B = 2, L = 8, Hq = 8, Hk = 2, D = 128;
  auto qb = bits_of(normal(5000, B * L * Hq * D), OR_BF16);
  auto kb = bits_of(normal(5001, B * L * Hk * D), OR_BF16);
  auto qwb = bits_of(normal(5002, D, 1.0f, 0.02f), OR_BF16);
  auto kwb = bits_of(normal(5003, D, 1.0f, 0.02f), OR_BF16);
  higgs::nn::RmsNorm qn{dev16(qwb, {D}, Dtype::Bfloat16), 1e-6f};
  higgs::nn::RmsNorm kn{dev16(kwb, {D}, Dtype::Bfloat16), 1e-6f};
  higgs::nn::Rope rope;
  rope.dimensions = 128;
  rope.base = 1e6f;
  auto qk = higgs::qk_norm_rope(dev16(qb, {B, L, Hq, D}, Dtype::Bfloat16),
                                dev16(kb, {B, L, Hk, D}, Dtype::Bfloat16), &qn, &kn, rope, 3);
  ASSERT(qk.first.shape() == Shape({B, Hq, L, D}), "q out %s", qk.first.describe().c_str());
  std::vector<float> inv(64);
  or_rope_inv_freq(1e6f, 128, nullptr, inv.data());
  for (int t = 0; t < 2; ++t) {
    const int64_t H = t ? Hk : Hq;
    const auto& in = t ? kb : qb;
    std::vector<uint16_t> want(in.size());
    const int64_t xs[3] = {L * H * D, H * D, D};
    const int64_t ys[3] = {H * L * D, D, L * D};
    ASSERT(or_norm_rope(OR_BF16, in.data(), xs, want.data(), ys, B, L, H, D, t ? kwb.data() : qwb.data(),
                        OR_BF16, 1e-6f, 128, inv.data(), 1.0f, 3, nullptr) == 0, "oracle");
    auto got = (t ? qk.second : qk.first).to_bits();
    ASSERT_BITS_EQ(got, want);
  }
}

// ---------------------------------------------------------------- gated norm
// GatedDeltaNet's norm: swiglu(z, norm(y)) with z read in place from the
// in_proj_qkvz output (qwen3_next.rs:1204-1205, 1214-1265).
TEST(test_gated_rms_norm_reads_z_in_place) {
  const int64_t S = 8, NK = 16, VPK = 2, DV = 128, BLK = 768;
  auto yb = bits_of(normal(6000, S * NK * VPK * DV), OR_BF16);
  auto qkvz = bits_of(normal(6001, S * NK * BLK), OR_BF16);
  auto wb = bits_of(normal(6002, DV, 1.0f, 0.02f), OR_BF16);
  Array z = dev16(qkvz, {S, NK, BLK}, Dtype::Bfloat16).slice(2, 512, 768).reshape({S, NK, VPK, DV});
  higgs::nn::RmsNorm norm{dev16(wb, {DV}, Dtype::Bfloat16), 1e-6f};
  Array out = higgs::gated_rms_norm(dev16(yb, {S, NK * VPK, DV}, Dtype::Bfloat16), z, norm);
  // the oracle takes z as plain rows
  std::vector<uint16_t> zc;
  for (int64_t s = 0; s < S; ++s)
    for (int64_t k = 0; k < NK; ++k)
      zc.insert(zc.end(), qkvz.begin() + (s * NK + k) * BLK + 512, qkvz.begin() + (s * NK + k + 1) * BLK);
  const int64_t R = S * NK * VPK;
  std::vector<uint16_t> want(R * DV);
  ASSERT(or_gated_rms_norm(OR_BF16, yb.data(), DV, zc.data(), DV, wb.data(), OR_BF16, 1e-6f, want.data(),
                           OR_BF16, DV, R, DV) == 0, "oracle");
  auto got = out.to_bits();
  ASSERT_BITS_EQ(got, want);
}

// ---------------------------------------------------------------- GLU
TEST(test_silu_mul_and_gelu_approximate_mul) {
  const int64_t R = 64, N = 1536;
  auto gb = bits_of(normal(7000, R * N, 0.0f, 3.0f), OR_BF16);
  auto ub = bits_of(normal(7001, R * N), OR_BF16);
  Array g = dev16(gb, {R, N}, Dtype::Bfloat16), u = dev16(ub, {R, N}, Dtype::Bfloat16);
  std::vector<uint16_t> want(R * N);
  ASSERT(or_glu(OR_ACT_SILU, OR_BF16, gb.data(), N, ub.data(), N, want.data(), OR_BF16, N, R, N) == 0, "oracle");
  auto silu = higgs::nn::silu_mul(g, u).to_bits();
  ASSERT_BITS_EQ(silu, want);
  ASSERT(or_glu(OR_ACT_GELU_TANH, OR_BF16, gb.data(), N, ub.data(), N, want.data(), OR_BF16, N, R, N) == 0,
         "oracle");
  // bf16 bar: within 1 ulp, or within atol 1e-3 next to zero where ulps
  // shrink without bound (rtol 1e-2 / atol 1e-3)
  auto gelu = higgs::nn::gelu_approximate_mul(g, u).to_bits();
  std::vector<float> gf(want.size()), wf(want.size());
  or_convert_to_f32(OR_BF16, gelu.data(), gf.data(), static_cast<int64_t>(gf.size()));
  or_convert_to_f32(OR_BF16, want.data(), wf.data(), static_cast<int64_t>(wf.size()));
  int64_t far = 0, exact = 0;
  for (std::size_t i = 0; i < want.size(); ++i) {
    const float d = std::fabs(gf[i] - wf[i]);
    exact += gelu[i] == want[i];
    if (ulp16(gelu[i], want[i]) > 1 && d > 1e-3f) ++far;
    ASSERT(d <= 1e-3f + 1e-2f * std::fabs(wf[i]), "GeGLU at %zu: %g vs %g", i, gf[i], wf[i]);
  }
  ASSERT(far == 0, "%lld GeGLU values are beyond 1 bf16 ulp and atol 1e-3", (long long)far);
  ASSERT(exact * 10 >= static_cast<int64_t>(want.size()) * 9, "only %lld of %zu GeGLU values exact",
         (long long)exact, want.size());
}

// phi3's fused gate_up projection (phi3.rs:261-265): two halves read in place.
TEST(test_swiglu_fused_gate_up_halves) {
  const int64_t R = 32, I = 2048;
  auto gu = bits_of(normal(7100, R * 2 * I), OR_BF16);
  Array a = dev16(gu, {R, 2 * I}, Dtype::Bfloat16);
  auto got = higgs::swiglu(a.slice(1, 0, I), a.slice(1, I, 2 * I)).to_bits();
  std::vector<uint16_t> want(R * I);
  ASSERT(or_glu(OR_ACT_SILU, OR_BF16, gu.data(), 2 * I, gu.data() + I, 2 * I, want.data(), OR_BF16, I, R,
                I) == 0, "oracle");
  ASSERT_BITS_EQ(got, want);
}

// ---------------------------------------------------------------- embedding
// nn::QuantizedEmbedding at the Llama-3.2-1B table size (vocab 128256, hidden
// 2048, group 64), bit-exact, with the first and last ids included.
TEST(test_quantized_embedding_llama_table) {
  const int64_t V = 128256, H = 2048, G = 64, T = 512;
  std::vector<uint32_t> wq(V * H / 8);
  or_fill_u32(8000, wq.data(), static_cast<int64_t>(wq.size()));
  auto sb = bits_of(uniform(8001, V * H / G, 0.005f, 0.02f), OR_BF16);
  auto bb = bits_of(uniform(8002, V * H / G, -0.1f, 0.1f), OR_BF16);
  std::vector<uint32_t> ids(T);
  or_fill_ids(8003, static_cast<uint32_t>(V), ids.data(), T);
  ids[0] = 0;
  ids[1] = static_cast<uint32_t>(V - 1);
  higgs::nn::QuantizedEmbedding emb{Array::from_slice(wq, {V, H / 8}), dev16(sb, {V, H / G}, Dtype::Bfloat16),
                                    dev16(bb, {V, H / G}, Dtype::Bfloat16), 64, 4};
  Array idv = Array::from_slice(ids, {4, T / 4});
  Array h = emb.forward(idv);
  ASSERT(h.shape() == Shape({4, T / 4, H}) && h.dtype() == Dtype::Bfloat16, "%s", h.describe().c_str());
  std::vector<uint16_t> want(T * H);
  ASSERT(or_qembed(ids.data(), OR_U32, T, wq.data(), sb.data(), bb.data(), OR_BF16, V, H, 64, 4, 0.0f,
                   want.data()) == 0, "oracle");
  auto got = h.to_bits();
  ASSERT_BITS_EQ(got, want);
  // Gemma's embedding scale fused into the gather (gemma2.rs:587-600)
  const float scale = std::sqrt(3584.0f);
  auto got_s = emb.forward_scaled(idv, scale).to_bits();
  ASSERT(or_qembed(ids.data(), OR_U32, T, wq.data(), sb.data(), bb.data(), OR_BF16, V, H, 64, 4, scale,
                   want.data()) == 0, "oracle");
  ASSERT_BITS_EQ(got_s, want);
}

// ---------------------------------------------------------------- fused forms
// The block boundary `h = x.add(r); post_attention_layernorm(h)`
// (transformer.rs:413-415) in one call, three blocks in a row.
TEST(test_add_rms_norm_block_boundaries) {
  const int64_t R = 256, N = 2048;
  auto hb = bits_of(normal(9100, R * N), OR_BF16);
  auto wb = bits_of(normal(9101, N, 1.0f, 0.02f), OR_BF16);
  higgs::nn::RmsNorm norm{dev16(wb, {N}, Dtype::Bfloat16), 1e-5f};
  Array h = dev16(hb, {R, N}, Dtype::Bfloat16);
  for (int blk = 0; blk < 3; ++blk) {
    auto rb = bits_of(normal(9110 + blk, R * N, 0.0f, 0.5f), OR_BF16);
    auto hy = higgs::add_rms_norm(h, dev16(rb, {R, N}, Dtype::Bfloat16), norm);
    std::vector<uint16_t> want_h(R * N), want_y(R * N);
    ASSERT(or_add(OR_BF16, hb.data(), N, rb.data(), N, want_h.data(), N, R, N) == 0, "oracle add");
    ASSERT(or_rms_norm(want_h.data(), OR_BF16, N, wb.data(), OR_BF16, 0, 1e-5f, want_y.data(), OR_BF16,
                       N, R, N) == 0, "oracle norm");
    auto got_h = hy.first.to_bits();
    auto got_y = hy.second.to_bits();
    ASSERT_BITS_EQ(got_h, want_h);
    ASSERT_BITS_EQ(got_y, want_y);
    h = hy.first;
    hb = want_h;
  }
}

// embed_tokens.forward(ids) then the first input_layernorm (transformer.rs:494,
// 407) in one call; Gemma's scale and (1 + w) norm (gemma2.rs:587-600, 491).
TEST(test_quantized_embedding_forward_rms_norm) {
  const int64_t V = 4096, H = 3584, G = 64, T = 300;
  std::vector<uint32_t> wq(V * H / 8);
  or_fill_u32(9200, wq.data(), static_cast<int64_t>(wq.size()));
  auto sb = bits_of(uniform(9201, V * H / G, 0.005f, 0.02f), OR_BF16);
  auto bb = bits_of(uniform(9202, V * H / G, -0.1f, 0.1f), OR_BF16);
  auto wb = bits_of(normal(9203, H, 0.0f, 0.02f), OR_BF16);
  std::vector<uint32_t> ids(T);
  or_fill_ids(9204, static_cast<uint32_t>(V), ids.data(), T);
  higgs::nn::QuantizedEmbedding emb{Array::from_slice(wq, {V, H / 8}), dev16(sb, {V, H / G}, Dtype::Bfloat16),
                                    dev16(bb, {V, H / G}, Dtype::Bfloat16), 64, 4};
  higgs::nn::RmsNorm norm{dev16(wb, {H}, Dtype::Bfloat16), 1e-6f, true};
  const float scale = std::sqrt(3584.0f);
  auto hy = emb.forward_rms_norm(Array::from_slice(ids, {T}), norm, scale);
  ASSERT(hy.second.dtype() == Dtype::Float32, "%s", hy.second.describe().c_str());
  std::vector<uint16_t> want_h(T * H);
  std::vector<float> want_y(T * H);
  ASSERT(or_qembed(ids.data(), OR_U32, T, wq.data(), sb.data(), bb.data(), OR_BF16, V, H, 64, 4, scale,
                   want_h.data()) == 0, "oracle embed");
  ASSERT(or_rms_norm(want_h.data(), OR_BF16, H, wb.data(), OR_BF16, 1, 1e-6f, want_y.data(), OR_F32, H, T,
                     H) == 0, "oracle norm");
  auto got_h = hy.first.to_bits();
  ASSERT_BITS_EQ(got_h, want_h);
  auto got_y = hy.second.to_f32();
  for (int64_t i = 0; i < T * H; ++i)
    ASSERT(std::memcmp(&got_y[i], &want_y[i], 4) == 0, "y at %lld: %.9g vs %.9g", (long long)i,
           got_y[i], want_y[i]);
}

// ---------------------------------------------------------------- gather_qmm
// SwitchMlpWeights::forward_gather (qwen3_next.rs:844-904): gate and up
// gather_qmm, swiglu, down gather_qmm. Floating-point contraction: each
// projection within 1 bf16 ulp of the oracle (or atol 1e-3 next to zero).
TEST(test_switch_mlp_forward_gather) {
  const int64_t T = 8, top_k = 4, E = 16, D = 1024, I = 256, G = 64;
  auto xb = bits_of(normal(9400, T * D), OR_BF16);
  std::vector<int32_t> idx(T * top_k);
  std::vector<uint32_t> tmp(T * top_k);
  or_fill_ids(9401, static_cast<uint32_t>(E), tmp.data(), T * top_k);
  for (size_t i = 0; i < tmp.size(); ++i) idx[i] = static_cast<int32_t>(tmp[i]);
  struct Mat { std::vector<uint32_t> w; std::vector<uint16_t> s, b; int64_t N, K; };
  auto make = [&](uint64_t key, int64_t N, int64_t K) {
    Mat m{std::vector<uint32_t>(E * N * K / 8), bits_of(uniform(key + 1, E * N * K / G, 0.005f, 0.02f), OR_BF16),
          bits_of(uniform(key + 2, E * N * K / G, -0.1f, 0.1f), OR_BF16), N, K};
    or_fill_u32(key, m.w.data(), static_cast<int64_t>(m.w.size()));
    return m;
  };
  Mat gm = make(9410, I, D), um = make(9420, I, D), dm = make(9430, D, I);
  auto ql = [&](const Mat& m) {
    return higgs::nn::QLinear{Array::from_slice(m.w, {E, m.N, m.K / 8}),
                              dev16(m.s, {E, m.N, m.K / G}, Dtype::Bfloat16),
                              dev16(m.b, {E, m.N, m.K / G}, Dtype::Bfloat16), 64, 4};
  };
  higgs::nn::SwitchMlpWeights sw{ql(gm), ql(um), ql(dm)};
  Array x = dev16(xb, {T, D}, Dtype::Bfloat16);
  Array y = sw.forward_gather(x, Array::from_slice(idx, {T, top_k}));
  ASSERT(y.shape() == Shape({T, top_k, D}), "%s", y.describe().c_str());
  // gate and up against the oracle, then down on the device's own activation
  const int64_t P = T * top_k;
  auto check_close = [&](const std::vector<uint16_t>& got, const std::vector<uint16_t>& want, const char* what) {
    std::vector<float> gf(got.size()), wf(want.size());
    or_convert_to_f32(OR_BF16, got.data(), gf.data(), static_cast<int64_t>(got.size()));
    or_convert_to_f32(OR_BF16, want.data(), wf.data(), static_cast<int64_t>(want.size()));
    for (size_t i = 0; i < got.size(); ++i) {
      const float d = std::fabs(gf[i] - wf[i]);
      ASSERT(ulp16(got[i], want[i]) <= 1 || d <= 1e-3f, "%s at %zu: %g vs %g", what, i, gf[i], wf[i]);
    }
  };
  Array idx_flat = Array::from_slice(idx, {P});
  auto g = higgs::gather_qmm(x, sw.gate_proj.weight, sw.gate_proj.scales, sw.gate_proj.biases, idx_flat, true, 64, 4, top_k);
  std::vector<uint16_t> want(P * I);
  ASSERT(or_gather_qmm(OR_BF16, xb.data(), T, D, top_k, nullptr, gm.w.data(), gm.s.data(), gm.b.data(), OR_BF16, E, I,
                       D, 64, idx.data(), P, want.data(), I) == 0, "oracle gate");
  check_close(g.to_bits(), want, "gate");
  auto u = higgs::gather_qmm(x, sw.up_proj.weight, sw.up_proj.scales, sw.up_proj.biases, idx_flat, true, 64, 4, top_k);
  auto act = higgs::swiglu(g, u);
  auto actb = act.to_bits();
  std::vector<uint16_t> want_d(P * D);
  ASSERT(or_gather_qmm(OR_BF16, actb.data(), P, I, 1, nullptr, dm.w.data(), dm.s.data(), dm.b.data(), OR_BF16, E, D,
                       I, 64, idx.data(), P, want_d.data(), D) == 0, "oracle down");
  check_close(y.to_bits(), want_d, "down");
}

// QLinear::forward = quantized_matmul (qwen3_next.rs:174-221): decode (8
// rows, the per-row path), a batch of 64 rows (the matrix-core path for few
// rows) and 600 rows as [2, 300, K] (the prefill path), against the oracle
// within 1 bf16 ulp (or 1e-3 next to zero), >= 99% bit-identical.
TEST(test_qlinear_forward_matches_oracle) {
  const int64_t N = 320, K = 1024, G = 64;
  std::vector<uint32_t> w(N * K / 8);
  or_fill_u32(9600, w.data(), static_cast<int64_t>(w.size()));
  auto sb = bits_of(uniform(9601, N * K / G, 0.005f, 0.02f), OR_BF16);
  auto bb = bits_of(uniform(9602, N * K / G, -0.1f, 0.1f), OR_BF16);
  higgs::nn::QLinear lin{Array::from_slice(w, {N, K / 8}), dev16(sb, {N, K / G}, Dtype::Bfloat16),
                         dev16(bb, {N, K / G}, Dtype::Bfloat16), 64, 4};
  std::vector<int32_t> zeros_idx;
  for (int64_t M : {8, 64, 600}) {
    auto xb = bits_of(normal(9610 + M, M * K), OR_BF16);
    Array x = M == 600 ? dev16(xb, {2, 300, K}, Dtype::Bfloat16) : dev16(xb, {M, K}, Dtype::Bfloat16);
    Array y = lin.forward(x);
    ASSERT(y.ndim() == x.ndim() && y.dim(-1) == N, "%s", y.describe().c_str());
    zeros_idx.assign(M, 0);
    std::vector<uint16_t> want(M * N);
    ASSERT(or_gather_qmm(OR_BF16, xb.data(), M, K, 1, nullptr, w.data(), sb.data(), bb.data(), OR_BF16, 1, N, K, 64,
                         zeros_idx.data(), M, want.data(), N) == 0,
           "oracle");
    auto got = y.to_bits();
    std::vector<float> gf(got.size()), wf(want.size());
    or_convert_to_f32(OR_BF16, got.data(), gf.data(), static_cast<int64_t>(got.size()));
    or_convert_to_f32(OR_BF16, want.data(), wf.data(), static_cast<int64_t>(want.size()));
    int64_t exact = 0;
    for (size_t i = 0; i < got.size(); ++i) {
      ASSERT(ulp16(got[i], want[i]) <= 1 || std::fabs(gf[i] - wf[i]) <= 1e-3f, "M=%lld y[%zu] %g vs %g",
             (long long)M, i, gf[i], wf[i]);
      exact += got[i] == want[i];
    }
    ASSERT(exact >= 0.99 * static_cast<double>(got.size()), "M=%lld: %lld of %zu bit-identical", (long long)M,
           (long long)exact, got.size());
  }
}

// The reference's gated-delta kernel tests (qwen3_next.rs:1700-1722,
// 2421-2450): all-ones q, k, v and a, zero a_log, dt_bias, b and state, Hk 2,
// Hv 4, Dk = Dv = 32, f32. One step gives delta = 1/2, s = 1/2 everywhere and
// y = 32 / 2 = 16 exactly; a second step from that state equals the oracle's,
// and one two-step call equals two one-step calls (sequential dependence).
// Then Qwen3-Next's decode shape in bf16 with the fused q/k norm against the
// oracle (1 ulp, atol 1e-3), and a 96-step prefill (>= 99% bit-identical).
TEST(test_gated_delta_reference_cases_and_decode) {
  const int64_t B = 1, Hk = 2, Dk = 32, Hv = 4, Dv = 32;
  auto ones = [](int64_t n) { return std::vector<float>(n, 1.0f); };
  auto zeros = [](int64_t n) { return std::vector<float>(n, 0.0f); };
  auto f32 = [](const std::vector<float>& v, const Shape& s) { return Array::from_slice(v, s); };
  for (int64_t T : {1, 2}) {
    Array q = f32(ones(B * T * Hk * Dk), {B, T, Hk, Dk});
    Array v = f32(ones(B * T * Hv * Dv), {B, T, Hv, Dv});
    Array a = f32(ones(B * T * Hv), {B, T, Hv}), b = f32(zeros(B * T * Hv), {B, T, Hv});
    Array al = f32(zeros(Hv), {Hv}), db = f32(zeros(Hv), {Hv});
    Array s0 = f32(zeros(B * Hv * Dv * Dk), {B, Hv, Dv, Dk});
    auto [y, s] = higgs::gated_delta(q, q, v, al, a, db, b, &s0);
    ASSERT(y.shape() == Shape({B, T, Hv, Dv}) && s.shape() == Shape({B, Hv, Dv, Dk}), "%s",
           y.describe().c_str());
    auto yv = y.to_f32();
    for (int64_t i = 0; i < Hv * Dv; ++i) ASSERT(yv[i] == 16.0f, "T=%lld y[%lld] = %g", (long long)T, (long long)i, yv[i]);
    // the oracle on the same inputs
    std::vector<float> oy(B * T * Hv * Dv), os(B * Hv * Dv * Dk);
    auto qh = ones(B * T * Hk * Dk), vh = ones(B * T * Hv * Dv), ah = ones(B * T * Hv), bh = zeros(B * T * Hv);
    auto alh = zeros(Hv), sh = zeros(B * Hv * Dv * Dk);
    ASSERT(or_gated_delta(OR_F32, qh.data(), qh.data(), vh.data(), alh.data(), ah.data(), alh.data(), bh.data(),
                          OR_F32, sh.data(), nullptr, nullptr, 1e-6f, B, T, Hk, Dk, Hv, Dv, oy.data(), os.data()) == 0,
           "oracle");
    for (size_t i = 0; i < oy.size(); ++i)
      ASSERT(std::fabs(yv[i] - oy[i]) <= 1e-4f * std::max(1.0f, std::fabs(oy[i])), "T=%lld y[%zu] %g vs %g",
             (long long)T, i, yv[i], oy[i]);
    if (T == 1) {
      // state passthrough: a second one-step call from s equals the T = 2 run
      auto [y2, s2] = higgs::gated_delta(q, q, v, al, a, db, b, &s);
      Array q2 = f32(ones(B * 2 * Hk * Dk), {B, 2, Hk, Dk}), v2 = f32(ones(B * 2 * Hv * Dv), {B, 2, Hv, Dv});
      Array a2 = f32(ones(B * 2 * Hv), {B, 2, Hv}), b2 = f32(zeros(B * 2 * Hv), {B, 2, Hv});
      auto [yy, ss] = higgs::gated_delta(q2, q2, v2, al, a2, db, b2, &s0);
      auto y2v = y2.to_f32(), yyv = yy.to_f32(), s2v = s2.to_f32(), ssv = ss.to_f32();
      ASSERT(y2v[0] != 16.0f, "the second step must see the first step's state");
      for (int64_t i = 0; i < Hv * Dv; ++i)
        ASSERT(std::fabs(y2v[i] - yyv[Hv * Dv + i]) <= 1e-5f * std::fabs(yyv[Hv * Dv + i]), "step 2 y[%lld]", (long long)i);
      for (size_t i = 0; i < s2v.size(); ++i)
        ASSERT(std::fabs(s2v[i] - ssv[i]) <= 1e-5f * std::max(1.0f, std::fabs(ssv[i])), "step 2 state[%zu]", i);
    }
  }
  // Qwen3-Next decode: 8 sequences, Hk 16, Dk 128, Hv 32, Dv 128, bf16, fused norm
  const int64_t Bd = 8, Hkd = 16, Dkd = 128, Hvd = 32, Dvd = 128;
  auto bq = bits_of(uniform(9500, Bd * Hkd * Dkd, -1, 1), OR_BF16), bk = bits_of(uniform(9501, Bd * Hkd * Dkd, -1, 1), OR_BF16);
  auto bv = bits_of(uniform(9502, Bd * Hvd * Dvd, -1, 1), OR_BF16);
  auto ba = bits_of(uniform(9503, Bd * Hvd, -1, 1), OR_BF16), bb = bits_of(uniform(9504, Bd * Hvd, -1, 1), OR_BF16);
  auto bs = bits_of(uniform(9505, Bd * Hvd * Dvd * Dkd, -0.1f, 0.1f), OR_BF16);
  auto alog = uniform(9506, Hvd, -1, 0), dtb = uniform(9507, Hvd, -0.5f, 0.5f);
  auto [wq, wk] = higgs::gdn_qk_norm_weights(Dkd, Dtype::Bfloat16);
  Array st = dev16(bs, {Bd, Hvd, Dvd, Dkd}, Dtype::Bfloat16);
  Array al = f32(alog, {Hvd}), db = f32(dtb, {Hvd});
  auto [y, s] = higgs::gated_delta(dev16(bq, {Bd, 1, Hkd, Dkd}, Dtype::Bfloat16), dev16(bk, {Bd, 1, Hkd, Dkd}, Dtype::Bfloat16),
                                   dev16(bv, {Bd, 1, Hvd, Dvd}, Dtype::Bfloat16), al, dev16(ba, {Bd, 1, Hvd}, Dtype::Bfloat16),
                                   db, dev16(bb, {Bd, 1, Hvd}, Dtype::Bfloat16), &st, &wq, &wk);
  auto wqb = wq.to_bits(), wkb = wk.to_bits();
  std::vector<uint16_t> oy(Bd * Hvd * Dvd), os(bs.size());
  ASSERT(or_gated_delta(OR_BF16, bq.data(), bk.data(), bv.data(), alog.data(), ba.data(), dtb.data(), bb.data(), OR_F32,
                        bs.data(), wqb.data(), wkb.data(), 1e-6f, Bd, 1, Hkd, Dkd, Hvd, Dvd, oy.data(), os.data()) == 0,
         "oracle decode");
  for (auto [got, want, what] : {std::tuple{y.to_bits(), oy, "y"}, std::tuple{s.to_bits(), os, "state"}}) {
    std::vector<float> gf(got.size()), wf(want.size());
    or_convert_to_f32(OR_BF16, got.data(), gf.data(), static_cast<int64_t>(got.size()));
    or_convert_to_f32(OR_BF16, want.data(), wf.data(), static_cast<int64_t>(want.size()));
    for (size_t i = 0; i < got.size(); ++i)
      ASSERT(ulp16(got[i], want[i]) <= 1 || std::fabs(gf[i] - wf[i]) <= 1e-3f, "%s[%zu] %g vs %g", what, i, gf[i], wf[i]);
  }
  // a 96-step bf16 prefill with the fused norm (the chunked matrix-core form,
  // a ragged last chunk), through the same call
  const int64_t Tp = 96, Hkp = 2, Hvp = 4, Dvp = 64;
  auto pq = bits_of(uniform(9510, Tp * Hkp * Dkd, -1, 1), OR_BF16), pk = bits_of(uniform(9511, Tp * Hkp * Dkd, -1, 1), OR_BF16);
  auto pv = bits_of(uniform(9512, Tp * Hvp * Dvp, -1, 1), OR_BF16);
  auto pa = bits_of(uniform(9513, Tp * Hvp, -1, 1), OR_BF16), pb = bits_of(uniform(9514, Tp * Hvp, -1, 1), OR_BF16);
  auto ps = bits_of(uniform(9515, Hvp * Dvp * Dkd, -0.1f, 0.1f), OR_BF16);
  auto palog = uniform(9516, Hvp, -1, 0), pdtb = uniform(9517, Hvp, -0.5f, 0.5f);
  Array pst = dev16(ps, {1, Hvp, Dvp, Dkd}, Dtype::Bfloat16);
  auto [py, pso] = higgs::gated_delta(dev16(pq, {1, Tp, Hkp, Dkd}, Dtype::Bfloat16), dev16(pk, {1, Tp, Hkp, Dkd}, Dtype::Bfloat16),
                                      dev16(pv, {1, Tp, Hvp, Dvp}, Dtype::Bfloat16), f32(palog, {Hvp}),
                                      dev16(pa, {1, Tp, Hvp}, Dtype::Bfloat16), f32(pdtb, {Hvp}),
                                      dev16(pb, {1, Tp, Hvp}, Dtype::Bfloat16), &pst, &wq, &wk);
  std::vector<uint16_t> opy(Tp * Hvp * Dvp), ops(ps.size());
  ASSERT(or_gated_delta(OR_BF16, pq.data(), pk.data(), pv.data(), palog.data(), pa.data(), pdtb.data(), pb.data(), OR_F32,
                        ps.data(), wqb.data(), wkb.data(), 1e-6f, 1, Tp, Hkp, Dkd, Hvp, Dvp, opy.data(), ops.data()) == 0,
         "oracle prefill");
  for (auto [got, want, what] : {std::tuple{py.to_bits(), opy, "prefill y"}, std::tuple{pso.to_bits(), ops, "prefill state"}}) {
    std::vector<float> gf(got.size()), wf(want.size());
    or_convert_to_f32(OR_BF16, got.data(), gf.data(), static_cast<int64_t>(got.size()));
    or_convert_to_f32(OR_BF16, want.data(), wf.data(), static_cast<int64_t>(want.size()));
    size_t same = 0;
    for (size_t i = 0; i < got.size(); ++i) {
      same += got[i] == want[i];
      ASSERT(ulp16(got[i], want[i]) <= 1 || std::fabs(gf[i] - wf[i]) <= 1e-3f, "%s[%zu] %g vs %g", what, i, gf[i], wf[i]);
    }
    ASSERT(same >= got.size() * 99 / 100, "%s: %zu of %zu bit-identical", what, same, got.size());
  }
}

// ---------------------------------------------------------------- checkpoints
// A safetensors file written byte by byte: an 8-byte little-endian header
// length, the JSON header, then the tensors' bytes in header order.
struct StTensorSpec {
  std::string name, dtype;
  Shape shape;
  std::vector<unsigned char> bytes;
};
template <class T>
StTensorSpec st_tensor(const std::string& name, const std::string& dtype, const Shape& shape,
                       const std::vector<T>& v) {
  StTensorSpec t{name, dtype, shape, {}};
  t.bytes.resize(v.size() * sizeof(T));
  std::memcpy(t.bytes.data(), v.data(), t.bytes.size());
  return t;
}
void write_safetensors(const std::string& path, const std::vector<StTensorSpec>& ts) {
  std::string h = "{\"__metadata__\":{\"format\":\"mlx\"}";
  size_t off = 0;
  for (const auto& t : ts) {
    h += ",\"" + t.name + "\":{\"dtype\":\"" + t.dtype + "\",\"shape\":[";
    for (size_t i = 0; i < t.shape.size(); ++i) h += (i ? "," : "") + std::to_string(t.shape[i]);
    h += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + t.bytes.size()) + "]}";
    off += t.bytes.size();
  }
  h += "}";
  FILE* f = std::fopen(path.c_str(), "wb");
  if (!f) throw Failure{"cannot write " + path};
  const uint64_t n = h.size();
  unsigned char len[8];
  for (int i = 0; i < 8; ++i) len[i] = (unsigned char)(n >> (8 * i));
  std::fwrite(len, 1, 8, f);
  std::fwrite(h.data(), 1, h.size(), f);
  for (const auto& t : ts) std::fwrite(t.bytes.data(), 1, t.bytes.size(), f);
  std::fclose(f);
}

// load_quantized_safetensors_weights (lib.rs:600-632) over a sharded MLX
// checkpoint: flat keys land on the `.inner.` parameter names, and the loaded
// tensors drive the embedding + first norm bit-exactly.
TEST(test_load_quantized_checkpoint_drives_embedding_and_norm) {
  const int64_t V = 2048, H = 1024, G = 64, T = 200;
  char tmpl[] = "/tmp/higgs_ckpt_XXXXXX";
  const char* dir = mkdtemp(tmpl);
  ASSERT(dir != nullptr, "mkdtemp");
  std::vector<uint32_t> wq(V * H / 8);
  or_fill_u32(9300, wq.data(), static_cast<int64_t>(wq.size()));
  auto sb = bits_of(uniform(9301, V * H / G, 0.005f, 0.02f), OR_BF16);
  auto bb = bits_of(uniform(9302, V * H / G, -0.1f, 0.1f), OR_BF16);
  auto lb = bits_of(normal(9303, H, 1.0f, 0.02f), OR_BF16);
  const std::string d = dir;
  write_safetensors(d + "/model-00001-of-00002.safetensors",
                    {st_tensor("model.embed_tokens.weight", "U32", {V, H / 8}, wq),
                     st_tensor("model.embed_tokens.scales", "BF16", {V, H / G}, sb),
                     st_tensor("model.embed_tokens.biases", "BF16", {V, H / G}, bb)});
  write_safetensors(d + "/model-00002-of-00002.safetensors",
                    {st_tensor("model.layers.0.input_layernorm.weight", "BF16", {H}, lb)});
  FILE* idx = std::fopen((d + "/model.safetensors.index.json").c_str(), "w");
  std::fprintf(idx, "{\"metadata\": {}, \"weight_map\": {"
                    "\"model.embed_tokens.weight\": \"model-00001-of-00002.safetensors\", "
                    "\"model.embed_tokens.scales\": \"model-00001-of-00002.safetensors\", "
                    "\"model.embed_tokens.biases\": \"model-00001-of-00002.safetensors\", "
                    "\"model.layers.0.input_layernorm.weight\": \"model-00002-of-00002.safetensors\"}}");
  std::fclose(idx);

  auto files = higgs::io::collect_safetensors_files(d);
  ASSERT(files.size() == 2, "%zu files", files.size());
  std::map<std::string, Array> params = {{"model.embed_tokens.inner.weight", Array()},
                                         {"model.embed_tokens.inner.scales", Array()},
                                         {"model.embed_tokens.inner.biases", Array()},
                                         {"model.layers.0.input_layernorm.weight", Array()}};
  const size_t n = higgs::io::load_quantized_safetensors_weights(params, d, true);
  ASSERT(n == 4, "loaded %zu", n);
  higgs::nn::QuantizedEmbedding emb{params["model.embed_tokens.inner.weight"],
                                    params["model.embed_tokens.inner.scales"],
                                    params["model.embed_tokens.inner.biases"], 64, 4};
  higgs::nn::RmsNorm norm{params["model.layers.0.input_layernorm.weight"], 1e-5f};
  std::vector<uint32_t> ids(T);
  or_fill_ids(9304, static_cast<uint32_t>(V), ids.data(), T);
  auto hy = emb.forward_rms_norm(Array::from_slice(ids, {T}), norm);
  std::vector<uint16_t> want_h(T * H), want_y(T * H);
  ASSERT(or_qembed(ids.data(), OR_U32, T, wq.data(), sb.data(), bb.data(), OR_BF16, V, H, 64, 4, 0.0f,
                   want_h.data()) == 0, "oracle embed");
  ASSERT(or_rms_norm(want_h.data(), OR_BF16, H, lb.data(), OR_BF16, 0, 1e-5f, want_y.data(), OR_BF16, H, T,
                     H) == 0, "oracle norm");
  auto got_h = hy.first.to_bits();
  auto got_y = hy.second.to_bits();
  ASSERT_BITS_EQ(got_h, want_h);
  ASSERT_BITS_EQ(got_y, want_y);
  ASSERT(higgs::io::remap_quantized_key("model.norm.weight").value_or("") == "model.norm.inner.weight", "remap");
  ASSERT(!higgs::io::remap_quantized_key("lm_head").has_value(), "remap none");
  bool threw = false;
  try {
    higgs::io::collect_safetensors_files(d + "/nope");
  } catch (const higgs::Exception& e) {
    threw = std::string(e.what()).find("MissingWeight") != std::string::npos;
  }
  ASSERT(threw, "a missing checkpoint must throw MissingWeight");
  for (const auto& f : files) std::remove(f.c_str());
  std::remove((d + "/model.safetensors.index.json").c_str());
  rmdir(dir);
}

// ---------------------------------------------------------------- empty inputs
TEST(test_empty_inputs_give_empty_results) {
  higgs::nn::RmsNorm norm{Array::from_slice(std::vector<float>(64, 1.0f), {64}, Dtype::Bfloat16), 1e-5f};
  Array x = Array::empty({0, 64}, Dtype::Bfloat16);
  ASSERT(norm.forward(x).shape() == Shape({0, 64}), "rms_norm");
  ASSERT(higgs::swiglu(x, x).size() == 0, "swiglu");
  higgs::nn::Rope rope;
  rope.dimensions = 64;
  ASSERT(higgs::apply_rope(Array::empty({2, 4, 0, 64}, Dtype::Bfloat16), rope, 0).size() == 0, "rope");
}

// ---------------------------------------------------------------- errors
// Failures surface as an Exception naming the op, the library's reason and
// the operands, after the reference's Exception::custom messages
// (qwen3_next.rs:337-361).
TEST(test_errors_name_the_op_and_operands) {
  Array x = Array::from_slice(std::vector<float>(32, 1.0f), {4, 8}, Dtype::Bfloat16);
  Array w = Array::from_slice(std::vector<float>(7, 1.0f), {7}, Dtype::Bfloat16);
  try {
    higgs::fast::rms_norm(x, w, 1e-5f);
    ASSERT(false, "rms_norm with a mismatched weight returned");
  } catch (const higgs::Exception& e) {
    const std::string m = e.what();
    ASSERT(e.status() == HGK_ERR_ARG, "status %d", e.status());
    ASSERT(m.find("rms_norm failed:") == 0, "message: %s", m.c_str());
    ASSERT(m.find("[x=[4, 8]/Bfloat16 w=[7]/Bfloat16]") != std::string::npos, "message: %s", m.c_str());
  }
  higgs::nn::Rope rope;
  rope.dimensions = 8;
  rope.traditional = true;
  Array x4 = Array::from_slice(std::vector<float>(64, 1.0f), {1, 2, 4, 8}, Dtype::Bfloat16);
  try {
    higgs::apply_rope(x4, rope, 0);
    ASSERT(false, "traditional rope returned");
  } catch (const higgs::Exception& e) {
    ASSERT(e.status() == HGK_ERR_UNSUPPORTED, "status %d: %s", e.status(), e.what());
  }
  try {
    std::vector<float> f(4, 1.0f);
    higgs::fast::rope(x4, 8, false, 10000.0f, 1.0f, 0, &f);
    ASSERT(false, "rope with both base and freqs returned");
  } catch (const higgs::Exception& e) {
    ASSERT(e.status() == HGK_ERR_ARG, "status %d", e.status());
  }
  try {
    Array ids = Array::from_slice(std::vector<float>(4, 0.0f), {4});
    higgs::nn::QuantizedEmbedding emb{Array::empty({16, 8}, Dtype::Uint32), Array::empty({16, 1}, Dtype::Bfloat16),
                                      Array::empty({16, 1}, Dtype::Bfloat16), 64, 4};
    emb.forward(ids);
    ASSERT(false, "Float32 ids returned");
  } catch (const higgs::Exception& e) {
    ASSERT(std::string(e.what()).find("ids must be Int32 or Uint32") != std::string::npos, "%s", e.what());
  }
}

// ---------------------------------------------------------------- streams
// Ops follow the thread's current stream; results do not depend on it.
TEST(test_ops_run_on_the_scoped_stream) {
  const int64_t R = 256, N = 2048;
  auto xb = bits_of(normal(9000, R * N), OR_BF16);
  auto wb = bits_of(normal(9001, N, 1.0f, 0.02f), OR_BF16);
  auto base = higgs::fast::rms_norm(dev16(xb, {R, N}, Dtype::Bfloat16), dev16(wb, {N}, Dtype::Bfloat16), 1e-5f)
                  .to_bits();
  higgs::Stream s = higgs::Stream::create();
  std::vector<uint16_t> other;
  {
    higgs::StreamScope scope(s);
    ASSERT(higgs::Stream::task_local_or_default().get() == s.get(), "scope did not set the stream");
    Array y = higgs::fast::rms_norm(dev16(xb, {R, N}, Dtype::Bfloat16), dev16(wb, {N}, Dtype::Bfloat16), 1e-5f);
    other = y.to_bits();
  }
  ASSERT(higgs::Stream::task_local_or_default().get() == nullptr, "scope did not restore the stream");
  ASSERT_BITS_EQ(other, base);
}

// An Array outlives the scope and the Stream object it was allocated under:
// the buffer keeps that stream alive, and its free waits for the other stream
// that read it.
TEST(test_array_outlives_its_stream_and_orders_cross_stream_frees) {
  const int64_t R = 512, N = 4096;
  auto xb = bits_of(normal(9010, R * N), OR_BF16);
  auto wb = bits_of(normal(9011, N, 1.0f, 0.02f), OR_BF16);
  const auto base =
      higgs::fast::rms_norm(dev16(xb, {R, N}, Dtype::Bfloat16), dev16(wb, {N}, Dtype::Bfloat16), 1e-5f)
          .to_bits();
  Array x, w;
  {
    higgs::Stream a = higgs::Stream::create();
    higgs::StreamScope scope(a);
    x = dev16(xb, {R, N}, Dtype::Bfloat16);
    w = dev16(wb, {N}, Dtype::Bfloat16);
  }  // the Stream object `a` is gone; x and w still hold its stream
  higgs::Stream b = higgs::Stream::create();
  std::vector<uint16_t> got;
  {
    higgs::StreamScope scope(b);
    Array y = higgs::fast::rms_norm(x, w, 1e-5f);
    x = Array();  // freed on stream a, ordered after b's read of it
    w = Array();
    for (int i = 0; i < 8; ++i) {  // reuse the pool while b's kernel may still run
      Array t = dev16(xb, {R, N}, Dtype::Bfloat16);
      (void)t;
    }
    got = y.to_bits();
  }
  ASSERT_BITS_EQ(got, base);
}

}  // namespace

int main(int argc, char** argv) {
  if (argc > 1 && std::strcmp(argv[1], "--list") == 0) {
    for (const auto& c : registry()) std::printf("%s\n", c.name);
    return 0;
  }
  int run = 0, failed = 0;
  for (const auto& c : registry()) {
    if (argc > 1) {
      bool want = false;
      for (int i = 1; i < argc; ++i) want |= std::strcmp(argv[i], c.name) == 0;
      if (!want) continue;
    }
    ++run;
    std::printf("%s ... ", c.name);
    std::fflush(stdout);
    try {
      c.fn();
      std::printf("ok\n");
    } catch (const Failure& f) {
      ++failed;
      std::printf("FAILED\n  %s\n", f.msg.c_str());
    } catch (const std::exception& e) {
      ++failed;
      std::printf("FAILED\n  exception: %s\n", e.what());
    }
    std::fflush(stdout);
  }
  std::printf("%d run, %d failed\n", run, failed);
  return failed || run == 0 ? 1 : 0;
}
