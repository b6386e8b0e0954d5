// gdn.hip -- the GatedDeltaNet recurrence of Qwen3-Next on gfx950, with the
// constant-weight q/k RMSNorm in front of it fused in.
//
// Reference: the gated-delta Metal kernel (crates/higgs-models/src/
// qwen3_next.rs:376-451) and its caller (1152-1201): q, k [B, T, Hk, Dk],
// v [B, T, Hv, Dv], a, b [B, T, Hv], a_log, dt_bias [Hv], state
// [B, Hv, Dv, Dk]. Per (b, hv, dv) the state row s (Dk values, f32 while the
// kernel runs, stored in the activation dtype) advances over t:
//   g    = exp(-exp(a_log) * softplus(a_t + dt_bias))
//   beta = sigmoid(b_t)
//   s    = s * g;  kv = s . k_t;  delta = (v_t[dv] - kv) * beta
//   s    = s + k_t * delta;      y_t[dv] = s . q_t
// q and k are first normalised by rms_norm(x, w, 1e-6) with constant weights
// (1/Dk for q, 1/sqrt(Dk) for k, in the activation dtype; 1172-1173) when the
// caller passes those weights.
//
// Work split: as in the reference, 32 lanes own one state row (Dk/32 values
// each), so a wave64 holds two rows and both dot products reduce over 32
// lanes; a block of 256 threads owns 8 rows (dv) of one (b, hv). The loads of
// step t+1 are issued before step t's arithmetic.
#include <cmath>

#include "../../include/higgs_hip.h"
#include "hgk_common.h"
#include "hgk_host.h"

namespace hgk {

struct GdnArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* a_log;
  const void* a;
  const void* dt_bias;
  const void* b;
  const void* state_in;
  const void* qw;  // fused norm weights [Dk] (activation dtype) or null
  const void* kw;
  int pdt;         // dtype of a_log / dt_bias
  float eps;
  float inv_dk;
  int64_t B, T, Hk, Dk, Hv, Dv;
  void* y;
  void* state_out;
};

// Sum over the 32 lanes of a half wave (every lane receives the sum).
__device__ inline float sum32(float v) {
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, 32);
  return v;
}

template <class X, int NPT>
struct GdnStep {
  float q[NPT], k[NPT];
  float v, at, bt;
};

template <class X, int NPT>
__device__ inline void gdn_load(const GdnArgs& a, GdnStep<X, NPT>& s, int64_t bi, int64_t t,
                                int64_t hk, int64_t hv, int64_t dv, int j) {
  const int64_t qk = ((bi * a.T + t) * a.Hk + hk) * a.Dk + (int64_t)j * NPT;
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    s.q[i] = load1<X>(a.q, qk + i);
    s.k[i] = load1<X>(a.k, qk + i);
  }
  s.v = load1<X>(a.v, ((bi * a.T + t) * a.Hv + hv) * a.Dv + dv);
  s.at = load1<X>(a.a, (bi * a.T + t) * a.Hv + hv);
  s.bt = load1<X>(a.b, (bi * a.T + t) * a.Hv + hv);
}

// q or k row normalised as rms_norm(x, w, eps) in dtype X: n = round(x * r),
// out = round(n * w), with the sum of squares taken in f64 over the row.
template <class X, int NPT>
__device__ inline void gdn_norm(float* x, const float* w, float inv_dk, float eps) {
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < NPT; ++i) ss = __builtin_fma((double)x[i], (double)x[i], ss);
  ss = group_sum<32>(ss);
  const float r = rms_scale(ss, inv_dk, eps);
#pragma unroll
  for (int i = 0; i < NPT; ++i) x[i] = X::round(X::round(x[i] * r) * w[i]);
}

template <class X, int NPT, bool NORM>
__global__ __launch_bounds__(256) void gated_delta_kernel(GdnArgs a) {
  const int row = threadIdx.x >> 5, j = threadIdx.x & 31;
  const int64_t bh = blockIdx.y;
  const int64_t bi = bh / a.Hv, hv = bh - bi * a.Hv;
  const int64_t hk = hv / (a.Hv / a.Hk);
  const int64_t dv0 = (int64_t)blockIdx.x * 8 + row;
  const bool live = dv0 < a.Dv;
  const int64_t dv = live ? dv0 : a.Dv - 1;
  const int64_t srow = ((bi * a.Hv + hv) * a.Dv + dv) * a.Dk + (int64_t)j * NPT;

  float st[NPT];
#pragma unroll
  for (int i = 0; i < NPT; ++i) st[i] = a.state_in ? load1<X>(a.state_in, srow + i) : 0.0f;
  float wq[NPT], wk[NPT];
  if constexpr (NORM) {
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      wq[i] = load1<X>(a.qw, (int64_t)j * NPT + i);
      wk[i] = load1<X>(a.kw, (int64_t)j * NPT + i);
    }
  }
  const float A = expf(load1_dt(a.a_log, a.pdt, hv));
  const float dtb = load1_dt(a.dt_bias, a.pdt, hv);

  GdnStep<X, NPT> cur, nxt;
  if (a.T > 0) gdn_load<X, NPT>(a, cur, bi, 0, hk, hv, dv, j);
  for (int64_t t = 0; t < a.T; ++t) {
    if (t + 1 < a.T) gdn_load<X, NPT>(a, nxt, bi, t + 1, hk, hv, dv, j);
    if constexpr (NORM) {
      gdn_norm<X, NPT>(cur.q, wq, a.inv_dk, a.eps);
      gdn_norm<X, NPT>(cur.k, wk, a.inv_dk, a.eps);
    }
    const float x = cur.at + dtb;
    const float sp = fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
    const float g = expf(-A * sp);
    const float beta = 1.0f / (1.0f + expf(-cur.bt));
    float kv = 0.0f;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      st[i] = st[i] * g;
      kv = __builtin_fmaf(st[i], cur.k[i], kv);
    }
    kv = sum32(kv);
    const float delta = (cur.v - kv) * beta;
    float out = 0.0f;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      st[i] = __builtin_fmaf(cur.k[i], delta, st[i]);
      out = __builtin_fmaf(st[i], cur.q[i], out);
    }
    out = sum32(out);
    if (j == 0 && live) store1<X>(a.y, ((bi * a.T + t) * a.Hv + hv) * a.Dv + dv, out);
    cur = nxt;
  }
  if (live) {
#pragma unroll
    for (int i = 0; i < NPT; ++i) store1<X>(a.state_out, srow + i, st[i]);
  }
}

namespace {

template <class X, bool NORM>
bool launch_x(const GdnArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)((a.Dv + 7) / 8), (unsigned)(a.B * a.Hv));
  switch (a.Dk) {
    case 32: hipLaunchKernelGGL((gated_delta_kernel<X, 1, NORM>), grid, dim3(256), 0, s, a); return true;
    case 64: hipLaunchKernelGGL((gated_delta_kernel<X, 2, NORM>), grid, dim3(256), 0, s, a); return true;
    case 128: hipLaunchKernelGGL((gated_delta_kernel<X, 4, NORM>), grid, dim3(256), 0, s, a); return true;
    case 256: hipLaunchKernelGGL((gated_delta_kernel<X, 8, NORM>), grid, dim3(256), 0, s, a); return true;
    default: return false;
  }
}

}  // namespace
}  // namespace hgk

using namespace hgk;

extern "C" int hgk_gated_delta(int dtype, const void* q, const void* k, const void* v,
                               const void* a_log, const void* a, const void* dt_bias, const void* b,
                               int param_dtype, const void* state_in, const void* q_norm_w,
                               const void* k_norm_w, float eps, int64_t batch, int64_t seq_len,
                               int64_t k_heads, int64_t head_k_dim, int64_t v_heads,
                               int64_t head_v_dim, void* y, void* state_out, void* stream) {
  clear_error();
  const char* fn = "hgk_gated_delta";
  if (dtype != DT_BF16 && dtype != DT_F16 && dtype != DT_F32)
    return fail(HGK_ERR_ARG, "%s: dtype must be f32, bf16 or f16", fn);
  if (!is_float_dtype(param_dtype)) return fail(HGK_ERR_ARG, "%s: a_log/dt_bias dtype must be a float type", fn);
  if (batch < 0 || seq_len < 0 || k_heads <= 0 || v_heads <= 0 || head_v_dim <= 0)
    return fail(HGK_ERR_ARG, "%s: bad shape", fn);
  if (v_heads % k_heads)
    return fail(HGK_ERR_ARG, "%s: v_heads=%lld must be a multiple of k_heads=%lld", fn,
                (long long)v_heads, (long long)k_heads);
  if (head_k_dim != 32 && head_k_dim != 64 && head_k_dim != 128 && head_k_dim != 256)
    return fail(HGK_ERR_UNSUPPORTED, "%s: head_k_dim=%lld (32, 64, 128 or 256)", fn, (long long)head_k_dim);
  if ((q_norm_w == nullptr) != (k_norm_w == nullptr))
    return fail(HGK_ERR_ARG, "%s: pass both q and k norm weights or neither", fn);
  if (!(eps >= 0.0f)) return fail(HGK_ERR_ARG, "%s: eps must be >= 0", fn);
  if (!q || !k || !v || !a_log || !a || !dt_bias || !b || !y || !state_out)
    return fail(HGK_ERR_ARG, "%s: null pointer", fn);
  if (batch * v_heads > 65535) return fail(HGK_ERR_UNSUPPORTED, "%s: batch * v_heads > 65535", fn);
  if (batch == 0) return HGK_OK;
  GdnArgs g{};
  g.q = q; g.k = k; g.v = v; g.a_log = a_log; g.a = a; g.dt_bias = dt_bias; g.b = b;
  g.state_in = state_in; g.qw = q_norm_w; g.kw = k_norm_w; g.pdt = param_dtype; g.eps = eps;
  g.inv_dk = (float)(1.0 / (double)head_k_dim);
  g.B = batch; g.T = seq_len; g.Hk = k_heads; g.Dk = head_k_dim; g.Hv = v_heads; g.Dv = head_v_dim;
  g.y = y; g.state_out = state_out;
  const hipStream_t s = as_stream(stream);
  const bool norm = q_norm_w != nullptr;
  bool ok;
  if (dtype == DT_BF16) ok = norm ? launch_x<BF16, true>(g, s) : launch_x<BF16, false>(g, s);
  else if (dtype == DT_F16) ok = norm ? launch_x<F16, true>(g, s) : launch_x<F16, false>(g, s);
  else ok = norm ? launch_x<F32, true>(g, s) : launch_x<F32, false>(g, s);
  if (!ok) return fail(HGK_ERR_UNSUPPORTED, "%s: head_k_dim not supported", fn);
  return launch_status(fn);
}
