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
// Kernels (the step kernels share the per-row arithmetic; their dot products
// are f32 sums whose order differs from the reference's, within the stated
// bars):
//  * token (T = 1, the decode step): no LDS and no barrier. A 16-lane group
//    owns 8 consecutive state rows (Dk/16 columns per lane), so each dot
//    product reduces inside a DPP row. The small loads (gates, q, k, v, norm
//    weights) go first, then the first 4 state rows, so the q/k norm and the
//    gates run while the state is in flight; each row is then waited on
//    alone, advanced, packed and stored, and the row 4 ahead is requested
//    (the state goes through buffer descriptors, so no load or store is
//    under a branch and the waits stay per row).
//  * decode (T = 2): the token kernel's layout (all loads up front, plain
//    global addressing), with the state held in f32 across the steps.
//  * chunk (T > 2): stages 16 steps at a time in LDS -- q and k normalised
//    once per step, g and beta once per step, v for the block's 32 rows -- and
//    every lane carries two state rows whose chains interleave; the next
//    chunk's global loads are issued before the current chunk's recurrence,
//    and y is staged in LDS and stored per step as one run of 32 rows.
//  * row (any alignment): 32 lanes per row, step t+1 loaded during step t.
//  * WY (bf16 prefill with the fused norm, Dk = 128, Dv a multiple of 64,
//    T >= 64): the chunked matrix form on MFMA, below.
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
  int hgrp;        // v heads per k head
  float eps;
  float inv_dk;
  int64_t B, T, Hk, Dk, Hv, Dv;
  void* y;
  void* state_out;
  // gated RMSNorm epilogue (token kernel): out = round(round(z*round(sigmoid z))
  // * rms_norm(y, gw, geps)) over each (b, v-head) row of Dv, z row r at
  // (r / gzg) * gzgs + (r % gzg) * gzs
  const void* gz;
  int64_t gzs, gzg, gzgs;
  const void* gw;
  float geps, inv_dv;
  void* gout;
};

// Sum over the 32 lanes of a half wave (every lane receives the sum).
__device__ inline float sum32(float v) {
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, 32);
  return v;
}

// Raw storage word of element e of X (16-bit types zero-extended), kept
// unconverted so that a load issued ahead of its use is not waited on early.
template <class X>
__device__ inline uint32_t ldraw(const void* base, int64_t e) {
  if constexpr (X::kBytes == 2) return reinterpret_cast<const uint16_t*>(base)[e];
  else return reinterpret_cast<const uint32_t*>(base)[e];
}

template <class X>
__device__ inline float cvt(uint32_t w) {
  if constexpr (X::kBytes == 2) return X::lo(w);
  else return u2f(w);
}

template <class X, int NPT>
struct GdnStep {
  uint32_t q[NPT], k[NPT];
  uint32_t v, at, bt;
};

template <class X, int NPT>
__device__ inline void gdn_load(const GdnArgs& a, GdnStep<X, NPT>& s, int64_t bi, int64_t t,
                                int64_t hk, int64_t hv, int64_t dv, int j) {
  const int64_t qk = ((bi * a.T + t) * a.Hk + hk) * a.Dk + (int64_t)j * NPT;
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    s.q[i] = ldraw<X>(a.q, qk + i);
    s.k[i] = ldraw<X>(a.k, qk + i);
  }
  s.v = ldraw<X>(a.v, ((bi * a.T + t) * a.Hv + hv) * a.Dv + dv);
  s.at = ldraw<X>(a.a, (bi * a.T + t) * a.Hv + hv);
  s.bt = ldraw<X>(a.b, (bi * a.T + t) * a.Hv + hv);
}

// One element of a_log / dt_bias (runtime dtype): the storage word is loaded
// unconverted in each dtype's branch and converted after the join, so the
// load is not waited on inside the branch.
__device__ inline float load_param(const void* base, int dt, int64_t e) {
  uint32_t w;
  if (dt == DT_F32) w = reinterpret_cast<const uint32_t*>(base)[e];
  else w = reinterpret_cast<const uint16_t*>(base)[e];
  if (dt == DT_F32) return u2f(w);
  if (dt == DT_BF16) return u2f(w << 16);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)w);
}

// Sum over the 16 lanes of a DPP row (every lane receives the sum).
template <int CTRL>
__device__ inline float dpp_f(float v) {
  return u2f((uint32_t)__builtin_amdgcn_update_dpp(0, (int)f2u(v), CTRL, 0xF, 0xF, true));
}

__device__ inline float sum16(float v) {
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror
  v += dpp_f<0x140>(v);  // row_mirror
  return v;
}

// softplus, g and beta of one step (qwen3_next.rs:398-402).
__device__ inline float gdn_gate(float at, float dtb, float A) {
  const float x = at + dtb;
  const float sp = fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
  return expf(-A * sp);
}

__device__ inline float gdn_beta(float bt) { return 1.0f / (1.0f + expf(-bt)); }

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
__global__ __launch_bounds__(256) void gated_delta_row_kernel(GdnArgs a) {
  const int row = threadIdx.x >> 5, j = threadIdx.x & 31;
  const int64_t hv = blockIdx.y, bi = blockIdx.z;
  const int64_t hk = (int)blockIdx.y / a.hgrp;
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
  const float A = expf(load_param(a.a_log, a.pdt, hv));
  const float dtb = load_param(a.dt_bias, a.pdt, hv);

  GdnStep<X, NPT> cur, nxt;
  if (a.T > 0) gdn_load<X, NPT>(a, cur, bi, 0, hk, hv, dv, j);
  for (int64_t t = 0; t < a.T; ++t) {
    // step t+1, or step t again on the last step: an unconditional load
    gdn_load<X, NPT>(a, nxt, bi, t + 1 < a.T ? t + 1 : t, hk, hv, dv, j);
    float q[NPT], k[NPT];
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      q[i] = cvt<X>(cur.q[i]);
      k[i] = cvt<X>(cur.k[i]);
    }
    if constexpr (NORM) {
      gdn_norm<X, NPT>(q, wq, a.inv_dk, a.eps);
      gdn_norm<X, NPT>(k, wk, a.inv_dk, a.eps);
    }
    const float g = gdn_gate(cvt<X>(cur.at), dtb, A);
    const float beta = gdn_beta(cvt<X>(cur.bt));
    float kv = 0.0f;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      st[i] = st[i] * g;
      kv = __builtin_fmaf(st[i], k[i], kv);
    }
    kv = sum32(kv);
    const float delta = (cvt<X>(cur.v) - kv) * beta;
    float out = 0.0f;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      st[i] = __builtin_fmaf(k[i], delta, st[i]);
      out = __builtin_fmaf(st[i], q[i], out);
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

// ---------------------------------------------------------------- chunked
// N contiguous elements of X at element e, N * sizeof(X) in {4 .. 64} bytes
// and aligned to min(16, N * sizeof(X)).
template <class X, int N>
__device__ inline void load_row_part(const void* base, int64_t e, float* v) {
  constexpr int BYTES = N * X::kBytes;
  const char* p = reinterpret_cast<const char*>(base) + e * X::kBytes;
  if constexpr (BYTES == 4) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
    if constexpr (X::kBytes == 2) { v[0] = X::lo(w); v[1] = X::hi(w); }
    else v[0] = u2f(w);
  } else if constexpr (BYTES == 8) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 w = *reinterpret_cast<const u32x2*>(p);
    if constexpr (X::kBytes == 2) { v[0] = X::lo(w[0]); v[1] = X::hi(w[0]); v[2] = X::lo(w[1]); v[3] = X::hi(w[1]); }
    else { v[0] = u2f(w[0]); v[1] = u2f(w[1]); }
  } else {
    static_assert(BYTES % 16 == 0, "whole chunks");
    load_elems<X, N>(base, e, v);
  }
}

template <class X, int N>
__device__ inline void store_row_part(void* base, int64_t e, const float* v) {
  constexpr int BYTES = N * X::kBytes;
  char* p = reinterpret_cast<char*>(base) + e * X::kBytes;
  if constexpr (BYTES == 4) {
    if constexpr (X::kBytes == 2) *reinterpret_cast<uint32_t*>(p) = X::pack(v[0], v[1]);
    else *reinterpret_cast<float*>(p) = v[0];
  } else if constexpr (BYTES == 8) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    u32x2 w;
    if constexpr (X::kBytes == 2) { w[0] = X::pack(v[0], v[1]); w[1] = X::pack(v[2], v[3]); }
    else { w[0] = f2u(v[0]); w[1] = f2u(v[1]); }
    *reinterpret_cast<u32x2*>(p) = w;
  } else {
    store_elems<X, N, false>(base, e, v);
  }
}

constexpr int kChunk = 16;  // steps staged per chunk
constexpr int kRows = 32;   // state rows per block (4 waves x 4 DPP rows x 2)

// Per-thread registers of one chunk's global loads, kept raw until publish.
// q/k: thread owns part (tid & 7) of row (tid >> 3) = step (tid >> 4), q or k
// by bit 3; v: step (tid >> 4), rows 2 * (tid & 15) + {0, 1}; a or b: the
// first 2 * kChunk threads, one step each.
template <class X, int DK>
struct GdnChunkRaw {
  static constexpr int NE = DK / 8;                 // q/k elements per thread
  static constexpr int NW = NE * X::kBytes / 4;     // as 32-bit words
  uint32_t qk[NW];
  uint32_t v0, v1, ab;
};

template <class X, int DK>
__device__ inline void gdn_fetch(const GdnArgs& a, GdnChunkRaw<X, DK>& r, int64_t bi, int64_t hk,
                                 int64_t hv, int64_t dv0, int64_t t0, int tid) {
  using R = GdnChunkRaw<X, DK>;
  const int64_t last = a.T - 1;
  {
    const int s = tid >> 4, isk = (tid >> 3) & 1, part = tid & 7;
    const int64_t t = t0 + s < last ? t0 + s : last;
    const void* src = isk ? (const void*)a.k : (const void*)a.q;
    const char* p = reinterpret_cast<const char*>(src) +
                    ((((bi * a.T + t) * a.Hk + hk) * DK) + part * R::NE) * X::kBytes;
    if constexpr (R::NW % 4 == 0) {
#pragma unroll
      for (int c = 0; c < R::NW / 4; ++c) {
        const u32x4 w = reinterpret_cast<const u32x4*>(p)[c];
#pragma unroll
        for (int i = 0; i < 4; ++i) r.qk[4 * c + i] = w[i];
      }
    } else {
      typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
      static_assert(R::NW == 2, "8-byte part");
      const u32x2 w = *reinterpret_cast<const u32x2*>(p);
      r.qk[0] = w[0];
      r.qk[1] = w[1];
    }
  }
  {
    const int s = tid >> 4, pr = tid & 15;
    const int64_t t = t0 + s < last ? t0 + s : last;
    const int64_t d0 = dv0 + 2 * pr < a.Dv ? dv0 + 2 * pr : a.Dv - 1;
    const int64_t d1 = dv0 + 2 * pr + 1 < a.Dv ? dv0 + 2 * pr + 1 : a.Dv - 1;
    const int64_t base = ((bi * a.T + t) * a.Hv + hv) * a.Dv;
    r.v0 = ldraw<X>(a.v, base + d0);
    r.v1 = ldraw<X>(a.v, base + d1);
  }
  {
    const int s = tid & (kChunk - 1);
    const int64_t t = t0 + s < last ? t0 + s : last;
    r.ab = ldraw<X>(tid < kChunk ? (const void*)a.a : (const void*)a.b, (bi * a.T + t) * a.Hv + hv);
  }
}

template <class X, int NPT, bool NORM>
__global__ __launch_bounds__(256) void gated_delta_chunk_kernel(GdnArgs a) {
  constexpr int DK = 16 * NPT;
  using Raw = GdnChunkRaw<X, DK>;
  constexpr int NE = Raw::NE;
  __shared__ __align__(16) float qs[kChunk][DK];
  __shared__ __align__(16) float ks[kChunk][DK];
  __shared__ __align__(16) float vs[kChunk][kRows];
  __shared__ __align__(16) float ys[kChunk][kRows];
  __shared__ __align__(16) float gb[kChunk][2];

  const int tid = threadIdx.x;
  const int64_t hv = blockIdx.y, bi = blockIdx.z;
  const int64_t hk = (int)blockIdx.y / a.hgrp;
  const int64_t dv0 = (int64_t)blockIdx.x * kRows;

  // this lane's two state rows: local rows rl, rl + 1; columns j * NPT ..
  const int lane = tid & 63, j = lane & 15;
  const int rl = (tid >> 6) * 8 + (lane >> 4) * 2;
  float st[2][NPT];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int64_t dv = dv0 + rl + r < a.Dv ? dv0 + rl + r : a.Dv - 1;
    const int64_t e = ((bi * a.Hv + hv) * a.Dv + dv) * DK + (int64_t)j * NPT;
    if (a.state_in) load_row_part<X, NPT>(a.state_in, e, st[r]);
    else {
#pragma unroll
      for (int i = 0; i < NPT; ++i) st[r][i] = 0.0f;
    }
  }

  Raw raw;
  if (a.T > 0) gdn_fetch<X, DK>(a, raw, bi, hk, hv, dv0, 0, tid);

  // publish-side constants: this thread's norm weights (q or k, fixed by tid)
  const int ns = tid >> 4, nisk = (tid >> 3) & 1, npart = tid & 7;
  float wn[NE];
  if constexpr (NORM) {
#pragma unroll
    for (int i = 0; i < NE; ++i) wn[i] = load1<X>(nisk ? a.kw : a.qw, npart * NE + i);
  }
  const float A = expf(load_param(a.a_log, a.pdt, hv));
  const float dtb = load_param(a.dt_bias, a.pdt, hv);
  const bool dv_even = (a.Dv & 1) == 0;

  // y of the chunk at t0 (n steps) from ys to global, one run of rows per step
  auto store_y = [&](int64_t t0, int n) {
    const int s = tid >> 4, pr = tid & 15;
    const int64_t d0 = dv0 + 2 * pr;
    if (s < n && d0 < a.Dv) {
      const int64_t e = ((bi * a.T + t0 + s) * a.Hv + hv) * a.Dv + d0;
      const float y0 = ys[s][2 * pr], y1 = ys[s][2 * pr + 1];
      if constexpr (X::kBytes == 2) {
        if (dv_even) {
          reinterpret_cast<uint32_t*>(a.y)[e >> 1] = X::pack(y0, y1);
        } else {
          store1<X>(a.y, e, y0);
          if (d0 + 1 < a.Dv) store1<X>(a.y, e + 1, y1);
        }
      } else {
        if (dv_even) {
          reinterpret_cast<f32x2*>(a.y)[e >> 1] = f32x2{y0, y1};
        } else {
          store1<X>(a.y, e, y0);
          if (d0 + 1 < a.Dv) store1<X>(a.y, e + 1, y1);
        }
      }
    }
  };

  for (int64_t t0 = 0; t0 < a.T; t0 += kChunk) {
    const int n = a.T - t0 < kChunk ? (int)(a.T - t0) : kChunk;
    __syncthreads();  // the previous chunk's readers of qs/ks/vs/gb and writers of ys are done
    if (t0 > 0) store_y(t0 - kChunk, kChunk);
    {
      float x[NE];
#pragma unroll
      for (int i = 0; i < NE; ++i) x[i] = elem<X>(raw.qk, i);
      if constexpr (NORM) {
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < NE; ++i) ss = __builtin_fma((double)x[i], (double)x[i], ss);
        ss = group_sum<8>(ss);
        const float r = rms_scale(ss, a.inv_dk, a.eps);
#pragma unroll
        for (int i = 0; i < NE; ++i) x[i] = X::round(X::round(x[i] * r) * wn[i]);
      }
      float* dst = (nisk ? &ks[ns][0] : &qs[ns][0]) + npart * NE;
#pragma unroll
      for (int i = 0; i < NE; i += 4)
        *reinterpret_cast<float4*>(dst + i) = make_float4(x[i], x[i + 1], x[i + 2], x[i + 3]);
      const int pr = tid & 15;
      *reinterpret_cast<f32x2*>(&vs[ns][2 * pr]) = f32x2{cvt<X>(raw.v0), cvt<X>(raw.v1)};
      if (tid < 2 * kChunk) {
        const float ab = cvt<X>(raw.ab);
        gb[tid & (kChunk - 1)][tid >> 4] = tid < kChunk ? gdn_gate(ab, dtb, A) : gdn_beta(ab);
      }
    }
    __syncthreads();
    if (t0 + kChunk < a.T) gdn_fetch<X, DK>(a, raw, bi, hk, hv, dv0, t0 + kChunk, tid);

    // LDS reads of the next step are issued before a step's arithmetic, into
    // the other of two register sets (steps alternate between them)
    float qa[NPT], ka[NPT], qb[NPT], kb[NPT];
    f32x2 va, ga, vb, gbb;
    auto rd = [&](float* q, float* k, f32x2& v, f32x2& g, int s) {
#pragma unroll
      for (int i = 0; i < NPT; i += 2) {
        const f32x2 qq = *reinterpret_cast<const f32x2*>(&qs[s][j * NPT + i]);
        const f32x2 kk = *reinterpret_cast<const f32x2*>(&ks[s][j * NPT + i]);
        q[i] = qq[0]; q[i + 1] = qq[1];
        k[i] = kk[0]; k[i + 1] = kk[1];
      }
      v = *reinterpret_cast<const f32x2*>(&vs[s][rl]);
      g = *reinterpret_cast<const f32x2*>(&gb[s][0]);
    };
    auto step = [&](const float* q, const float* k, f32x2 vv, f32x2 g2, int s) {
      const float g = g2[0], beta = g2[1];
      float out[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        float kv = 0.0f;
#pragma unroll
        for (int i = 0; i < NPT; ++i) {
          st[r][i] = st[r][i] * g;
          kv = __builtin_fmaf(st[r][i], k[i], kv);
        }
        kv = sum16(kv);
        const float delta = (vv[r] - kv) * beta;
        float o = 0.0f;
#pragma unroll
        for (int i = 0; i < NPT; ++i) {
          st[r][i] = __builtin_fmaf(k[i], delta, st[r][i]);
          o = __builtin_fmaf(st[r][i], q[i], o);
        }
        out[r] = sum16(o);
      }
      if (j == 0) *reinterpret_cast<f32x2*>(&ys[s][rl]) = f32x2{out[0], out[1]};
    };
    rd(qa, ka, va, ga, 0);
    for (int s = 0; s < n; s += 2) {
      rd(qb, kb, vb, gbb, s + 1 < n ? s + 1 : s);
      step(qa, ka, va, ga, s);
      if (s + 1 < n) {
        rd(qa, ka, va, ga, s + 2 < n ? s + 2 : s + 1);
        step(qb, kb, vb, gbb, s + 1);
      }
    }
  }
  if (a.T > 0) {
    __syncthreads();
    const int64_t tl = ((a.T - 1) / kChunk) * kChunk;
    store_y(tl, (int)(a.T - tl));
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    if (dv0 + rl + r < a.Dv) {
      const int64_t e = ((bi * a.Hv + hv) * a.Dv + dv0 + rl + r) * DK + (int64_t)j * NPT;
      store_row_part<X, NPT>(a.state_out, e, st[r]);
    }
  }
}

// State rows per lane and rows in flight per lane group of the token kernel.
// At 64 sequences x 32 value heads of 128 x 128 (two probe calls each): 4
// rows per lane 24.80-24.91 us and 16 rows 26.49-26.56 against 24.59-24.78
// with 8; 3 and 6 rows in flight 25.11-25.12 and 25.26-25.27 against
// 24.49-24.62 with 4 (8, all of them: 3-4 % slower).
#ifndef HGK_GDN_RPL
#define HGK_GDN_RPL 8
#endif
#ifndef HGK_GDN_WIN
#define HGK_GDN_WIN 4
#endif
#ifndef HGK_GDN_WPB
#define HGK_GDN_WPB 4
#endif
// ---------------------------------------------------------------- decode
// Few steps (decode): no LDS and no barrier. Each 16-lane group owns RPL
// consecutive state rows (Dk/16 columns per lane), normalises the step's q
// and k itself and computes g and beta itself; the state rows' vector loads
// are issued first, so a wave keeps RPL * 16 * Dk * sizeof(X) bytes in
// flight from its first instructions.
template <class X, int NPT, bool NORM, int RPL>
__global__ __launch_bounds__(256) void gated_delta_decode_kernel(GdnArgs a) {
  constexpr int DK = 16 * NPT;
  const int tid = threadIdx.x, lane = tid & 63, j = lane & 15;
  const int64_t hv = blockIdx.y, bi = blockIdx.z;
  const int64_t hk = (int)blockIdx.y / a.hgrp;
  const int64_t r0 = (int64_t)blockIdx.x * (16 * RPL) + ((tid >> 6) * 4 + (lane >> 4)) * RPL;

  float st[RPL][NPT];
#pragma unroll
  for (int r = 0; r < RPL; ++r) {
    const int64_t dv = r0 + r < a.Dv ? r0 + r : a.Dv - 1;
    const int64_t e = ((bi * a.Hv + hv) * a.Dv + dv) * DK + (int64_t)j * NPT;
    if (a.state_in) load_row_part<X, NPT>(a.state_in, e, st[r]);
    else {
#pragma unroll
      for (int i = 0; i < NPT; ++i) st[r][i] = 0.0f;
    }
  }
  float wq[NPT], wk[NPT];
  if constexpr (NORM) {
    load_row_part<X, NPT>(a.qw, (int64_t)j * NPT, wq);
    load_row_part<X, NPT>(a.kw, (int64_t)j * NPT, wk);
  }
  const float A = expf(load_param(a.a_log, a.pdt, hv));
  const float dtb = load_param(a.dt_bias, a.pdt, hv);

  for (int64_t t = 0; t < a.T; ++t) {
    const int64_t row = (bi * a.T + t) * a.Hv + hv;
    float q[NPT], k[NPT], v[RPL];
    load_row_part<X, NPT>(a.q, ((bi * a.T + t) * a.Hk + hk) * DK + (int64_t)j * NPT, q);
    load_row_part<X, NPT>(a.k, ((bi * a.T + t) * a.Hk + hk) * DK + (int64_t)j * NPT, k);
#pragma unroll
    for (int r = 0; r < RPL; ++r) v[r] = load1<X>(a.v, row * a.Dv + (r0 + r < a.Dv ? r0 + r : a.Dv - 1));
    const float g = gdn_gate(load1<X>(a.a, row), dtb, A);
    const float beta = gdn_beta(load1<X>(a.b, row));
    if constexpr (NORM) {
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        float* x = w ? k : q;
        const float* wt = w ? wk : wq;
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < NPT; ++i) ss = __builtin_fma((double)x[i], (double)x[i], ss);
        ss = group_sum<16>(ss);
        const float rs = rms_scale(ss, a.inv_dk, a.eps);
#pragma unroll
        for (int i = 0; i < NPT; ++i) x[i] = X::round(X::round(x[i] * rs) * wt[i]);
      }
    }
    float out[RPL];
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
      float kv = 0.0f;
#pragma unroll
      for (int i = 0; i < NPT; ++i) {
        st[r][i] = st[r][i] * g;
        kv = __builtin_fmaf(st[r][i], k[i], kv);
      }
      kv = sum16(kv);
      const float delta = (v[r] - kv) * beta;
      float o = 0.0f;
#pragma unroll
      for (int i = 0; i < NPT; ++i) {
        st[r][i] = __builtin_fmaf(k[i], delta, st[r][i]);
        o = __builtin_fmaf(st[r][i], q[i], o);
      }
      out[r] = sum16(o);
    }
    if (j == 0) {
#pragma unroll
      for (int r = 0; r < RPL; ++r)
        if (r0 + r < a.Dv) store1<X>(a.y, row * a.Dv + r0 + r, out[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < RPL; ++r) {
    if (r0 + r < a.Dv) {
      const int64_t e = ((bi * a.Hv + hv) * a.Dv + r0 + r) * DK + (int64_t)j * NPT;
      store_row_part<X, NPT>(a.state_out, e, st[r]);
    }
  }
}

// One token (T = 1): as the decode kernel, but the state rows stay packed in
// their storage words until their turn, and each row is converted, advanced,
// packed and stored on its own, so only one row is live in f32 at a time
// (fewer VGPRs, more waves per SIMD to overlap the loads).
template <class X, int NPT>
__device__ inline void load_row_raw(const void* base, int64_t e, uint32_t* w) {
  constexpr int NW = NPT * X::kBytes / 4;
  const char* p = reinterpret_cast<const char*>(base) + e * X::kBytes;
  if constexpr (NW == 1) {
    w[0] = *reinterpret_cast<const uint32_t*>(p);
  } else if constexpr (NW == 2) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 v = *reinterpret_cast<const u32x2*>(p);
    w[0] = v[0]; w[1] = v[1];
  } else {
#pragma unroll
    for (int c = 0; c < NW / 4; ++c) {
      const u32x4 v = reinterpret_cast<const u32x4*>(p)[c];
#pragma unroll
      for (int i = 0; i < 4; ++i) w[4 * c + i] = v[i];
    }
  }
}

// NW 32-bit words at byte offset `off` of a buffer: offsets at or past the
// buffer's size read zeros (a zero-size buffer reads zeros everywhere) and
// drop stores, so the state rows need no branch around their loads or stores.
// The state is read once and written once per call: both go with the
// non-temporal cache policy (bit 1 of the buffer instructions' policy operand).
typedef uint32_t gd_u32x2 __attribute__((ext_vector_type(2)));
constexpr int kNt = 2;

template <int NW>
__device__ inline void buf_load_words(__amdgpu_buffer_rsrc_t rs, uint32_t off, uint32_t (&w)[NW]) {
  if constexpr (NW == 1) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, kNt);
  } else if constexpr (NW == 2) {
    const gd_u32x2 v = __builtin_bit_cast(gd_u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, kNt));
    w[0] = v[0];
    w[1] = v[1];
  } else {
    static_assert(NW % 4 == 0, "whole 16-byte pieces");
#pragma unroll
    for (int c = 0; c < NW / 4; ++c) {
      const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 * c, 0, kNt));
#pragma unroll
      for (int i = 0; i < 4; ++i) w[4 * c + i] = v[i];
    }
  }
}

template <int NW>
__device__ inline void buf_store_words(__amdgpu_buffer_rsrc_t rs, uint32_t off, const uint32_t (&w)[NW]) {
  if constexpr (NW == 1) {
    __builtin_amdgcn_raw_buffer_store_b32(w[0], rs, off, 0, kNt);
  } else if constexpr (NW == 2) {
    __builtin_amdgcn_raw_buffer_store_b64(gd_u32x2{w[0], w[1]}, rs, off, 0, kNt);
  } else {
#pragma unroll
    for (int c = 0; c < NW / 4; ++c)
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{w[4 * c], w[4 * c + 1], w[4 * c + 2], w[4 * c + 3]},
                                             rs, off + 16 * c, 0, kNt);
  }
}

template <class X, class P, int NPT, bool NORM, int RPL, bool GN = false>
__global__ __launch_bounds__(256) void gated_delta_token_kernel(GdnArgs a) {
  constexpr int DK = 16 * NPT;
  constexpr int NW = NPT * X::kBytes / 4;
  const int tid = threadIdx.x, lane = tid & 63, j = lane & 15;
  const int64_t hv = blockIdx.y, bi = blockIdx.z;
  const int64_t hk = (int)blockIdx.y / a.hgrp;
  const int64_t r0 = (int64_t)blockIdx.x * (blockDim.x / 16 * RPL) + ((tid >> 6) * 4 + (lane >> 4)) * RPL;
  const int64_t sbase = (bi * a.Hv + hv) * a.Dv;
  const int64_t row = bi * a.Hv + hv;  // T == 1

  // Issue order: the small loads first, then the state rows, so that the
  // norm and the gates wait only for the former while the state is in flight.
  uint32_t araw, braw, vraw[RPL];
  uint32_t qraw[NW], kraw[NW], wqraw[NW], wkraw[NW];
  const uint32_t alog_raw = ldraw<P>(a.a_log, hv);
  const uint32_t dtb_raw = ldraw<P>(a.dt_bias, hv);
  araw = ldraw<X>(a.a, row);
  braw = ldraw<X>(a.b, row);
  load_row_raw<X, NPT>(a.q, (bi * a.Hk + hk) * DK + (int64_t)j * NPT, qraw);
  load_row_raw<X, NPT>(a.k, (bi * a.Hk + hk) * DK + (int64_t)j * NPT, kraw);
  if constexpr (NORM) {
    load_row_raw<X, NPT>(a.qw, (int64_t)j * NPT, wqraw);
    load_row_raw<X, NPT>(a.kw, (int64_t)j * NPT, wkraw);
  }
#pragma unroll
  for (int r = 0; r < RPL; ++r) vraw[r] = ldraw<X>(a.v, row * a.Dv + (r0 + r < a.Dv ? r0 + r : a.Dv - 1));
  // gated-norm epilogue: this group's RPL rows of z and of the norm weight
  // (contiguous in dv; the launcher checks their 16-byte alignment)
  constexpr int GW = GN ? RPL * X::kBytes / 4 : 1;
  uint32_t zraw[GW], gwraw[GW];
  if constexpr (GN) {
    const int64_t rc = r0 < a.Dv ? r0 : 0;
    const int64_t zrow = (row / a.gzg) * a.gzgs + (row % a.gzg) * a.gzs;
    load_row_raw<X, RPL>(a.gz, zrow + rc, zraw);
    load_row_raw<X, RPL>(a.gw, rc, gwraw);
  }
  // the state rows through buffer descriptors (the launcher keeps the state
  // under 2^31 bytes): no state reads zeros, rows past Dv read zeros and
  // their stores are dropped, so no load or store sits under a branch and
  // each row is waited on alone, its store issued while later rows load
  const int64_t sbytes = a.B * a.Hv * a.Dv * DK * X::kBytes;
  const __amdgpu_buffer_rsrc_t sin = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(a.state_in), (short)0, a.state_in ? (int)sbytes : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t sout = __builtin_amdgcn_make_buffer_rsrc(a.state_out, (short)0, (int)sbytes, 0x00020000);
  uint32_t soff[RPL];
#pragma unroll
  for (int r = 0; r < RPL; ++r)
    soff[r] = r0 + r < a.Dv ? (uint32_t)(((sbase + r0 + r) * DK + (int64_t)j * NPT) * X::kBytes) : 0x80000000u;
  uint32_t raw[RPL][NW];
#pragma unroll
  for (int r = 0; r < RPL; ++r)
    if (r < HGK_GDN_WIN) buf_load_words<NW>(sin, soff[r], raw[r]);
  __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the first wait below

  const float g = gdn_gate(cvt<X>(araw), cvt<P>(dtb_raw), expf(cvt<P>(alog_raw)));
  const float beta = gdn_beta(cvt<X>(braw));
  float q[NPT], k[NPT];
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    q[i] = elem<X>(qraw, i);
    k[i] = elem<X>(kraw, i);
  }
  if constexpr (NORM) {
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      float* x = w ? k : q;
      const uint32_t* wr = w ? wkraw : wqraw;
      double ss = 0.0;
#pragma unroll
      for (int i = 0; i < NPT; ++i) ss = __builtin_fma((double)x[i], (double)x[i], ss);
      ss = group_sum<16>(ss);
      const float rs = rms_scale(ss, a.inv_dk, a.eps);
#pragma unroll
      for (int i = 0; i < NPT; ++i) x[i] = X::round(X::round(x[i] * rs) * elem<X>(wr, i));
    }
  }
  float out[RPL];
#pragma unroll
  for (int r = 0; r < RPL; ++r) {
    float st[NPT];
#pragma unroll
    for (int i = 0; i < NPT; ++i) st[i] = elem<X>(raw[r], i);
    float kv = 0.0f;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      st[i] = st[i] * g;
      kv = __builtin_fmaf(st[i], k[i], kv);
    }
    kv = sum16(kv);
    const float delta = (cvt<X>(vraw[r]) - kv) * beta;
    float o = 0.0f;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      st[i] = __builtin_fmaf(k[i], delta, st[i]);
      o = __builtin_fmaf(st[i], q[i], o);
    }
    out[r] = sum16(o);
    uint32_t w[NW];
    if constexpr (X::kBytes == 2) {
#pragma unroll
      for (int i = 0; i < NW; ++i) w[i] = X::pack(st[2 * i], st[2 * i + 1]);
    } else {
#pragma unroll
      for (int i = 0; i < NW; ++i) w[i] = f2u(st[i]);
    }
    buf_store_words<NW>(sout, soff[r], w);
    if (r + HGK_GDN_WIN < RPL) buf_load_words<NW>(sin, soff[r + HGK_GDN_WIN], raw[r + HGK_GDN_WIN]);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (j == 0 && (!GN || a.y != nullptr)) {
#pragma unroll
    for (int r = 0; r < RPL; ++r)
      if (r0 + r < a.Dv) store1<X>(a.y, row * a.Dv + r0 + r, out[r]);
  }
  if constexpr (GN) {
    // the block holds the whole (b, v-head) row of Dv outputs (one row tile):
    // each lane group sums its rows' squares (y rounded to X, as the norm
    // reads it) in f64, and every thread adds the groups' sums in one order
    constexpr int G = 256 / 16;
    __shared__ double part[G];
    const int grp = tid >> 4;
    float yr[RPL];
    double ss = 0.0;
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
      yr[r] = r0 + r < a.Dv ? X::round(out[r]) : 0.0f;
      ss = __builtin_fma((double)yr[r], (double)yr[r], ss);
    }
    if (j == 0) part[grp] = ss;
    __syncthreads();
    double tot = 0.0;
#pragma unroll
    for (int q = 0; q < G; ++q) tot += part[q];
    const float rs = rms_scale(tot, a.inv_dv, a.geps);
    // lane j < RPL of the group finishes row r0 + j (every lane holds the
    // group's y, z and weights)
    if (j < RPL && r0 + j < a.Dv) {
      float yj = yr[0], zj = elem<X>(zraw, 0), wj = elem<X>(gwraw, 0);
#pragma unroll
      for (int r = 1; r < RPL; ++r) {
        if (j == r) {
          yj = yr[r];
          zj = elem<X>(zraw, r);
          wj = elem<X>(gwraw, r);
        }
      }
      const float nv = X::round(X::round(yj * rs) * wj);
      const float sg = X::round(mlx_sigmoid(zj));
      const float act = X::round(zj * sg);
      store1<X>(a.gout, row * a.Dv + r0 + j, act * nv);
    }
  }
}

// ---------------------------------------------------------------- WY chunks
// bf16 prefill with the fused q/k norm at Dk = 128: the chunked (WY) form of
// the same recurrence, on the matrix cores. Per chunk of C = 64 steps with
// lam_t = sum_{u <= t} log g_u (log g = -exp(a_log) * softplus(a + dt_bias),
// the exponent of the reference's g) and the block's 64 state rows S (f32):
//   L = strictly_lower(beta_i e^{lam_i - lam_j} k_i.k_j)
//   R = beta * (V - e^lam * (K S^T))
//   Delta = (I + L)^{-1} R
//   Y = e^lam * (Q S^T) + lower(e^{lam_i - lam_j} q_i.k_j) Delta
//   S <- e^{lam_C} S + (e^{lam_C - lam} * Delta)^T K
// which unrolls the per-step update s = s*g; d = (v - s.k)*beta; s += k*d;
// y = s.q exactly (in exact arithmetic). Step by step this is the
// reference's recurrence; only the rounding differs, as for the other kernels.
// Products: k.k and q.k on v_mfma_f32_16x16x32_bf16 (the normalised q and k
// are bf16, so every product is exact in the f32 accumulator); K S^T, Q S^T
// and the state update on the same instruction with the f32 operand split
// into bf16 hi + lo (relative error ~2^-17); the triangular solve and M Delta
// on v_mfma_f32_16x16x4_f32 (f32 throughout): 16 x 16 diagonal blocks of
// (I + L) inverted by forward substitution, the rest by blocked substitution.
// A block owns (b, v-head, 64 state rows), 8 waves, the state in LDS for the
// whole sequence; the next chunk's q, k, v, a, b are loaded during the current
// chunk's products, and its q/k rows are normalised (and its gates computed)
// while waves 0..3 run the triangular solve. Steps past T in the last chunk
// are zero rows (k = q = v = beta = 0, log g = 0), which leave S unchanged.
typedef __bf16 wy_bf8 __attribute__((ext_vector_type(8)));
typedef float wy_f4 __attribute__((ext_vector_type(4)));

constexpr int kWyC = 64;             // steps per chunk
constexpr int kWyDK = 128;           // head_k_dim
constexpr int kWyRows = 64;          // state rows per block
constexpr int kWySP = kWyDK + 4;     // f32 pitch of the state rows
constexpr int kWyKP = kWyDK + 8;     // bf16 pitch of k / q rows
constexpr int kWyTP = kWyC + 8;      // bf16 pitch of k^T rows and of the v / y staging rows
constexpr int kWyLP = kWyC + 4;      // f32 pitch of L, M and R^T / Delta^T rows
constexpr int64_t kWyMinSteps = 64;  // shorter sequences take the chunk kernel

struct WyLds {
  float S[kWyRows][kWySP];
  uint16_t Kh[kWyC][kWyKP];
  uint16_t Qh[kWyC][kWyKP];
  uint16_t KT[kWyDK][kWyTP];
  float L[kWyC][kWyLP];     // after the solve: the y staging rows (bf16, pitch kWyTP)
  float M[kWyC][kWyLP];
  float RD[kWyRows][kWyLP];  // R^T, overwritten block by block with Delta^T ([row][step])
  float Td[4][16][20];       // inverses of the 16 x 16 diagonal blocks of I + L
  uint16_t V[kWyC][kWyTP];
  float lam2[kWyC], beta[kWyC], eL[kWyC], eC[kWyC];  // lam2 = lam * log2(e)
  uint16_t wk[kWyDK], wq[kWyDK];                       // the norm weights
};

// Raw global loads of one chunk. Thread u of a wave group of four holds 32
// elements (part u & 3) of row u >> 2: q rows in waves 0..3 (u = tid), k rows
// in waves 4..7 (u = tid - 256), which also hold 16 elements (part u & 3) of
// v row u >> 2; wave 4 holds step (lane)'s a and b.
struct WyRaw {
  u32x4 x[4];
  u32x4 v[2];
  uint32_t a, b;
};

__device__ inline void wy_fetch(const GdnArgs& g, WyRaw& r, int64_t bi, int64_t hk, int64_t hv,
                                int64_t dv0, int64_t t0, int u, bool kwave, bool wave4) {
  const int64_t last = g.T - 1;
  const int row = u >> 2, part = u & 3;
  const int64_t t = t0 + row < last ? t0 + row : last;
  const u32x4* px = reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(kwave ? g.k : g.q) +
                                                   ((bi * g.T + t) * g.Hk + hk) * kWyDK + 32 * part);
#pragma unroll
  for (int c = 0; c < 4; ++c) r.x[c] = px[c];
  if (kwave) {
    const u32x4* pv = reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(g.v) +
                                                     ((bi * g.T + t) * g.Hv + hv) * g.Dv + dv0 + 16 * part);
    r.v[0] = pv[0];
    r.v[1] = pv[1];
  }
  if (wave4) {
    const int lane = u & 63;
    const int64_t ts = t0 + lane < last ? t0 + lane : last;
    r.a = ldraw<BF16>(g.a, (bi * g.T + ts) * g.Hv + hv);
    r.b = ldraw<BF16>(g.b, (bi * g.T + ts) * g.Hv + hv);
  }
}

// The gates of one chunk on one wave, lane = step: lam2 = lam * log2(e) with
// lam the inclusive prefix sum of log g = -A * softplus(a + dt_bias) over the
// chunk, beta = sigmoid(b), e^lam and e^{lam_C - lam}; steps at or past n
// have log g = 0 and beta = 0.
struct WyGates {
  float lam2, beta, eL, eC;
};

__device__ inline WyGates wy_gates(const WyRaw& r, float A, float dtb, int lane, int n) {
  const bool lv = lane < n;
  const float x = BF16::lo(r.a) + dtb;
  const float sp = fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
  float lam = lv ? -A * sp : 0.0f;
  WyGates o;
  o.beta = lv ? 1.0f / (1.0f + expf(-BF16::lo(r.b))) : 0.0f;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const float t = __shfl_up(lam, d, 64);
    if (lane >= d) lam += t;
  }
  const float lamC = __shfl(lam, 63, 64);
  o.lam2 = lam * 1.4426950408889634f;
  o.eL = expf(lam);
  o.eC = expf(lamC - lam);
  return o;
}

// 32 elements (part u & 3) of one q or k row normalised as rms_norm(x, w, eps)
// in bf16 (n = round(x * r), out = round(n * w), sum of squares in f64 over
// the row's four lanes), packed; rows past the chunk's live steps are zero.
__device__ inline void wy_norm(const u32x4 (&raw)[4], const uint16_t* w, float inv_dk, float eps,
                               bool live, u32x4 (&out)[4]) {
  float x[32];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) x[8 * c + e] = elem<BF16>(raw[c], e);
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < 32; ++i) ss = __builtin_fma((double)x[i], (double)x[i], ss);
  ss = group_sum<4>(ss);
  const float rs = rms_scale(ss, inv_dk, eps);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const u32x4 wr = *reinterpret_cast<const u32x4*>(w + 8 * c);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      float a0 = x[8 * c + 2 * p] * rs, a1 = x[8 * c + 2 * p + 1] * rs;
      round2<BF16>(a0, a1);
      a0 = a0 * BF16::lo(wr[p]);
      a1 = a1 * BF16::hi(wr[p]);
      out[c][p] = live ? BF16::pack(a0, a1) : 0u;
    }
  }
}

// Eight f32 values as bf16 hi and lo parts (x = hi + lo + O(2^-17 |x|)).
__device__ inline void wy_split(const float* x, wy_bf8& hi, wy_bf8& lo) {
  u32x4 h, l;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    h[p] = BF16::pack(x[2 * p], x[2 * p + 1]);
    l[p] = BF16::pack(x[2 * p] - BF16::lo(h[p]), x[2 * p + 1] - BF16::hi(h[p]));
  }
  hi = __builtin_bit_cast(wy_bf8, h);
  lo = __builtin_bit_cast(wy_bf8, l);
}

__device__ inline wy_f4 wy_ld4(const float* p) { return *reinterpret_cast<const wy_f4*>(p); }
__device__ inline wy_bf8 wy_ld8(const uint16_t* p) { return *reinterpret_cast<const wy_bf8*>(p); }

__device__ inline void wy_wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__global__ __launch_bounds__(512) void gated_delta_wy_kernel(GdnArgs g) {
  __shared__ __align__(16) WyLds sm;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, l16 = lane & 15, lg = lane >> 4;
  const int64_t hv = blockIdx.y, bi = blockIdx.z;
  const int64_t hk = (int)blockIdx.y / g.hgrp;
  const int64_t dv0 = (int64_t)blockIdx.x * kWyRows;
  const int64_t srow0 = (bi * g.Hv + hv) * g.Dv + dv0;
  const bool kwave = w >= 4;                  // k rows, v and gates; else q rows
  const int u = kwave ? tid - 256 : tid, urow = u >> 2, upart = u & 3;

  // the state rows (f32) and the norm weights into LDS
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int c = tid + 512 * h, row = c >> 4, part = c & 15;
    float x[8];
    if (g.state_in) {
      const u32x4 raw = *reinterpret_cast<const u32x4*>(
          reinterpret_cast<const uint16_t*>(g.state_in) + (srow0 + row) * kWyDK + 8 * part);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = elem<BF16>(raw, e);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = 0.0f;
    }
    *reinterpret_cast<wy_f4*>(&sm.S[row][8 * part]) = wy_f4{x[0], x[1], x[2], x[3]};
    *reinterpret_cast<wy_f4*>(&sm.S[row][8 * part + 4]) = wy_f4{x[4], x[5], x[6], x[7]};
  }
  if (tid < 32) {
    const int part = tid & 15;
    const void* src = tid < 16 ? g.kw : g.qw;
    const u32x4 wv = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(src) + 8 * part);
    *reinterpret_cast<u32x4*>(tid < 16 ? &sm.wk[8 * part] : &sm.wq[8 * part]) = wv;
  }
  const float A = expf(load_param(g.a_log, g.pdt, hv));
  const float dtb = load_param(g.dt_bias, g.pdt, hv);
  const int64_t nch = (g.T + kWyC - 1) / kWyC;
  const int rt = w & 3;                              // this wave's 16-row tile of the state rows
  const int tA = w < 4 ? 0 : 1, tB = w < 4 ? 3 : 2;  // its two step tiles (balanced for M Delta)
  const uint16_t* wrow = kwave ? &sm.wk[32 * upart] : &sm.wq[32 * upart];

  // chunk 0: loads, normalised q / k rows, gates
  WyRaw raw;
  u32x4 nx[4];
  WyGates gt{};
  wy_fetch(g, raw, bi, hk, hv, dv0, 0, u, kwave, w == 4);
  __syncthreads();  // the norm weights
  wy_norm(raw.x, wrow, g.inv_dk, g.eps, urow < g.T, nx);
  if (w == 4) gt = wy_gates(raw, A, dtb, lane, (int)(g.T < kWyC ? g.T : kWyC));

  for (int64_t ch = 0; ch < nch; ++ch) {
    const int64_t t0 = ch * kWyC;
    const int n = (int)(g.T - t0 < kWyC ? g.T - t0 : kWyC);

    // ---- A: this chunk's normalised q / k rows, k^T, v and gates into LDS
    {
      uint16_t* dst = kwave ? &sm.Kh[urow][32 * upart] : &sm.Qh[urow][32 * upart];
#pragma unroll
      for (int c = 0; c < 4; ++c) *reinterpret_cast<u32x4*>(dst + 8 * c) = nx[c];
    }
    if (kwave) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          sm.KT[32 * upart + 8 * c + 2 * p][urow] = (uint16_t)(nx[c][p] & 0xffffu);
          sm.KT[32 * upart + 8 * c + 2 * p + 1][urow] = (uint16_t)(nx[c][p] >> 16);
        }
      const bool live = urow < n;
      *reinterpret_cast<u32x4*>(&sm.V[urow][16 * upart]) = live ? raw.v[0] : u32x4{0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4*>(&sm.V[urow][16 * upart + 8]) = live ? raw.v[1] : u32x4{0u, 0u, 0u, 0u};
      if (w == 4) {
        sm.lam2[lane] = gt.lam2;
        sm.beta[lane] = gt.beta;
        sm.eL[lane] = gt.eL;
        sm.eC[lane] = gt.eC;
      }
    }
    __syncthreads();

    // the next chunk's loads fly during this chunk's products (the last chunk
    // reloads its own steps, clamped into range)
    const int64_t tn = ch + 1 < nch ? t0 + kWyC : t0;
    wy_fetch(g, raw, bi, hk, hv, dv0, tn, u, kwave, w == 4);

    // ---- B1: tiles (i, j), j <= i, of k.k and q.k together (one k operand,
    // one decay factor) -> L, M
    for (int jj = w; jj < 10; jj += 8) {
      const int i = jj >= 6 ? 3 : jj >= 3 ? 2 : jj >= 1 ? 1 : 0;
      const int j = jj - i * (i + 1) / 2;
      const uint16_t* Ki = &sm.Kh[16 * i + l16][8 * lg];
      const uint16_t* Qi = &sm.Qh[16 * i + l16][8 * lg];
      const uint16_t* Kj = &sm.Kh[16 * j + l16][8 * lg];
      wy_f4 gk = {0.0f, 0.0f, 0.0f, 0.0f}, gq = gk;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const wy_bf8 bk = wy_ld8(Kj + 32 * ks);
        gk = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wy_ld8(Ki + 32 * ks), bk, gk, 0, 0, 0);
        gq = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wy_ld8(Qi + 32 * ks), bk, gq, 0, 0, 0);
      }
      const int tj = 16 * j + l16, ti0 = 16 * i + 4 * lg;
      const float lj = sm.lam2[tj];
      const wy_f4 li = wy_ld4(&sm.lam2[ti0]);
      const wy_f4 bi4 = wy_ld4(&sm.beta[ti0]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int ti = ti0 + r;
        const float dec = __builtin_amdgcn_exp2f(li[r] - lj);
        sm.M[ti][tj] = tj <= ti ? dec * gq[r] : 0.0f;
        sm.L[ti][tj] = tj < ti ? bi4[r] * dec * gk[r] : 0.0f;
      }
    }

    // ---- B2: K S^T -> R^T, and e^lam * Q S^T kept for y
    wy_f4 yacc[2];
    {
      wy_bf8 sh[4], sl[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const float* sp = &sm.S[16 * rt + l16][32 * ks + 8 * lg];
        const wy_f4 a0 = wy_ld4(sp), a1 = wy_ld4(sp + 4);
        const float x[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
        wy_split(x, sh[ks], sl[ks]);
      }
#pragma unroll
      for (int ts = 0; ts < 2; ++ts) {
        const int tt = ts ? tB : tA;
        wy_f4 p = {0.0f, 0.0f, 0.0f, 0.0f}, qs = p;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          const wy_bf8 ak = wy_ld8(&sm.Kh[16 * tt + l16][32 * ks + 8 * lg]);
          const wy_bf8 aq = wy_ld8(&sm.Qh[16 * tt + l16][32 * ks + 8 * lg]);
          p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak, sh[ks], p, 0, 0, 0);
          p = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak, sl[ks], p, 0, 0, 0);
          qs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aq, sh[ks], qs, 0, 0, 0);
          qs = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aq, sl[ks], qs, 0, 0, 0);
        }
        const int rr = 16 * rt + l16;
        wy_f4 rv;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 16 * tt + 4 * lg + r;
          const float vv = BF16::lo((uint32_t)sm.V[t][rr]);
          rv[r] = sm.beta[t] * (vv - sm.eL[t] * p[r]);
          yacc[ts][r] = sm.eL[t] * qs[r];
        }
        *reinterpret_cast<wy_f4*>(&sm.RD[rr][16 * tt + 4 * lg]) = rv;
      }
    }
    __syncthreads();

    // ---- C: Delta = (I + L)^{-1} R, waves 0..3, one 16-row tile of the state each
    // the next chunk's q rows (waves 0..3, interleaved with their solve) and k
    // rows and gates (waves 4..7); on the last chunk the results are unused
    {
      const int nn = (int)(g.T - tn < kWyC ? g.T - tn : kWyC);
      wy_norm(raw.x, wrow, g.inv_dk, g.eps, urow < nn, nx);
      if (w == 4) gt = wy_gates(raw, A, dtb, lane, nn);
    }
    if (w < 4) {
      {
        // column l16 of the inverse of diagonal block lg, by forward substitution;
        // every wave computes all four blocks and writes the same values
        float x[16];
        const int o = 16 * lg;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          float s = k == l16 ? 1.0f : 0.0f;
#pragma unroll
          for (int m = 0; m < k; ++m) s = __builtin_fmaf(-sm.L[o + k][o + m], x[m], s);
          x[k] = s;
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) sm.Td[lg][k][l16] = x[k];
      }
      wy_wave_sync();
      const int rr = 16 * rt + l16;
      wy_f4 dl[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        wy_f4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < i; ++j) {
          const wy_f4 a4 = wy_ld4(&sm.L[16 * i + l16][16 * j + 4 * lg]);
#pragma unroll
          for (int m = 0; m < 4; ++m) s = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[m], dl[j][m], s, 0, 0, 0);
        }
        const wy_f4 acc = wy_ld4(&sm.RD[rr][16 * i + 4 * lg]) - s;
        const wy_f4 td = wy_ld4(&sm.Td[i][l16][4 * lg]);
        wy_f4 d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int m = 0; m < 4; ++m) d = __builtin_amdgcn_mfma_f32_16x16x4f32(td[m], acc[m], d, 0, 0, 0);
        dl[i] = d;
        *reinterpret_cast<wy_f4*>(&sm.RD[rr][16 * i + 4 * lg]) = d;
      }
    }
    __syncthreads();

    // ---- D1: y = e^lam * Q S^T + M Delta, staged as bf16 in L's space
    uint16_t* ys = reinterpret_cast<uint16_t*>(&sm.L[0][0]);
    {
      const int rr = 16 * rt + l16;
#pragma unroll
      for (int ts = 0; ts < 2; ++ts) {
        const int tt = ts ? tB : tA;
        wy_f4 y = yacc[ts];
        for (int j = 0; j <= tt; ++j) {
          const wy_f4 a4 = wy_ld4(&sm.M[16 * tt + l16][16 * j + 4 * lg]);
          const wy_f4 b4 = wy_ld4(&sm.RD[rr][16 * j + 4 * lg]);
#pragma unroll
          for (int m = 0; m < 4; ++m) y = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[m], b4[m], y, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
          ys[(16 * tt + 4 * lg + r) * kWyTP + rr] = (uint16_t)(BF16::pack(y[r], 0.0f) & 0xffffu);
      }
    }
    // ---- D2: S <- e^{lam_C} S + (e^{lam_C - lam} * Delta)^T K, four 16 x 16 tiles per wave
    {
      wy_bf8 wh[2], wl[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int tb = 32 * ks + 8 * lg;
        const wy_f4 d0 = wy_ld4(&sm.RD[16 * rt + l16][tb]), d1 = wy_ld4(&sm.RD[16 * rt + l16][tb + 4]);
        const wy_f4 e0 = wy_ld4(&sm.eC[tb]), e1 = wy_ld4(&sm.eC[tb + 4]);
        const float x[8] = {d0[0] * e0[0], d0[1] * e0[1], d0[2] * e0[2], d0[3] * e0[3],
                            d1[0] * e1[0], d1[1] * e1[1], d1[2] * e1[2], d1[3] * e1[3]};
        wy_split(x, wh[ks], wl[ks]);
      }
      const float dec = sm.eL[kWyC - 1];
#pragma unroll
      for (int dd = 0; dd < 4; ++dd) {
        const int dt = (w >> 2) * 4 + dd;
        wy_f4 acc;
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = dec * sm.S[16 * rt + 4 * lg + r][16 * dt + l16];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const wy_bf8 b = wy_ld8(&sm.KT[16 * dt + l16][32 * ks + 8 * lg]);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wh[ks], b, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wl[ks], b, acc, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) sm.S[16 * rt + 4 * lg + r][16 * dt + l16] = acc[r];
      }
    }
    __syncthreads();

    // ---- D3: y rows of the live steps
    {
      const int s = tid >> 3, part = tid & 7;
      if (s < n) {
        const u32x4 o = *reinterpret_cast<const u32x4*>(&ys[s * kWyTP + 8 * part]);
        *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(g.y) +
                                  ((bi * g.T + t0 + s) * g.Hv + hv) * g.Dv + dv0 + 8 * part) = o;
      }
    }
  }

  // the state rows back, in bf16 (every wave's last state update is behind the
  // final barrier of the loop)
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int c = tid + 512 * h, row = c >> 4, part = c & 15;
    const wy_f4 a0 = wy_ld4(&sm.S[row][8 * part]), a1 = wy_ld4(&sm.S[row][8 * part + 4]);
    u32x4 o;
    o[0] = BF16::pack(a0[0], a0[1]);
    o[1] = BF16::pack(a0[2], a0[3]);
    o[2] = BF16::pack(a1[0], a1[1]);
    o[3] = BF16::pack(a1[2], a1[3]);
    *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(g.state_out) + (srow0 + row) * kWyDK + 8 * part) = o;
  }
}

// The state after zero steps when no input state is given: zeros.
__global__ __launch_bounds__(256) void gdn_zero_kernel(uint32_t* p, int64_t words) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < words; i += (int64_t)gridDim.x * 256)
    p[i] = 0u;
}

namespace {

template <class X, bool NORM>
bool launch_decode(const GdnArgs& a, hipStream_t s) {
  constexpr int RPL = 4;
  const dim3 grid((unsigned)((a.Dv + 16 * RPL - 1) / (16 * RPL)), (unsigned)a.Hv, (unsigned)a.B);
  switch (a.Dk) {
    case 32: HGK_LAUNCH((gated_delta_decode_kernel<X, 2, NORM, RPL>), grid, dim3(256), 0, s, a); return true;
    case 64: HGK_LAUNCH((gated_delta_decode_kernel<X, 4, NORM, RPL>), grid, dim3(256), 0, s, a); return true;
    case 128: HGK_LAUNCH((gated_delta_decode_kernel<X, 8, NORM, RPL>), grid, dim3(256), 0, s, a); return true;
    case 256: HGK_LAUNCH((gated_delta_decode_kernel<X, 16, NORM, RPL>), grid, dim3(256), 0, s, a); return true;
    default: return false;
  }
}

template <class X, class P, bool NORM>
bool launch_token_p(const GdnArgs& a, hipStream_t s) {
  constexpr int RPL = HGK_GDN_RPL, WPB = HGK_GDN_WPB, ROWS = 4 * RPL * WPB;
  const dim3 grid((unsigned)((a.Dv + ROWS - 1) / ROWS), (unsigned)a.Hv, (unsigned)a.B);
  const dim3 block(64 * WPB);
  switch (a.Dk) {
    case 32: HGK_LAUNCH((gated_delta_token_kernel<X, P, 2, NORM, RPL>), grid, block, 0, s, a); return true;
    case 64: HGK_LAUNCH((gated_delta_token_kernel<X, P, 4, NORM, RPL>), grid, block, 0, s, a); return true;
    case 128: HGK_LAUNCH((gated_delta_token_kernel<X, P, 8, NORM, RPL>), grid, block, 0, s, a); return true;
    case 256: HGK_LAUNCH((gated_delta_token_kernel<X, P, 16, NORM, RPL>), grid, block, 0, s, a); return true;
    default: return false;
  }
}

// The token kernel with the gated-norm epilogue: one block per (b, v-head)
// row of Dv (Dv <= the block's rows, a multiple of the rows per lane group).
template <class X, bool NORM>
bool launch_token_gn(const GdnArgs& a, hipStream_t s) {
  constexpr int RPL = HGK_GDN_RPL, WPB = HGK_GDN_WPB;
  static_assert(WPB == 4, "the epilogue reduces over a 256-thread block");
  const dim3 grid(1u, (unsigned)a.Hv, (unsigned)a.B);
  const dim3 block(64 * WPB);
  const bool p32 = a.pdt == DT_F32;
#define HGK_GDN_GN(NPT)                                                                          \
  if (p32) HGK_LAUNCH((gated_delta_token_kernel<X, F32, NPT, NORM, RPL, true>), grid,    \
                      block, 0, s, a);                                                   \
  else HGK_LAUNCH((gated_delta_token_kernel<X, X, NPT, NORM, RPL, true>), grid, block,  \
                          0, s, a);                                                              \
  return true;
  switch (a.Dk) {
    case 32: HGK_GDN_GN(2)
    case 64: HGK_GDN_GN(4)
    case 128: HGK_GDN_GN(8)
    case 256: HGK_GDN_GN(16)
    default: return false;
  }
#undef HGK_GDN_GN
}

// a_log / dt_bias in f32 or in the activation dtype (other pairings take the
// decode kernel, which reads them in any float dtype)
template <class X, bool NORM>
bool launch_token(const GdnArgs& a, hipStream_t s) {
  // the token kernel addresses the state with 32-bit buffer offsets
  if (a.B * a.Hv * a.Dv * a.Dk * X::kBytes >= ((int64_t)1 << 31)) return launch_decode<X, NORM>(a, s);
  if (a.pdt == DT_F32) return launch_token_p<X, F32, NORM>(a, s);
  if (a.pdt == X::kCode) return launch_token_p<X, X, NORM>(a, s);
  return launch_decode<X, NORM>(a, s);
}

template <class X, bool NORM>
bool launch_rows(const GdnArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)((a.Dv + 7) / 8), (unsigned)a.Hv, (unsigned)a.B);
  switch (a.Dk) {
    case 32: HGK_LAUNCH((gated_delta_row_kernel<X, 1, NORM>), grid, dim3(256), 0, s, a); return true;
    case 64: HGK_LAUNCH((gated_delta_row_kernel<X, 2, NORM>), grid, dim3(256), 0, s, a); return true;
    case 128: HGK_LAUNCH((gated_delta_row_kernel<X, 4, NORM>), grid, dim3(256), 0, s, a); return true;
    case 256: HGK_LAUNCH((gated_delta_row_kernel<X, 8, NORM>), grid, dim3(256), 0, s, a); return true;
    default: return false;
  }
}

template <class X, bool NORM>
bool launch_chunks(const GdnArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)((a.Dv + kRows - 1) / kRows), (unsigned)a.Hv, (unsigned)a.B);
  switch (a.Dk) {
    case 32: HGK_LAUNCH((gated_delta_chunk_kernel<X, 2, NORM>), grid, dim3(256), 0, s, a); return true;
    case 64: HGK_LAUNCH((gated_delta_chunk_kernel<X, 4, NORM>), grid, dim3(256), 0, s, a); return true;
    case 128: HGK_LAUNCH((gated_delta_chunk_kernel<X, 8, NORM>), grid, dim3(256), 0, s, a); return true;
    case 256: HGK_LAUNCH((gated_delta_chunk_kernel<X, 16, NORM>), grid, dim3(256), 0, s, a); return true;
    default: return false;
  }
}

// Steps per call up to which the barrier-free decode kernel runs.
constexpr int64_t kDecodeMaxSteps = 2;

// The WY kernel's shape: bf16 with the fused norm, Dk = 128, whole 64-row
// state tiles, 16-byte rows of v and y, and sequences long enough to fill
// its chunks.
bool wy_fits(const GdnArgs& a) {
  auto al = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  return a.Dk == kWyDK && a.Dv % kWyRows == 0 && a.T >= kWyMinSteps && al(a.v) && al(a.y) &&
         al(a.qw) && al(a.kw);
}

template <class X, bool NORM>
bool launch_x(const GdnArgs& a, hipStream_t s, bool aligned) {
  if (!aligned) return launch_rows<X, NORM>(a, s);
  if (a.T == 1) return launch_token<X, NORM>(a, s);
  if (a.T <= kDecodeMaxSteps) return launch_decode<X, NORM>(a, s);
  if constexpr (X::kCode == DT_BF16 && NORM) {
    if (wy_fits(a)) {
      const dim3 grid((unsigned)(a.Dv / kWyRows), (unsigned)a.Hv, (unsigned)a.B);
      HGK_LAUNCH(gated_delta_wy_kernel, grid, dim3(512), 0, s, a);
      return true;
    }
  }
  return launch_chunks<X, NORM>(a, s);
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
  // an empty call (no sequences, or no steps) may pass null data pointers
  if (!a_log || !dt_bias || (!state_out && batch > 0) ||
      ((!q || !k || !v || !a || !b || !y) && batch > 0 && seq_len > 0))
    return fail(HGK_ERR_ARG, "%s: null pointer", fn);
  if (batch > 65535 || v_heads > 65535) return fail(HGK_ERR_UNSUPPORTED, "%s: batch or v_heads > 65535", fn);
  if (batch == 0) return HGK_OK;
  if (seq_len == 0) {
    // no steps: the state passes through unchanged (zeros without an input state)
    const hipStream_t s0 = as_stream(stream);
    const int64_t bytes = batch * v_heads * head_v_dim * head_k_dim * dtype_bytes(dtype);
    if (state_in && state_in != state_out) {
      if (hipMemcpyAsync(state_out, state_in, (size_t)bytes, hipMemcpyDeviceToDevice, s0) != hipSuccess)
        return fail(HGK_ERR_HIP, "%s: state copy failed", fn);
    } else if (!state_in) {
      const int64_t words = bytes / 4;  // head_k_dim >= 32: whole words
      const int64_t blocks = std::min<int64_t>((words + 255) / 256, 4096);
      HGK_LAUNCH(gdn_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, s0,
                 static_cast<uint32_t*>(state_out), words);
    }
    return launch_status(fn);
  }
  GdnArgs g{};
  g.q = q; g.k = k; g.v = v; g.a_log = a_log; g.a = a; g.dt_bias = dt_bias; g.b = b;
  g.state_in = state_in; g.qw = q_norm_w; g.kw = k_norm_w; g.pdt = param_dtype; g.eps = eps;
  g.inv_dk = (float)(1.0 / (double)head_k_dim);
  g.B = batch; g.T = seq_len; g.Hk = k_heads; g.Dk = head_k_dim; g.Hv = v_heads; g.Dv = head_v_dim;
  g.hgrp = (int)(v_heads / k_heads);
  g.y = y; g.state_out = state_out;
  const hipStream_t s = as_stream(stream);
  const bool norm = q_norm_w != nullptr;
  // the chunked kernel loads q, k and state rows with 4- to 16-byte vector loads
  auto al = [](const void* p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; };
  const bool aligned = al(q) && al(k) && al(state_in) && al(state_out);
  bool ok;
  if (dtype == DT_BF16) ok = norm ? launch_x<BF16, true>(g, s, aligned) : launch_x<BF16, false>(g, s, aligned);
  else if (dtype == DT_F16) ok = norm ? launch_x<F16, true>(g, s, aligned) : launch_x<F16, false>(g, s, aligned);
  else ok = norm ? launch_x<F32, true>(g, s, aligned) : launch_x<F32, false>(g, s, aligned);
  if (!ok) return fail(HGK_ERR_UNSUPPORTED, "%s: head_k_dim not supported", fn);
  return launch_status(fn);
}

extern "C" int hgk_gated_delta_gated_norm(
    int dtype, const void* q, const void* k, const void* v, const void* a_log, const void* a,
    const void* dt_bias, const void* b, int param_dtype, const void* state_in,
    const void* q_norm_w, const void* k_norm_w, float eps, int64_t batch, int64_t k_heads,
    int64_t head_k_dim, int64_t v_heads, int64_t head_v_dim, void* state_out, void* y,
    const void* z, int64_t z_row_stride, int64_t z_group_rows, int64_t z_group_stride,
    const void* norm_w, int norm_w_dtype, float norm_eps, void* out, void* stream) {
  clear_error();
  const char* fn = "hgk_gated_delta_gated_norm";
  if (dtype != DT_BF16 && dtype != DT_F16 && dtype != DT_F32)
    return fail(HGK_ERR_ARG, "%s: dtype must be f32, bf16 or f16", fn);
  if (param_dtype != DT_F32 && param_dtype != dtype)
    return fail(HGK_ERR_UNSUPPORTED, "%s: a_log/dt_bias must be f32 or the activation dtype", fn);
  if (norm_w_dtype != dtype)
    return fail(HGK_ERR_UNSUPPORTED, "%s: the norm weight must have the activation dtype", fn);
  if (batch < 0 || k_heads <= 0 || v_heads <= 0 || head_v_dim <= 0 || v_heads % k_heads)
    return fail(HGK_ERR_ARG, "%s: bad shape", fn);
  if (head_k_dim != 32 && head_k_dim != 64 && head_k_dim != 128 && head_k_dim != 256)
    return fail(HGK_ERR_UNSUPPORTED, "%s: head_k_dim=%lld (32, 64, 128 or 256)", fn, (long long)head_k_dim);
  constexpr int RPL = HGK_GDN_RPL, ROWS = 4 * RPL * HGK_GDN_WPB;
  if (head_v_dim > ROWS || head_v_dim % RPL)
    return fail(HGK_ERR_UNSUPPORTED, "%s: head_v_dim=%lld (a multiple of %d up to %d)", fn,
                (long long)head_v_dim, RPL, ROWS);
  if ((q_norm_w == nullptr) != (k_norm_w == nullptr))
    return fail(HGK_ERR_ARG, "%s: pass both q and k norm weights or neither", fn);
  if (!(eps >= 0.0f) || !(norm_eps >= 0.0f)) return fail(HGK_ERR_ARG, "%s: eps must be >= 0", fn);
  if (!a_log || !dt_bias || !norm_w ||
      ((!q || !k || !v || !a || !b || !state_out || !z || !out) && batch > 0))
    return fail(HGK_ERR_ARG, "%s: null pointer", fn);
  const int64_t rows = batch * v_heads;
  if (z_group_rows <= 0 || z_group_rows > rows) {
    z_group_rows = rows > 0 ? rows : 1;
    z_group_stride = 0;
  }
  if ((z_group_rows > 1 && z_row_stride < head_v_dim) || z_row_stride < 0 ||
      (rows > z_group_rows && z_group_stride < (z_group_rows - 1) * z_row_stride + head_v_dim))
    return fail(HGK_ERR_ARG, "%s: z rows overlap", fn);
  if (batch > 65535 || v_heads > 65535) return fail(HGK_ERR_UNSUPPORTED, "%s: batch or v_heads > 65535", fn);
  const int64_t dk_bytes = dtype_bytes(dtype);
  if (batch * v_heads * head_v_dim * head_k_dim * dk_bytes >= ((int64_t)1 << 31))
    return fail(HGK_ERR_UNSUPPORTED, "%s: state of 2 GiB or more", fn);
  auto al = [](const void* p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; };
  const int vpc = 16 / (int)dk_bytes;  // elements per 16 bytes
  if (!al(q) || !al(k) || !al(state_in) || !al(state_out) || !al(z) || !al(norm_w) ||
      z_row_stride % vpc || z_group_stride % vpc)
    return fail(HGK_ERR_UNSUPPORTED, "%s: q, k, the state, z and the norm weight must be 16-byte aligned", fn);
  if (batch == 0) return HGK_OK;
  GdnArgs g{};
  g.q = q; g.k = k; g.v = v; g.a_log = a_log; g.a = a; g.dt_bias = dt_bias; g.b = b;
  g.state_in = state_in; g.qw = q_norm_w; g.kw = k_norm_w; g.pdt = param_dtype; g.eps = eps;
  g.inv_dk = (float)(1.0 / (double)head_k_dim);
  g.B = batch; g.T = 1; g.Hk = k_heads; g.Dk = head_k_dim; g.Hv = v_heads; g.Dv = head_v_dim;
  g.hgrp = (int)(v_heads / k_heads);
  g.y = y; g.state_out = state_out;
  g.gz = z; g.gzs = z_row_stride; g.gzg = z_group_rows; g.gzgs = z_group_stride; g.gw = norm_w;
  g.geps = norm_eps; g.inv_dv = (float)(1.0 / (double)head_v_dim); g.gout = out;
  const hipStream_t s = as_stream(stream);
  const bool norm = q_norm_w != nullptr;
  bool ok;
  if (dtype == DT_BF16) ok = norm ? launch_token_gn<BF16, true>(g, s) : launch_token_gn<BF16, false>(g, s);
  else if (dtype == DT_F16) ok = norm ? launch_token_gn<F16, true>(g, s) : launch_token_gn<F16, false>(g, s);
  else ok = norm ? launch_token_gn<F32, true>(g, s) : launch_token_gn<F32, false>(g, s);
  if (!ok) return fail(HGK_ERR_UNSUPPORTED, "%s: head_k_dim not supported", fn);
  return launch_status(fn);
}
