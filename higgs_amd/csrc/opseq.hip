// opseq.hip -- a decode step's per-layer op sequence in one launch.
//
// The reference runs each decoder layer as (qwen3_next.rs:1508-1547, for each
// of the 64 sequences of a continuous batch, batch_engine.rs:395-403):
//   normed = input_layernorm(h)                        -- add + RMSNorm
//   r = attention(normed)   gated RMSNorm (linear-attention layers) or
//                           q/k RMSNorm + partial RoPE (full-attention layers)
//   h2 = h + r; normed_post = post_attention_layernorm(h2)  -- add + RMSNorm
//   mlp_out = mlp(normed_post)                         -- SwiGLU of the experts
//   h = h2 + mlp_out
// Every one of those ops is row-wise: token t's outputs depend only on token
// t's inputs, and the residual stream of token t feeds only token t. So one
// workgroup per token walks the whole op list in order, with nothing but
// workgroup barriers between ops; no workgroup ever waits on another, so the
// grid needs no co-residency and no wait can hang.
//
// Each op waits for the previous op's stores to complete before any thread of
// the workgroup issues its first load (a wait on every outstanding memory
// operation, then the workgroup barrier), as the next op of a real layer
// would need them: the launch's time is the latency of the dependent chain,
// not the throughput of independent ops. Every consumer of an op's output
// inside the launch is the same workgroup, so workgroup-scope ordering is all
// the data needs; other consumers see it after the launch.
//
// Each op's arithmetic is the standalone kernel's (norm.hip, rope.hip,
// glu.hip) for 16-bit activations and weights of the same type: results are
// the same bits as the separate calls.
//
// The op list is a device array written by hgk_op_list_upload into memory the
// caller owns; this file allocates nothing.
#include <algorithm>
#include <cmath>
#include <vector>

#include "../../include/higgs_hip.h"
#include "hgk_act.h"
#include "hgk_common.h"
#include "hgk_host.h"

namespace hgk {

constexpr uint32_t kOpListMagic = 0x6f70736bu;  // "opsk"
constexpr int kOpMaxHalf = 256;                 // rotated dims / 2
constexpr int kOpThreads = 1024;

// One op as the kernel reads it (written by the host from an hgk_op).
struct alignas(16) DevOp {
  int32_t kind, act, rows, n;
  int32_t k_rows, dims, half, lpr;      // rope: k heads, rotated dims, dims / 2, lanes per row
  int32_t g, same_table, pad0, pad3;    // norms: lanes per row; rope: the cos/sin table of
                                        // the previous rope op serves (same positions, freqs)
  float eps, inv_n, scale, pad1;
  int64_t zg, zgs;                      // gated: z rows per group, group stride
  const void* x; int64_t x_tok, x_row;  // x / gate / q
  const void* r; int64_t r_tok, r_row;  // r / z / up / k
  const void* w; const void* w2;        // norm weight (q), k norm weight
  void* y; int64_t y_tok, y_row;        // y / out / q out
  void* h; int64_t h_tok, h_row;        // residual out / k out
  const int32_t* offsets;
  int32_t offset, pad2;
  float inv_freq[kOpMaxHalf];
};

struct alignas(16) DevOpList {
  uint32_t magic;
  int32_t dtype;
  int32_t count;
  int32_t pad;
  DevOp ops[1];  // count entries
};

constexpr int64_t op_list_bytes(int n) {
  return (int64_t)sizeof(DevOpList) + (int64_t)(n - 1) * (int64_t)sizeof(DevOp);
}

enum { kOpRms = 0, kOpAddRms = 1, kOpGated = 2, kOpRope = 3, kOpGlu = 4 };

// Whether an op waits for its stores to complete before the next op starts
// (1), or only orders them before the next op's loads through the barrier (0).
#ifndef HGK_OPSEQ_STORE_WAIT
#define HGK_OPSEQ_STORE_WAIT 1
#endif
// Whether each op brings the next op's descriptor into the scalar cache.
#ifndef HGK_OPSEQ_PREFETCH
#define HGK_OPSEQ_PREFETCH 1
#endif

// Every store of this op has completed before any thread of the workgroup
// issues the next op's loads.
__device__ inline void op_boundary() {
  if (HGK_OPSEQ_STORE_WAIT) __builtin_amdgcn_s_waitcnt(0);  // all counters: loads, stores, LDS
  __syncthreads();
}

// f64 sum over the G lanes of a row group; G = 128 or 256 spans waves and
// goes through LDS (`part`, one slot per wave). Every thread calls it (it
// holds a workgroup barrier when G > 64).
template <int G>
__device__ inline double row_sum(double v, double* part) {
  if constexpr (G <= 64) {
    return group_sum<G>(v);
  } else {
    v = group_sum<64>(v);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) part[wave] = v;
    __syncthreads();
    constexpr int WPG = G / 64;  // waves per group
    const int first = wave / WPG * WPG;
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < WPG; ++k) s += part[first + k];
    __syncthreads();  // the slots are reused by the next row
    return s;
  }
}

// RMSNorm / add + RMSNorm / gated RMSNorm over the token's rows: G lanes per
// row (G a power of two, 4..1024), one 16-byte unit per lane, 1024 / G rows
// per pass (a token's 32 head rows of 128 in one pass). rms_norm_kernel's
// arithmetic, 16-bit X, weights in X.
template <class X, int MODE, int G>
__device__ void op_norm(const DevOp& op, int64_t t, double* part) {
  constexpr int V = Vec<X>::N;
  constexpr int P = kOpThreads / G;  // rows per pass
  const int slot = threadIdx.x / G, j = threadIdx.x % G;
  const int nch = op.n / V;
  const bool has_w = op.w != nullptr;
  const int chc = j < nch ? j : nch - 1;
  const char* xb = reinterpret_cast<const char*>(op.x) + t * op.x_tok * X::kBytes;
  const char* rb = reinterpret_cast<const char*>(op.r) + t * op.r_tok * X::kBytes;
  char* yb = reinterpret_cast<char*>(op.y) + t * op.y_tok * X::kBytes;
  char* hb = reinterpret_cast<char*>(op.h) + t * op.h_tok * X::kBytes;
  const u32x4 wr = has_w ? ld16<X>(op.w, (int64_t)chc * V) : u32x4{0u, 0u, 0u, 0u};
  for (int pass = 0; pass * P < op.rows; ++pass) {  // uniform over the workgroup
    const int row = pass * P + slot;
    const bool live = row < op.rows;
    const int rr = live ? row : op.rows - 1;
    int64_t zoff = 0;
    if constexpr (MODE == kOpGated) zoff = (rr / op.zg) * op.zgs + (rr % op.zg) * op.r_row;
    if constexpr (MODE == kOpAddRms) zoff = (int64_t)rr * op.r_row;
    u32x4 xr = ld16<X>(xb, (int64_t)rr * op.x_row + (int64_t)chc * V);
    u32x4 zr{0u, 0u, 0u, 0u};
    if constexpr (MODE != kOpRms) zr = ld16<X>(rb, zoff + (int64_t)chc * V);
    const bool own = live && j < nch;
    if constexpr (MODE == kOpAddRms) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        xr[k] = X::pack(X::lo(xr[k]) + X::lo(zr[k]), X::hi(xr[k]) + X::hi(zr[k]));
      if (op.h && own)
        *reinterpret_cast<u32x4*>(hb + ((int64_t)row * op.h_row + (int64_t)j * V) * X::kBytes) = xr;
    }
    double ss = 0.0;
    if (j < nch) {
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const double d = (double)elem<X>(xr, e);
        ss = __builtin_fma(d, d, ss);
      }
    }
    ss = row_sum<G>(ss, part);
    const float rs = rms_scale(ss, op.inv_n, op.eps);
    if (!own) continue;
    float o[V];
#pragma unroll
    for (int e = 0; e < V; e += 2) {
      float n0 = elem<X>(xr, e) * rs, n1 = elem<X>(xr, e + 1) * rs;
      round2<X>(n0, n1);
      const float w0 = has_w ? elem<X>(wr, e) : 1.0f, w1 = has_w ? elem<X>(wr, e + 1) : 1.0f;
      n0 = n0 * w0;
      n1 = n1 * w1;
      if constexpr (MODE == kOpGated) {
        round2<X>(n0, n1);
        const float z0 = elem<X>(zr, e), z1 = elem<X>(zr, e + 1);
        float s0, s1;
        sigmoid2_rounded<X>(z0, z1, s0, s1);
        float g0 = z0 * s0, g1 = z1 * s1;
        round2<X>(g0, g1);
        n0 = g0 * n0;
        n1 = g1 * n1;
      }
      o[e] = n0;
      o[e + 1] = n1;
    }
    store_elems<X, V, false>(yb, (int64_t)row * op.y_row + (int64_t)j * V, o);
  }
}

// q/k RMSNorm (where a weight is given) + RoPE of the token's q and k heads:
// rope_kernel's two-chunk layout (lane j < R holds the rotation pair j, j + R;
// the others hold two pass-through chunks), LPR lanes per head row, every
// load issued before the cos/sin table is built. The table (cos/sin of the
// token's position from f64 sincos, rounded to X) lives in LDS; an op whose
// positions and frequencies are those of the previous rope op reuses it.
template <class X, int LPR>
__device__ void op_rope(const DevOp& op, int64_t t, float* cs, float* sn) {
  constexpr int V = Vec<X>::N;
  constexpr int P = kOpThreads / LPR;
  const int R = op.dims / (2 * V);
  const int slot = threadIdx.x / LPR, j = threadIdx.x % LPR;
  const bool rot = j < R;
  const int c0 = rot ? j : 2 * j, c1 = rot ? j + R : 2 * j + 1;
  const int total = op.rows + op.k_rows;
  for (int pass = 0; pass * P < total; ++pass) {  // uniform over the workgroup
    const int row = pass * P + slot;
    const int rc = row < total ? row : total - 1;
    const bool isk = rc >= op.rows;
    const int hh = isk ? rc - op.rows : rc;
    const char* xp = isk ? reinterpret_cast<const char*>(op.r) +
                               (t * op.r_tok + (int64_t)hh * op.r_row) * X::kBytes
                         : reinterpret_cast<const char*>(op.x) +
                               (t * op.x_tok + (int64_t)hh * op.x_row) * X::kBytes;
    char* yp = isk ? reinterpret_cast<char*>(op.h) + (t * op.h_tok + (int64_t)hh * op.h_row) * X::kBytes
                   : reinterpret_cast<char*>(op.y) + (t * op.y_tok + (int64_t)hh * op.y_row) * X::kBytes;
    const void* nw = isk ? op.w2 : op.w;
    const bool has = nw != nullptr;
    const u32x4 d0 = ld16<X>(xp, (int64_t)c0 * V), d1 = ld16<X>(xp, (int64_t)c1 * V);
    const u32x4 wa = has ? ld16<X>(nw, (int64_t)c0 * V) : u32x4{0u, 0u, 0u, 0u};
    const u32x4 wb = has ? ld16<X>(nw, (int64_t)c1 * V) : u32x4{0u, 0u, 0u, 0u};
    if (pass == 0 && !op.same_table) {  // built while the loads are in flight
      const int32_t off = op.offsets ? op.offsets[t] : op.offset;
      const float pos = (0.0f + (float)off) * op.scale;
      for (int i = threadIdx.x; i < op.half; i += kOpThreads) {
        float c, s;
        cos_sin_f32(pos * op.inv_freq[i], c, s);
        cs[i] = X::round(c);
        sn[i] = X::round(s);
      }
      __syncthreads();
    }
    if (row >= total) continue;  // whole lane groups leave together; no barrier below
    float v0[V], v1[V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
      v0[e] = elem<X>(d0, e);
      v1[e] = elem<X>(d1, e);
    }
    if (has) {  // uniform over the row's lanes
      double ss = 0.0;
#pragma unroll
      for (int e = 0; e < V; ++e) ss = __builtin_fma((double)v0[e], (double)v0[e], ss);
#pragma unroll
      for (int e = 0; e < V; ++e) ss = __builtin_fma((double)v1[e], (double)v1[e], ss);
      ss = group_sum<LPR>(ss);
      const float rs = rms_scale(ss, op.inv_n, op.eps);
#pragma unroll
      for (int e = 0; e < V; e += 2) {
        float p0 = v0[e] * rs, p1 = v0[e + 1] * rs, q0 = v1[e] * rs, q1 = v1[e + 1] * rs;
        round2<X>(p0, p1);
        round2<X>(q0, q1);
        p0 = p0 * elem<X>(wa, e);
        p1 = p1 * elem<X>(wa, e + 1);
        q0 = q0 * elem<X>(wb, e);
        q1 = q1 * elem<X>(wb, e + 1);
        round2<X>(p0, p1);
        round2<X>(q0, q1);
        v0[e] = p0; v0[e + 1] = p1; v1[e] = q0; v1[e + 1] = q1;
      }
    }
    if (rot) {
      const float* cp = cs + j * V;
      const float* sp = sn + j * V;
#pragma unroll
      for (int e = 0; e < V; e += 2) {
        const float ca = cp[e], sa = sp[e], cb = cp[e + 1], sb = sp[e + 1];
        const float x10 = v0[e], x20 = v1[e], x11 = v0[e + 1], x21 = v1[e + 1];
        float a0 = x10 * ca, a1 = x11 * cb, b0 = x20 * sa, b1 = x21 * sb;
        float d0v = x10 * sa, d1v = x11 * sb, f0 = x20 * ca, f1 = x21 * cb;
        round2<X>(a0, a1);
        round2<X>(b0, b1);
        round2<X>(d0v, d1v);
        round2<X>(f0, f1);
        v0[e] = a0 - b0;
        v0[e + 1] = a1 - b1;
        v1[e] = d0v + f0;
        v1[e + 1] = d1v + f1;
      }
    }
    store_elems<X, V, false>(yp, (int64_t)c0 * V, v0);
    store_elems<X, V, false>(yp, (int64_t)c1 * V, v1);
  }
}

// act(gate) * up over the token's rows: one 16-byte unit per thread per pass
// (glu_kernel's arithmetic).
template <class X, int ACT>
__device__ void op_glu(const DevOp& op, int64_t t) {
  constexpr int V = Vec<X>::N;
  const int cpr = op.n / V;
  const int total = op.rows * cpr;
  const char* gb = reinterpret_cast<const char*>(op.x) + t * op.x_tok * X::kBytes;
  const char* ub = reinterpret_cast<const char*>(op.r) + t * op.r_tok * X::kBytes;
  char* ob = reinterpret_cast<char*>(op.y) + t * op.y_tok * X::kBytes;
  for (int q = threadIdx.x; q < total; q += kOpThreads) {
    const int row = q / cpr, c = q - row * cpr;
    const u32x4 gr = ld16<X>(gb, (int64_t)row * op.x_row + (int64_t)c * V);
    const u32x4 ur = ld16<X>(ub, (int64_t)row * op.r_row + (int64_t)c * V);
    float o[V];
    if constexpr (ACT == HGK_ACT_SILU) {
      float gv[V], uv[V];
#pragma unroll
      for (int e = 0; e < V; ++e) {
        gv[e] = elem<X>(gr, e);
        uv[e] = elem<X>(ur, e);
      }
      swiglu16<X, V>(gv, uv, o);
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e) o[e] = glu1<X, ACT>(elem<X>(gr, e), elem<X>(ur, e));
    }
    store_elems<X, V, false>(ob, (int64_t)row * op.y_row + (int64_t)c * V, o);
  }
}

template <class X, int MODE>
__device__ void norm_dispatch(const DevOp& op, int64_t t, double* part) {
  switch (op.g) {
    case 4: op_norm<X, MODE, 4>(op, t, part); break;
    case 8: op_norm<X, MODE, 8>(op, t, part); break;
    case 16: op_norm<X, MODE, 16>(op, t, part); break;
    case 32: op_norm<X, MODE, 32>(op, t, part); break;
    case 64: op_norm<X, MODE, 64>(op, t, part); break;
    case 128: op_norm<X, MODE, 128>(op, t, part); break;
    case 256: op_norm<X, MODE, 256>(op, t, part); break;
    case 512: op_norm<X, MODE, 512>(op, t, part); break;
    default: op_norm<X, MODE, 1024>(op, t, part); break;
  }
}

template <class X>
__global__ __launch_bounds__(kOpThreads) void opseq_kernel(const DevOpList* __restrict__ list,
                                                           int n_ops) {
  __shared__ float cs[kOpMaxHalf], sn[kOpMaxHalf];
  __shared__ double part[kOpThreads / 64];
  const int64_t t = blockIdx.x;
  // a list that hgk_op_list_upload did not write for this dtype and length
  // is not walked (no pointer in it is trusted)
  if (list->magic != kOpListMagic || list->dtype != X::kCode || list->count < n_ops) return;
  for (int i = 0; i < n_ops; ++i) {
    const DevOp& op = list->ops[i];
    uint32_t pf[4] = {0u, 0u, 0u, 0u};
    if (HGK_OPSEQ_PREFETCH && i + 1 < n_ops) {
      // one dword of each 64-byte line of the next descriptor's fields
      const uint32_t* nx = reinterpret_cast<const uint32_t*>(&list->ops[i + 1]);
      pf[0] = nx[0]; pf[1] = nx[16]; pf[2] = nx[32]; pf[3] = nx[48];
    }
    switch (op.kind) {
      case kOpRms: norm_dispatch<X, kOpRms>(op, t, part); break;
      case kOpAddRms: norm_dispatch<X, kOpAddRms>(op, t, part); break;
      case kOpGated: norm_dispatch<X, kOpGated>(op, t, part); break;
      case kOpRope:
        switch (op.lpr) {
          case 2: op_rope<X, 2>(op, t, cs, sn); break;
          case 4: op_rope<X, 4>(op, t, cs, sn); break;
          case 8: op_rope<X, 8>(op, t, cs, sn); break;
          case 16: op_rope<X, 16>(op, t, cs, sn); break;
          default: op_rope<X, 32>(op, t, cs, sn); break;
        }
        break;
      default:
        if (op.act == HGK_ACT_SILU) op_glu<X, HGK_ACT_SILU>(op, t);
        else op_glu<X, HGK_ACT_GELU_TANH>(op, t);
        break;
    }
    if (HGK_OPSEQ_PREFETCH) asm volatile("" ::"s"(pf[0]), "s"(pf[1]), "s"(pf[2]), "s"(pf[3]));
    op_boundary();
  }
}

namespace {

bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int next_pow2(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

// Translate and check one host op; returns HGK_OK or an error status.
int translate(const hgk_op& s, int i, DevOp& d) {
  const char* fn = "hgk_op_list_upload";
  const int V = 8;  // 16-bit elements per 16-byte unit
  d = DevOp{};
  d.kind = s.kind;
  d.rows = s.rows;
  d.n = s.n;
  d.eps = s.eps;
  d.x = s.x; d.x_tok = s.x_tok; d.x_row = s.x_row;
  d.r = s.r; d.r_tok = s.r_tok; d.r_row = s.r_row;
  d.w = s.w; d.w2 = s.w2;
  d.y = s.y; d.y_tok = s.y_tok; d.y_row = s.y_row;
  d.h = s.h; d.h_tok = s.h_tok; d.h_row = s.h_row;
  if (s.rows <= 0 || s.n <= 0 || s.n % V)
    return fail(HGK_ERR_ARG, "%s: op %d: rows=%d n=%d (rows > 0, n a positive multiple of 8)", fn,
                i, s.rows, s.n);
  auto strides_ok = [&](const void* p, int64_t tok, int64_t row) {
    return p && a16(p) && tok % V == 0 && row % V == 0 && tok >= 0 && row >= 0;
  };
  if (!strides_ok(s.x, s.x_tok, s.x_row) || !strides_ok(s.y, s.y_tok, s.y_row))
    return fail(HGK_ERR_ARG, "%s: op %d: x and y must be 16-byte aligned with strides in whole "
                "16-byte units", fn, i);
  if (s.w && !a16(s.w)) return fail(HGK_ERR_ARG, "%s: op %d: weight not 16-byte aligned", fn, i);
  const int nch = s.n / V;
  switch (s.kind) {
    case HGK_OP_RMS_NORM:
    case HGK_OP_ADD_RMS_NORM:
    case HGK_OP_GATED_RMS_NORM: {
      if (!(s.eps >= 0.0f)) return fail(HGK_ERR_ARG, "%s: op %d: eps must be >= 0", fn, i);
      if (nch > kOpThreads)
        return fail(HGK_ERR_UNSUPPORTED, "%s: op %d: n=%d (at most %d)", fn, i, s.n, 8 * kOpThreads);
      if (s.kind != HGK_OP_RMS_NORM && !strides_ok(s.r, s.r_tok, s.r_row))
        return fail(HGK_ERR_ARG, "%s: op %d: r/z must be 16-byte aligned with strides in whole "
                    "16-byte units", fn, i);
      if (s.kind == HGK_OP_ADD_RMS_NORM && s.h && !strides_ok(s.h, s.h_tok, s.h_row))
        return fail(HGK_ERR_ARG, "%s: op %d: h must be 16-byte aligned with strides in whole "
                    "16-byte units", fn, i);
      if (s.kind == HGK_OP_GATED_RMS_NORM) {
        if (!s.w) return fail(HGK_ERR_ARG, "%s: op %d: the gated norm needs a weight", fn, i);
        d.zg = s.z_group_rows > 0 ? s.z_group_rows : s.rows;
        d.zgs = s.z_group_rows > 0 ? s.z_group_stride : 0;
        if (d.zgs % V) return fail(HGK_ERR_ARG, "%s: op %d: z group stride not whole units", fn, i);
      } else {
        d.zg = 1;
      }
      d.g = std::min(kOpThreads, std::max(4, next_pow2(nch)));
      d.inv_n = (float)(1.0 / (double)s.n);
      return HGK_OK;
    }
    case HGK_OP_QK_NORM_ROPE: {
      const int D = s.n;
      if (D < 32 || D > 512 || (D & (D - 1)))
        return fail(HGK_ERR_UNSUPPORTED, "%s: op %d: head_dim %d (a power of two, 32..512)", fn,
                    i, D);
      if (s.dims <= 0 || s.dims > D || s.dims % 16)
        return fail(HGK_ERR_UNSUPPORTED, "%s: op %d: rotated dims %d (a multiple of 16 up to "
                    "head_dim)", fn, i, s.dims);
      if (s.k_heads < 0) return fail(HGK_ERR_ARG, "%s: op %d: k_heads < 0", fn, i);
      if (s.k_heads > 0 && (!strides_ok(s.r, s.r_tok, s.r_row) || !strides_ok(s.h, s.h_tok, s.h_row)))
        return fail(HGK_ERR_ARG, "%s: op %d: k and its output must be 16-byte aligned with "
                    "strides in whole 16-byte units", fn, i);
      if (s.w2 && !a16(s.w2)) return fail(HGK_ERR_ARG, "%s: op %d: k weight not aligned", fn, i);
      if (s.w && !(s.eps >= 0.0f)) return fail(HGK_ERR_ARG, "%s: op %d: eps must be >= 0", fn, i);
      if (s.offsets && (reinterpret_cast<uintptr_t>(s.offsets) & 3u))
        return fail(HGK_ERR_ARG, "%s: op %d: offsets not 4-byte aligned", fn, i);
      d.k_rows = s.k_heads;
      d.dims = s.dims;
      d.half = s.dims / 2;
      d.lpr = D / 16;
      d.scale = s.scale;
      d.offsets = s.offsets;
      d.offset = s.offset;
      d.inv_n = (float)(1.0 / (double)D);
      const int st = hgk_rope_inv_freq(s.base, s.dims, s.freqs, d.inv_freq);
      if (st) return st;
      return HGK_OK;
    }
    case HGK_OP_GLU: {
      if (s.act != HGK_ACT_SILU && s.act != HGK_ACT_GELU_TANH)
        return fail(HGK_ERR_ARG, "%s: op %d: activation %d", fn, i, s.act);
      if (!strides_ok(s.r, s.r_tok, s.r_row))
        return fail(HGK_ERR_ARG, "%s: op %d: up must be 16-byte aligned with strides in whole "
                    "16-byte units", fn, i);
      if ((int64_t)s.rows * s.n > ((int64_t)1 << 30))
        return fail(HGK_ERR_UNSUPPORTED, "%s: op %d: rows x n too large", fn, i);
      d.act = s.act;
      return HGK_OK;
    }
    default:
      return fail(HGK_ERR_ARG, "%s: op %d: unknown kind %d", fn, i, s.kind);
  }
}

}  // namespace
}  // namespace hgk

using namespace hgk;

extern "C" int64_t hgk_op_list_bytes(int n_ops) {
  if (n_ops <= 0 || n_ops > HGK_OP_LIST_MAX) return -1;
  return op_list_bytes(n_ops);
}

extern "C" int hgk_op_list_upload(int dtype, const hgk_op* ops, int n_ops, void* dev_list,
                                  int64_t dev_bytes, void* stream) {
  clear_error();
  const char* fn = "hgk_op_list_upload";
  if (dtype != DT_BF16 && dtype != DT_F16)
    return fail(HGK_ERR_UNSUPPORTED, "%s: dtype %s (bf16 or f16)", fn, dtype_name(dtype));
  if (!ops || n_ops <= 0 || n_ops > HGK_OP_LIST_MAX)
    return fail(HGK_ERR_ARG, "%s: %d ops (1..%d)", fn, n_ops, HGK_OP_LIST_MAX);
  if (!dev_list || !a16(dev_list)) return fail(HGK_ERR_ARG, "%s: null or unaligned list", fn);
  const int64_t need = op_list_bytes(n_ops);
  if (dev_bytes < need)
    return fail(HGK_ERR_ARG, "%s: %lld bytes given, %lld needed", fn, (long long)dev_bytes,
                (long long)need);
  std::vector<char> host((size_t)need, 0);
  DevOpList* L = reinterpret_cast<DevOpList*>(host.data());
  L->magic = kOpListMagic;
  L->dtype = dtype;
  L->count = n_ops;
  int last_rope = -1;
  for (int i = 0; i < n_ops; ++i) {
    const int st = translate(ops[i], i, L->ops[i]);
    if (st) return st;
    DevOp& d = L->ops[i];
    if (d.kind != kOpRope) continue;
    // the previous rope op's table is still in LDS when this op runs: reuse it
    // when the positions and frequencies are the same
    if (last_rope >= 0) {
      const DevOp& p = L->ops[last_rope];
      d.same_table = p.offsets == d.offsets && p.offset == d.offset && p.scale == d.scale &&
                     p.half == d.half &&
                     std::equal(d.inv_freq, d.inv_freq + d.half, p.inv_freq);
    }
    last_rope = i;
  }
  hipError_t e = hipMemcpyAsync(dev_list, host.data(), (size_t)need, hipMemcpyHostToDevice,
                                as_stream(stream));
  if (e == hipSuccess) e = hipStreamSynchronize(as_stream(stream));
  if (e != hipSuccess) return fail(HGK_ERR_HIP, "%s: copy failed: %s", fn, hipGetErrorString(e));
  return HGK_OK;
}

extern "C" int hgk_op_list_run(int dtype, const void* dev_list, int n_ops, int64_t tokens,
                               void* stream) {
  clear_error();
  const char* fn = "hgk_op_list_run";
  if (dtype != DT_BF16 && dtype != DT_F16)
    return fail(HGK_ERR_UNSUPPORTED, "%s: dtype %s (bf16 or f16)", fn, dtype_name(dtype));
  if (!dev_list || !a16(dev_list)) return fail(HGK_ERR_ARG, "%s: null or unaligned list", fn);
  if (n_ops <= 0 || n_ops > HGK_OP_LIST_MAX)
    return fail(HGK_ERR_ARG, "%s: %d ops (1..%d)", fn, n_ops, HGK_OP_LIST_MAX);
  if (tokens < 0 || tokens > ((int64_t)1 << 31) - 1)
    return fail(HGK_ERR_ARG, "%s: tokens=%lld", fn, (long long)tokens);
  if (tokens == 0) return HGK_OK;
  const DevOpList* L = static_cast<const DevOpList*>(dev_list);
  const dim3 g((unsigned)tokens), b(kOpThreads);
  if (dtype == DT_BF16) HGK_LAUNCH((opseq_kernel<BF16>), g, b, 0, as_stream(stream), L, n_ops);
  else HGK_LAUNCH((opseq_kernel<F16>), g, b, 0, as_stream(stream), L, n_ops);
  return launch_status(fn);
}
