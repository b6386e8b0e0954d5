// rope.hip -- RoPE (default / explicit-frequency e.g. llama3 / partial rotary,
// per-sequence offsets) with an optional fused per-head RMSNorm (Qwen3
// q_norm/k_norm), for q and k in one launch, on gfx950.
//
// Work split: a block owns `tpb` consecutive tokens (token = b*L + l) and
// every head row of q and k for those tokens.
//  phase A: the block fills an LDS table of cos/sin for its tokens x dims/2
//           frequencies (computed once per (token, frequency) and shared by all
//           heads), rounded to the activation dtype as MLX's fallback does.
//  phase B: a group of LPR = head_dim/(2*V) lanes owns one head row; lane j
//           holds two 16-byte chunks: the rotation pair (j, j+R) when
//           j < R = dims/(2*V), else the pass-through chunks (2j, 2j+1). The
//           row is read once, optionally normalised (group shuffle reduction),
//           rotated and written once to an arbitrary (b, l, h) layout, which
//           folds the [B,L,H,D] -> [B,H,L,D] transpose into the store.
//
// Arithmetic (MLX CPU fallback of fast::rope, T = activation dtype):
//   pos = (f32(l) + offset_b) * scale;  th = pos * inv_freq[i]
//   c = round_T(cos th), s = round_T(sin th)
//   y1 = round_T(round_T(x1*c) - round_T(x2*s))
//   y2 = round_T(round_T(x1*s) + round_T(x2*c))
// cos/sin are evaluated in f64 and rounded to f32 (close to correctly rounded
// even at |th| ~ 3e4), then to T.
#include <algorithm>

#include "../../include/higgs_hip.h"
#include "hgk_common.h"
#include "hgk_host.h"

namespace hgk {

constexpr int kMaxHalf = 256;
constexpr int kMaxTpb = 16;

struct RopeTensor {
  const void* x;
  void* y;
  int64_t xs0, xs1, xs2;
  int64_t ys0, ys1, ys2;
  const void* nw;  // per-head norm weight [D] or null
  int heads;
};

struct RopeArgs {
  RopeTensor t[2];  // q, k
  const int32_t* offsets;
  int32_t offset;
  uint32_t L;
  uint32_t tokens;
  int D, dims, half, R, tpb, hsum;
  float scale, eps, inv_d;
  float inv_freq[kMaxHalf];
};

template <class X>
__device__ inline void fill_table(const RopeArgs& a, float* cs, float* sn, uint32_t t0, int ntok) {
  for (int e = threadIdx.x; e < ntok * a.half; e += blockDim.x) {
    const int tk = e / a.half;
    const int i = e - tk * a.half;
    const uint32_t tok = t0 + tk;
    const uint32_t b = tok / a.L, l = tok - b * a.L;
    const int32_t off = a.offsets ? a.offsets[b] : a.offset;
    const float pos = ((float)l + (float)off) * a.scale;
    const float th = pos * a.inv_freq[i];
    double s, c;
    sincos((double)th, &s, &c);
    cs[e] = X::round((float)c);
    sn[e] = X::round((float)s);
  }
}

template <class X, int LPR, bool NORM>
__global__ __launch_bounds__(256) void rope_kernel(RopeArgs a) {
  constexpr int V = Vec<X>::N;
  extern __shared__ float smem[];
  float* cs = smem;
  float* sn = smem + a.tpb * a.half;
  const uint32_t t0 = blockIdx.x * (uint32_t)a.tpb;
  const int ntok = (int)min((uint32_t)a.tpb, a.tokens - t0);
  fill_table<X>(a, cs, sn, t0, ntok);
  __syncthreads();

  const int slots = blockDim.x / LPR;
  const int slot = threadIdx.x / LPR;
  const int j = threadIdx.x % LPR;
  const bool rot = j < a.R;
  const int c0 = rot ? j : 2 * j;
  const int c1 = rot ? j + a.R : 2 * j + 1;

  float wq[2][V], wk[2][V];
  if constexpr (NORM) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const void* nw = a.t[h].nw;
      float(*w)[V] = h ? wk : wq;
      if (nw) {
        load_chunk<X>(nw, c0 * V, w[0]);
        load_chunk<X>(nw, c1 * V, w[1]);
      } else {
#pragma unroll
        for (int e = 0; e < V; ++e) w[0][e] = w[1][e] = 1.0f;
      }
    }
  }

  const int rows = ntok * a.hsum;
  for (int rr = slot; rr < rows; rr += slots) {
    const int tk = rr / a.hsum;
    const int h = rr - tk * a.hsum;
    const bool isk = h >= a.t[0].heads;
    const int hh = isk ? h - a.t[0].heads : h;
    const uint32_t tok = t0 + tk;
    const uint32_t b = tok / a.L, l = tok - b * a.L;
    const void* xp = isk ? a.t[1].x : a.t[0].x;
    void* yp = isk ? a.t[1].y : a.t[0].y;
    const int64_t xb = (int64_t)b * (isk ? a.t[1].xs0 : a.t[0].xs0) +
                       (int64_t)l * (isk ? a.t[1].xs1 : a.t[0].xs1) +
                       (int64_t)hh * (isk ? a.t[1].xs2 : a.t[0].xs2);
    const int64_t yb = (int64_t)b * (isk ? a.t[1].ys0 : a.t[0].ys0) +
                       (int64_t)l * (isk ? a.t[1].ys1 : a.t[0].ys1) +
                       (int64_t)hh * (isk ? a.t[1].ys2 : a.t[0].ys2);
    float v0[V], v1[V];
    load_chunk<X>(xp, xb + c0 * V, v0);
    load_chunk<X>(xp, xb + c1 * V, v1);
    if constexpr (NORM) {
      const bool has = isk ? (a.t[1].nw != nullptr) : (a.t[0].nw != nullptr);
      if (has) {  // uniform across the row's lane group
        double ss = 0.0;
#pragma unroll
        for (int e = 0; e < V; ++e) ss = __builtin_fma((double)v0[e], (double)v0[e], ss);
#pragma unroll
        for (int e = 0; e < V; ++e) ss = __builtin_fma((double)v1[e], (double)v1[e], ss);
        ss = group_sum<LPR>(ss);
        const float r = rms_scale(ss, a.inv_d, a.eps);
#pragma unroll
        for (int e = 0; e < V; ++e) {
          const float w0 = isk ? wk[0][e] : wq[0][e];
          const float w1 = isk ? wk[1][e] : wq[1][e];
          v0[e] = X::round(X::round(v0[e] * r) * w0);
          v1[e] = X::round(X::round(v1[e] * r) * w1);
        }
      }
    }
    if (rot) {
      const float* cp = cs + tk * a.half + j * V;
      const float* sp = sn + tk * a.half + j * V;
#pragma unroll
      for (int e = 0; e < V; ++e) {
        const float c = cp[e], s = sp[e];
        const float x1 = v0[e], x2 = v1[e];
        const float y1 = X::round(X::round(x1 * c) - X::round(x2 * s));
        const float y2 = X::round(X::round(x1 * s) + X::round(x2 * c));
        v0[e] = y1;
        v1[e] = y2;
      }
    }
    store_elems<X, V>(yp, yb + c0 * V, v0);
    store_elems<X, V>(yp, yb + c1 * V, v1);
  }
}

// Fallback for any head_dim / dims / alignment: one wave per (token, head).
template <class X, bool NORM>
__global__ __launch_bounds__(256) void rope_generic_kernel(RopeArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= (int64_t)a.tokens * a.hsum) return;  // whole wave leaves together
  const uint32_t tok = (uint32_t)(row / a.hsum);
  const int h = (int)(row - (int64_t)tok * a.hsum);
  const bool isk = h >= a.t[0].heads;
  const RopeTensor& T = a.t[isk ? 1 : 0];
  const int hh = isk ? h - a.t[0].heads : h;
  const uint32_t b = tok / a.L, l = tok - b * a.L;
  const int64_t xb = (int64_t)b * T.xs0 + (int64_t)l * T.xs1 + (int64_t)hh * T.xs2;
  const int64_t yb = (int64_t)b * T.ys0 + (int64_t)l * T.ys1 + (int64_t)hh * T.ys2;
  float r = 1.0f;
  const bool do_norm = NORM && T.nw != nullptr;
  if (do_norm) {
    double ss = 0.0;
    for (int d = lane; d < a.D; d += 64) {
      const double v = (double)load1<X>(T.x, xb + d);
      ss = __builtin_fma(v, v, ss);
    }
    ss = group_sum<64>(ss);
    r = rms_scale(ss, a.inv_d, a.eps);
  }
  auto val = [&](int d) {
    float v = load1<X>(T.x, xb + d);
    if (do_norm) v = X::round(X::round(v * r) * load1<X>(T.nw, d));
    return v;
  };
  const int32_t off = a.offsets ? a.offsets[b] : a.offset;
  const float pos = ((float)l + (float)off) * a.scale;
  // Each element is read before any lane overwrites it, so y may alias x.
  for (int base = 0; base < a.D; base += 64) {
    const int d = base + lane;
    float o1 = 0.0f, o2 = 0.0f;
    const bool act = d < a.D;
    if (act) {
      if (d < a.half) {
        const float th = pos * a.inv_freq[d];
        double s, c;
        sincos((double)th, &s, &c);
        const float cf = X::round((float)c), sf = X::round((float)s);
        const float x1 = val(d), x2 = val(d + a.half);
        o1 = X::round(X::round(x1 * cf) - X::round(x2 * sf));
        o2 = X::round(X::round(x1 * sf) + X::round(x2 * cf));
      } else if (d >= a.dims) {
        o1 = val(d);
      }
    }
    if (act && d < a.half) {
      store1<X>(T.y, yb + d, o1);
      store1<X>(T.y, yb + d + a.half, o2);
    } else if (act && d >= a.dims) {
      store1<X>(T.y, yb + d, o1);
    }
  }
}

namespace {

int gcd_i(int a, int b) { while (b) { int t = a % b; a = b; b = t; } return a; }

template <class X, int LPR, bool NORM>
void launch_fast(RopeArgs& a, hipStream_t s) {
  const int slots = 256 / LPR;
  int tpb = slots / gcd_i(slots, a.hsum);  // lcm(slots, hsum) / hsum
  tpb = std::max(1, std::min(tpb, kMaxTpb));
  while (tpb > 1 && (a.tokens + tpb - 1) / tpb < 1024u) tpb = (tpb + 1) / 2;
  a.tpb = tpb;
  const unsigned blocks = (a.tokens + tpb - 1) / tpb;
  const size_t shmem = 2u * tpb * a.half * sizeof(float);
  hipLaunchKernelGGL((rope_kernel<X, LPR, NORM>), dim3(blocks), dim3(256), shmem, s, a);
}

template <class X, bool NORM>
void launch_x(RopeArgs& a, bool vec_ok, hipStream_t s) {
  constexpr int V = Vec<X>::N;
  const bool shape_ok = a.D % (2 * V) == 0 && a.dims % (2 * V) == 0;
  const int lpr = a.D / (2 * V);
  if (vec_ok && shape_ok) {
    a.R = a.dims / (2 * V);
    switch (lpr) {
      case 2: launch_fast<X, 2, NORM>(a, s); return;
      case 4: launch_fast<X, 4, NORM>(a, s); return;
      case 8: launch_fast<X, 8, NORM>(a, s); return;
      case 16: launch_fast<X, 16, NORM>(a, s); return;
      case 32: launch_fast<X, 32, NORM>(a, s); return;
      default: break;
    }
  }
  const int64_t rows = (int64_t)a.tokens * a.hsum;
  const int wpb = 4;
  hipLaunchKernelGGL((rope_generic_kernel<X, NORM>), dim3((unsigned)((rows + wpb - 1) / wpb)),
                     dim3(64 * wpb), 0, s, a);
}

bool tensor_aligned(const void* x, const int64_t* st, int V) {
  return aligned16(x) && st[0] % V == 0 && st[1] % V == 0 && st[2] % V == 0;
}

int check_strides(const char* fn, const char* nm, const void* p, const int64_t* st) {
  if (!p) return fail(HGK_ERR_ARG, "%s: null %s", fn, nm);
  if (!st) return fail(HGK_ERR_ARG, "%s: null strides for %s", fn, nm);
  if (st[0] < 0 || st[1] < 0 || st[2] < 0)
    return fail(HGK_ERR_ARG, "%s: negative stride for %s", fn, nm);
  return HGK_OK;
}

int run(const char* fn, int dtype, const void* q, const int64_t* qs, void* qo, const int64_t* qos,
        int64_t qh, const void* qw, const void* k, const int64_t* ks, void* ko,
        const int64_t* kos, int64_t kh, const void* kw, int wdt, float eps, int64_t B,
        int64_t L, int64_t D, int dims, int traditional, float base, float scale,
        const float* freqs, int32_t offset, const int32_t* offsets, hipStream_t s) {
  if (!is_float_dtype(dtype)) return fail(HGK_ERR_ARG, "%s: dtype %d is not a float type", fn, dtype);
  if (traditional) return fail(HGK_ERR_UNSUPPORTED, "%s: traditional (interleaved) RoPE is not implemented", fn);
  if (B < 0 || L < 0 || D <= 0 || qh < 0 || kh < 0)
    return fail(HGK_ERR_ARG, "%s: bad shape B=%lld L=%lld D=%lld", fn, (long long)B, (long long)L, (long long)D);
  if (dims <= 0 || dims > D || (dims & 1))
    return fail(HGK_ERR_ARG, "%s: dims=%d must be even and in (0, head_dim=%lld]", fn, dims, (long long)D);
  if (dims / 2 > kMaxHalf) return fail(HGK_ERR_UNSUPPORTED, "%s: dims=%d > %d", fn, dims, 2 * kMaxHalf);
  if (B * L > 0x7fffffffLL || qh + kh > 0x7fffffffLL || D > (1 << 20))
    return fail(HGK_ERR_UNSUPPORTED, "%s: problem too large", fn);
  if ((qw || kw) && wdt != dtype)
    return fail(HGK_ERR_UNSUPPORTED, "%s: norm weight dtype %s must equal the activation dtype %s",
                fn, dtype_name(wdt), dtype_name(dtype));
  if (!(eps >= 0.0f)) return fail(HGK_ERR_ARG, "%s: eps must be >= 0", fn);
  int st;
  if (qh > 0) {
    if ((st = check_strides(fn, "q", q, qs)) || (st = check_strides(fn, "q_out", qo, qos))) return st;
  }
  if (kh > 0) {
    if ((st = check_strides(fn, "k", k, ks)) || (st = check_strides(fn, "k_out", ko, kos))) return st;
  }
  RopeArgs a{};
  a.half = dims / 2;
  if (freqs) {
    for (int i = 0; i < a.half; ++i) {
      if (!(freqs[i] > 0.0f)) return fail(HGK_ERR_ARG, "%s: freqs[%d] must be > 0", fn, i);
      a.inv_freq[i] = 1.0f / freqs[i];
    }
  } else {
    if ((st = hgk_rope_inv_freq(base, dims, nullptr, a.inv_freq))) return st;
  }
  if (B == 0 || L == 0 || qh + kh == 0) return HGK_OK;
  a.t[0] = RopeTensor{q, qo, qh ? qs[0] : 0, qh ? qs[1] : 0, qh ? qs[2] : 0,
                      qh ? qos[0] : 0, qh ? qos[1] : 0, qh ? qos[2] : 0, qw, (int)qh};
  a.t[1] = RopeTensor{k, ko, kh ? ks[0] : 0, kh ? ks[1] : 0, kh ? ks[2] : 0,
                      kh ? kos[0] : 0, kh ? kos[1] : 0, kh ? kos[2] : 0, kw, (int)kh};
  a.offsets = offsets;
  a.offset = offset;
  a.L = (uint32_t)L;
  a.tokens = (uint32_t)(B * L);
  a.D = (int)D;
  a.dims = dims;
  a.hsum = (int)(qh + kh);
  a.scale = scale;
  a.eps = eps;
  a.inv_d = (float)(1.0 / (double)D);
  const int V = 16 / dtype_bytes(dtype);
  bool vec_ok = true;
  if (qh) vec_ok = vec_ok && tensor_aligned(q, qs, V) && tensor_aligned(qo, qos, V) && (!qw || aligned16(qw));
  if (kh) vec_ok = vec_ok && tensor_aligned(k, ks, V) && tensor_aligned(ko, kos, V) && (!kw || aligned16(kw));
  const bool norm = (qw && qh) || (kw && kh);
  if (!qh) a.t[0].nw = nullptr;
  if (!kh) a.t[1].nw = nullptr;
  switch (dtype) {
    case DT_BF16: norm ? launch_x<BF16, true>(a, vec_ok, s) : launch_x<BF16, false>(a, vec_ok, s); break;
    case DT_F16: norm ? launch_x<F16, true>(a, vec_ok, s) : launch_x<F16, false>(a, vec_ok, s); break;
    default: norm ? launch_x<F32, true>(a, vec_ok, s) : launch_x<F32, false>(a, vec_ok, s); break;
  }
  return launch_status(fn);
}

}  // namespace
}  // namespace hgk

using namespace hgk;

extern "C" int hgk_rope(int dtype, const void* x, const int64_t x_strides[3], void* y,
                        const int64_t y_strides[3], int64_t batch, int64_t seq_len, int64_t heads,
                        int64_t head_dim, int dims, int traditional, float base, float scale,
                        const float* freqs, int32_t offset, const int32_t* offsets, void* stream) {
  clear_error();
  return run("hgk_rope", dtype, x, x_strides, y, y_strides, heads, nullptr, nullptr, nullptr,
             nullptr, nullptr, 0, nullptr, dtype, 0.0f, batch, seq_len, head_dim, dims,
             traditional, base, scale, freqs, offset, offsets, as_stream(stream));
}

extern "C" int hgk_qk_norm_rope(int dtype, const void* q, const int64_t q_strides[3], void* q_out,
                                const int64_t q_out_strides[3], int64_t q_heads,
                                const void* q_norm_w, const void* k, const int64_t k_strides[3],
                                void* k_out, const int64_t k_out_strides[3], int64_t k_heads,
                                const void* k_norm_w, int norm_w_dtype, float eps, int64_t batch,
                                int64_t seq_len, int64_t head_dim, int dims, float base,
                                float scale, const float* freqs, int32_t offset,
                                const int32_t* offsets, void* stream) {
  clear_error();
  return run("hgk_qk_norm_rope", dtype, q, q_strides, q_out, q_out_strides, q_heads, q_norm_w,
             k, k_strides, k_out, k_out_strides, k ? k_heads : 0, k_norm_w, norm_w_dtype, eps,
             batch, seq_len, head_dim, dims, 0, base, scale, freqs, offset, offsets,
             as_stream(stream));
}
