// norm.hip -- RMSNorm, Gemma (1+w) RMSNorm, per-head q/k RMSNorm, the
// Qwen3-Next gated RMSNorm and the fused residual add + RMSNorm on gfx950.
//
// Layout: rows of n contiguous elements, arbitrary row stride. A group of LPR
// lanes owns one row (LPR = 64 for hidden-size rows, fewer for head_dim rows,
// so a wave64 covers 64/LPR rows); each lane holds CPL units of its row in
// registers, strided by LPR so the wave's loads are fully coalesced. A unit is
// 16 bytes of x, or 8 bytes when the output is wider than x (f32 out of a
// 16-bit x), so that each unit's output is exactly one 16-byte store.
// The f32 sum of squares is reduced across the group with xor shuffles, then
// the same registers are scaled and written: x crosses HBM once, y once.
//
// Arithmetic follows MLX's CPU composition (fast::rms_norm fallback):
//   r = 1 / sqrt(f32(sum(x*x)) * f32(1/n) + eps)   (sum accumulated in f64)
//   n = round_T(x * r);  y = round_T(n * w')        (T = promote(x, w'))
// and, gated, out = round_T(round_T(z * round_T(sigmoid(z))) * y), the
// rounded sigmoid taken from the hardware exp2 / reciprocal form wherever it
// provably rounds like MLX's exact one (sigmoid2_rounded).
// The residual form first forms h = round_X(x + r) (MLX's add), writes h and
// normalises it: the block boundary `h = x.add(residual); norm(h)` of
// transformer.rs:413-415 in one pass.
#include "../../include/higgs_hip.h"
#include "hgk_act.h"
#include "hgk_common.h"
#include "hgk_host.h"

namespace hgk {

enum NormMode { kPlain = 0, kGated = 1, kResid = 2 };

struct NormArgs {
  const void* x;
  int64_t xs;
  const void* z;  // gated: z; residual: r. Row r at (r / zg) * zgs + (r % zg) * zs
  int64_t zs;
  int64_t zg;
  int64_t zgs;
  const void* w;  // may be null
  int wdt;
  int plus_one;
  int round_x;  // computation type is the activation type (else f32)
  float eps;
  float inv_n;
  void* y;
  int64_t ys;
  void* h;  // residual form: h = x + r (may be null)
  int64_t hs;
  int64_t rows;
  int n;
};

__device__ inline int64_t z_row_offset(const NormArgs& a, int64_t r) {
  const int64_t g = r / a.zg;
  return g * a.zgs + (r - g * a.zg) * a.zs;
}

// X activation, Y output, W weight storage type (X's type or f32). A lane's
// unit is UB bytes of x (16, or 8 when Y is wider than X, so that a unit's
// output is one 16-byte store and every store instruction of the wave covers
// a contiguous span). Every load of the row (x, weights, z) is issued before
// the reduction; all stay packed in registers until the element is consumed.
template <class X, class Y, class W, int LPR, int CPL, int MODE, int UB>
__global__ __launch_bounds__(256) void rms_norm_kernel(NormArgs a) {
  constexpr bool GATED = MODE == kGated, RESID = MODE == kResid, TWO = GATED || RESID;
  constexpr int UE = UB / X::kBytes;     // elements per unit
  constexpr int UW = UB / 4;             // 32-bit words of x per unit
  constexpr int WW = UE * W::kBytes / 4;  // 32-bit words of weights per unit
  typedef typename RawVec<UB>::type XR;
  constexpr int RPW = 64 / LPR;
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t row = wave * RPW + lane / LPR;
  const int j = lane % LPR;
  const bool live = row < a.rows;
  const int64_t r = live ? row : a.rows - 1;
  const int nchunks = a.n / UE;
  const bool has_w = a.w != nullptr;

  // Loads are unconditional: unit indices past the row are clamped to its
  // last unit (then ignored), so no select waits on a loaded value before
  // the next load can issue. x and z are read once, non-temporally: the
  // residual add + RMSNorm at 16384 x 4096 took 90.6 us against 94.0 with
  // the default policy, at 4096 x 2048 13.8 against 15.1, the plain norm
  // at 16384 x 4096 46.6 against 47.5.
  XR xr[CPL];
  uint32_t wr[CPL][WW];
  XR zr[TWO ? CPL : 1];
  const int64_t zoff = TWO ? z_row_offset(a, r) : 0;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = j + c * LPR;
    const int chc = ch < nchunks ? ch : nchunks - 1;
    xr[c] = ld_raw_nt<UB>(a.x, (r * a.xs + (int64_t)chc * UE) * X::kBytes);
    if constexpr (TWO) zr[c] = ld_raw_nt<UB>(a.z, (zoff + (int64_t)chc * UE) * X::kBytes);
  }
  if (has_w) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int ch = j + c * LPR;
      const int chc = ch < nchunks ? ch : nchunks - 1;
      const int64_t wb = (int64_t)chc * UE * W::kBytes;
      if constexpr (WW == 2) {
        const u32x2 t = ld_raw<8>(a.w, wb);
        wr[c][0] = t[0];
        wr[c][1] = t[1];
      } else {
#pragma unroll
        for (int q = 0; q < WW / 4; ++q) {
          const u32x4 t = ld_raw<16>(a.w, wb + 16 * q);
#pragma unroll
          for (int k = 0; k < 4; ++k) wr[c][4 * q + k] = t[k];
        }
      }
    }
  }
  if constexpr (RESID) {
    // h = round_X(x + r), one packed conversion per pair; h replaces x
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
#pragma unroll
      for (int k = 0; k < UW; ++k) {
        if constexpr (X::kBytes == 2) {
          xr[c][k] = X::pack(X::lo(xr[c][k]) + X::lo(zr[c][k]), X::hi(xr[c][k]) + X::hi(zr[c][k]));
        } else {
          xr[c][k] = f2u(u2f(xr[c][k]) + u2f(zr[c][k]));
        }
      }
      const int ch = j + c * LPR;
      if (a.h && live && ch < nchunks)
        st_raw_nt<UB>(a.h, (r * a.hs + (int64_t)ch * UE) * X::kBytes, xr[c]);
    }
  }
  double ss = 0.0;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    if (j + c * LPR >= nchunks) continue;
#pragma unroll
    for (int e = 0; e < UE; ++e) {
      const double d = (double)elem<X>(xr[c], e);
      ss = __builtin_fma(d, d, ss);
    }
  }
  ss = group_sum<LPR>(ss);
  const float rr = rms_scale(ss, a.inv_n, a.eps);

  // Roundings to X go in pairs (one packed conversion for two values). The
  // last rounding of each output is the store's own conversion when Y is X.
  const bool rx = a.round_x != 0;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = j + c * LPR;
    if (ch >= nchunks) continue;
    float o[UE];
#pragma unroll
    for (int e = 0; e < UE; e += 2) {
      float n0 = elem<X>(xr[c], e) * rr, n1 = elem<X>(xr[c], e + 1) * rr;
      if (rx) round2<X>(n0, n1);
      float w0 = has_w ? elem<W>(wr[c], e) : 1.0f, w1 = has_w ? elem<W>(wr[c], e + 1) : 1.0f;
      if (a.plus_one) {
        w0 = w0 + 1.0f;
        w1 = w1 + 1.0f;
      }
      n0 = n0 * w0;
      n1 = n1 * w1;
      if constexpr (GATED) {
        if (rx) round2<X>(n0, n1);
        const float z0 = elem<X>(zr[c], e), z1 = elem<X>(zr[c], e + 1);
        float s0, s1;
        sigmoid2_rounded<X>(z0, z1, s0, s1);
        float g0 = z0 * s0, g1 = z1 * s1;
        round2<X>(g0, g1);
        n0 = g0 * n0;
        n1 = g1 * n1;
      }
      if constexpr (Y::kCode != X::kCode) {
        if (rx) round2<X>(n0, n1);
      }
      o[e] = n0;
      o[e + 1] = n1;
    }
    if (live) store_elems<Y, UE>(a.y, r * a.ys + (int64_t)ch * UE, o);
  }
}

// Any n, any alignment: one wave per row, element-strided, two passes over x.
template <class X, class Y, int MODE>
__global__ __launch_bounds__(256) void rms_norm_generic_kernel(NormArgs a) {
  constexpr bool GATED = MODE == kGated, RESID = MODE == kResid;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (row >= a.rows) return;  // whole wave leaves together
  // the row's input value: x, or round_X(x + r) in the residual form
  auto in = [&](int i) {
    const float xv = load1<X>(a.x, row * a.xs + i);
    if constexpr (RESID) return X::round(xv + load1<X>(a.z, z_row_offset(a, row) + i));
    else return xv;
  };
  double ss = 0.0;
  for (int i = lane; i < a.n; i += 64) {
    const double xv = (double)in(i);
    ss = __builtin_fma(xv, xv, ss);
  }
  ss = group_sum<64>(ss);
  const float rr = rms_scale(ss, a.inv_n, a.eps);
  for (int i = lane; i < a.n; i += 64) {
    const float hv = in(i);
    if constexpr (RESID) {
      if (a.h) store1<X>(a.h, row * a.hs + i, hv);
    }
    float nv = hv * rr;
    nv = a.round_x ? X::round(nv) : nv;
    float we = a.w ? load1_dt(a.w, a.wdt, i) : 1.0f;
    we = a.plus_one ? we + 1.0f : we;
    nv = nv * we;
    nv = a.round_x ? X::round(nv) : nv;
    if constexpr (GATED) {
      const float zz = load1<X>(a.z, z_row_offset(a, row) + i);
      const float sg = X::round(mlx_sigmoid(zz));
      const float act = X::round(zz * sg);
      nv = act * nv;
      nv = a.round_x ? X::round(nv) : nv;
    }
    store1<Y>(a.y, row * a.ys + i, nv);
  }
}

namespace {

// Unit bytes of x per lane: 8 when Y is wider than X (so a unit's output is
// one 16-byte store), else 16.
template <class X, class Y>
constexpr int unit_bytes() { return Y::kBytes > X::kBytes ? 8 : 16; }

template <class X, class Y, class W, int LPR, int CPL, int MODE, int UB = unit_bytes<X, Y>()>
void launch_fast(const NormArgs& a, hipStream_t s) {
  constexpr int RPW = 64 / LPR;
  const int64_t waves = (a.rows + RPW - 1) / RPW;
  // small problems: one wave per block, spread over CUs. Large ones: 2 waves
  // per block for the plain norm (against 4, in two probe calls: Llama-3.2-1B
  // 4096 x 2048 7.44 -> 7.22 and 7.25 -> 7.20 us, Qwen3-8B 16384 x 4096
  // 47.02 -> 46.33 and 46.13 -> 45.70, the Gemma-2 (1+w) norm unchanged),
  // 4 for the residual add + RMSNorm (14.18 with 2 against 13.90 at
  // 4096 x 2048).
  const int wpb = waves < 4096 ? 1 : MODE == kPlain ? 2 : 4;
  const int64_t blocks = (waves + wpb - 1) / wpb;
  HGK_LAUNCH((rms_norm_kernel<X, Y, W, LPR, CPL, MODE, UB>),
             dim3((unsigned)blocks), dim3(64 * wpb), 0, s, a);
}

template <class X, class Y, int MODE>
void launch_generic(const NormArgs& a, hipStream_t s) {
  const int wpb = a.rows >= 4096 ? 4 : 1;
  const int64_t blocks = (a.rows + wpb - 1) / wpb;
  HGK_LAUNCH((rms_norm_generic_kernel<X, Y, MODE>), dim3((unsigned)blocks),
             dim3(64 * wpb), 0, s, a);
}

// Pick (LPR, CPL) for a row of `nchunks` units; false -> generic.
// The gated form (head_dim rows) stops at 128 units.
template <class X, class Y, class W, int MODE>
bool launch_by_shape(const NormArgs& a, int nchunks, hipStream_t s) {
  if (nchunks <= 4) { launch_fast<X, Y, W, 4, 1, MODE>(a, s); return true; }
  if (nchunks <= 8) { launch_fast<X, Y, W, 8, 1, MODE>(a, s); return true; }
  if (nchunks <= 16) { launch_fast<X, Y, W, 16, 1, MODE>(a, s); return true; }
  if (nchunks <= 32) { launch_fast<X, Y, W, 32, 1, MODE>(a, s); return true; }
  if (nchunks <= 64) { launch_fast<X, Y, W, 64, 1, MODE>(a, s); return true; }
  if (nchunks <= 128) { launch_fast<X, Y, W, 64, 2, MODE>(a, s); return true; }
  if constexpr (MODE != kGated) {
    const int cpl = (nchunks + 63) / 64;
    switch (cpl) {
      case 3: launch_fast<X, Y, W, 64, 3, MODE>(a, s); return true;
      case 4: launch_fast<X, Y, W, 64, 4, MODE>(a, s); return true;
      case 5: launch_fast<X, Y, W, 64, 5, MODE>(a, s); return true;
      case 6: launch_fast<X, Y, W, 64, 6, MODE>(a, s); return true;
      case 7: launch_fast<X, Y, W, 64, 7, MODE>(a, s); return true;
      case 8: launch_fast<X, Y, W, 64, 8, MODE>(a, s); return true;
      case 9: case 10: launch_fast<X, Y, W, 64, 10, MODE>(a, s); return true;
      case 11: case 12: launch_fast<X, Y, W, 64, 12, MODE>(a, s); return true;
      case 13: case 14: launch_fast<X, Y, W, 64, 14, MODE>(a, s); return true;
      case 15: case 16: launch_fast<X, Y, W, 64, 16, MODE>(a, s); return true;
      default: break;
    }
  }
  return false;
}

// The vectorised kernels take weights in the activation type or in f32;
// any other weight dtype goes to the generic kernel.
// Rows too long for 8-byte units (more than 16 per lane: a 16-bit x with an
// f32 output and n > 4096, e.g. hidden 4608 or 5376) take 16-byte units
// instead, up to 16 per lane (n <= 8192 for a 16-bit x): each unit's output is
// then two 16-byte stores rather than one.
template <class X, class Y, class W, int MODE>
bool launch_wide_units(const NormArgs& a, hipStream_t s) {
  if constexpr (MODE == kGated || unit_bytes<X, Y>() == 16) {
    return false;
  } else {
    const int cpl = (a.n / (16 / X::kBytes) + 63) / 64;
    switch (cpl) {
      case 9: case 10: launch_fast<X, Y, W, 64, 10, MODE, 16>(a, s); return true;
      case 11: case 12: launch_fast<X, Y, W, 64, 12, MODE, 16>(a, s); return true;
      case 13: case 14: launch_fast<X, Y, W, 64, 14, MODE, 16>(a, s); return true;
      case 15: case 16: launch_fast<X, Y, W, 64, 16, MODE, 16>(a, s); return true;
      default: return false;
    }
  }
}

template <class X, class Y, int MODE>
void launch_xy(const NormArgs& a, bool vec_ok, hipStream_t s) {
  const int nchunks = a.n / (unit_bytes<X, Y>() / X::kBytes);
  if (vec_ok) {
    if (!a.w || a.wdt == X::kCode) {
      if (launch_by_shape<X, Y, X, MODE>(a, nchunks, s)) return;
      if (a.n % (16 / X::kBytes) == 0 && launch_wide_units<X, Y, X, MODE>(a, s)) return;
    } else if (a.wdt == DT_F32) {
      if (launch_by_shape<X, Y, F32, MODE>(a, nchunks, s)) return;
      if (a.n % (16 / X::kBytes) == 0 && launch_wide_units<X, Y, F32, MODE>(a, s)) return;
    }
  }
  launch_generic<X, Y, MODE>(a, s);
}

constexpr const char* mode_fn(int mode) {
  return mode == kGated ? "hgk_gated_rms_norm" : (mode == kResid ? "hgk_add_rms_norm" : "hgk_rms_norm");
}

template <int MODE>
int dispatch(const NormArgs& a, int xdt, int ydt, bool vec_ok, hipStream_t s) {
  if (xdt == DT_BF16 && ydt == DT_BF16) launch_xy<BF16, BF16, MODE>(a, vec_ok, s);
  else if (xdt == DT_BF16 && ydt == DT_F32) launch_xy<BF16, F32, MODE>(a, vec_ok, s);
  else if (xdt == DT_F16 && ydt == DT_F16) launch_xy<F16, F16, MODE>(a, vec_ok, s);
  else if (xdt == DT_F16 && ydt == DT_F32) launch_xy<F16, F32, MODE>(a, vec_ok, s);
  else if (xdt == DT_F32 && ydt == DT_F32) launch_xy<F32, F32, MODE>(a, vec_ok, s);
  else
    return fail(HGK_ERR_UNSUPPORTED, "%s: output dtype %s for input %s is not implemented "
                "(output must be the input dtype or f32)",
                mode_fn(MODE), dtype_name(ydt), dtype_name(xdt));
  return launch_status(mode_fn(MODE));
}

int check_common(const char* fn, const void* x, int xdt, int64_t xs, const void* w, int wdt,
                 void* y, int ydt, int64_t ys, int64_t rows, int64_t n, float eps) {
  if (rows < 0 || n < 0) return fail(HGK_ERR_ARG, "%s: negative shape rows=%lld n=%lld", fn,
                                     (long long)rows, (long long)n);
  if (n > (int64_t)1 << 30) return fail(HGK_ERR_UNSUPPORTED, "%s: n=%lld too large", fn, (long long)n);
  // an empty call (no rows or columns) may pass null data pointers
  if ((!x || !y) && rows > 0 && n > 0) return fail(HGK_ERR_ARG, "%s: null x or y", fn);
  if (!is_float_dtype(xdt) || !is_float_dtype(ydt))
    return fail(HGK_ERR_ARG, "%s: x/y dtype must be f32, bf16 or f16 (got %d, %d)", fn, xdt, ydt);
  if (w && !is_float_dtype(wdt)) return fail(HGK_ERR_ARG, "%s: bad weight dtype %d", fn, wdt);
  if (rows > 1 && (xs < n || ys < n))
    return fail(HGK_ERR_ARG, "%s: row strides (%lld, %lld) smaller than n=%lld", fn,
                (long long)xs, (long long)ys, (long long)n);
  if (!(eps >= 0.0f)) return fail(HGK_ERR_ARG, "%s: eps must be >= 0", fn);
  return HGK_OK;
}

}  // namespace
}  // namespace hgk

using namespace hgk;

extern "C" int hgk_rms_norm(const void* x, int x_dtype, int64_t x_row_stride, const void* w,
                            int w_dtype, int w_plus_one, float eps, void* y, int y_dtype,
                            int64_t y_row_stride, int64_t rows, int64_t n, void* stream) {
  clear_error();
  int st = check_common("hgk_rms_norm", x, x_dtype, x_row_stride, w, w_dtype, y, y_dtype,
                        y_row_stride, rows, n, eps);
  if (st) return st;
  if (w_plus_one && !w) return fail(HGK_ERR_ARG, "hgk_rms_norm: w_plus_one needs a weight");
  if (rows == 0 || n == 0) return HGK_OK;
  const int w_eff = w ? (w_plus_one ? DT_F32 : w_dtype) : x_dtype;
  const int t_out = promote(x_dtype, w_eff);
  if (t_out != x_dtype && t_out != DT_F32)
    return fail(HGK_ERR_UNSUPPORTED, "hgk_rms_norm: computation type %s not implemented",
                dtype_name(t_out));
  NormArgs a{};
  a.x = x; a.xs = x_row_stride; a.w = w; a.wdt = w_dtype; a.plus_one = w_plus_one ? 1 : 0;
  a.round_x = (t_out == x_dtype) ? 1 : 0;
  a.eps = eps; a.inv_n = (float)(1.0 / (double)n);
  a.y = y; a.ys = y_row_stride; a.rows = rows; a.n = (int)n;
  a.zg = 1;
  const int vx = 16 / dtype_bytes(x_dtype);
  const bool vec_ok = aligned16(x) && aligned16(y) && (!w || aligned16(w)) && n % vx == 0 &&
                      x_row_stride % vx == 0 && (y_row_stride * dtype_bytes(y_dtype)) % 16 == 0 &&
                      (n * dtype_bytes(y_dtype)) % 16 == 0;
  return dispatch<kPlain>(a, x_dtype, y_dtype, vec_ok, as_stream(stream));
}

extern "C" int hgk_gated_rms_norm(int dtype, const void* x, int64_t x_row_stride, const void* z,
                                  int64_t z_row_stride, int64_t z_group_rows,
                                  int64_t z_group_stride, const void* w, int w_dtype, float eps,
                                  void* out, int out_dtype, int64_t out_row_stride, int64_t rows,
                                  int64_t n, void* stream) {
  clear_error();
  int st = check_common("hgk_gated_rms_norm", x, dtype, x_row_stride, w, w_dtype, out,
                        out_dtype, out_row_stride, rows, n, eps);
  if (st) return st;
  if (!w || (!z && rows > 0 && n > 0)) return fail(HGK_ERR_ARG, "hgk_gated_rms_norm: null z or weight");
  if (z_group_rows <= 0 || z_group_rows > rows) {
    z_group_rows = rows > 0 ? rows : 1;
    z_group_stride = 0;
  }
  if ((z_group_rows > 1 && z_row_stride < n) || z_row_stride < 0 ||
      (rows > z_group_rows && z_group_stride < (z_group_rows - 1) * z_row_stride + n))
    return fail(HGK_ERR_ARG, "hgk_gated_rms_norm: z rows overlap (row stride %lld, group %lld x %lld)",
                (long long)z_row_stride, (long long)z_group_rows, (long long)z_group_stride);
  if (rows == 0 || n == 0) return HGK_OK;
  const int t_n = promote(dtype, w_dtype);
  NormArgs a{};
  a.x = x; a.xs = x_row_stride; a.z = z; a.zs = z_row_stride; a.zg = z_group_rows;
  a.zgs = z_group_stride; a.w = w; a.wdt = w_dtype;
  a.plus_one = 0; a.round_x = (t_n == dtype) ? 1 : 0;
  a.eps = eps; a.inv_n = (float)(1.0 / (double)n);
  a.y = out; a.ys = out_row_stride; a.rows = rows; a.n = (int)n;
  const int vx = 16 / dtype_bytes(dtype);
  const bool vec_ok = aligned16(x) && aligned16(z) && aligned16(out) && aligned16(w) &&
                      n % vx == 0 && x_row_stride % vx == 0 && z_row_stride % vx == 0 &&
                      z_group_stride % vx == 0 &&
                      (out_row_stride * dtype_bytes(out_dtype)) % 16 == 0 &&
                      (n * dtype_bytes(out_dtype)) % 16 == 0;
  return dispatch<kGated>(a, dtype, out_dtype, vec_ok, as_stream(stream));
}

extern "C" int hgk_add_rms_norm(int dtype, const void* x, int64_t x_row_stride, const void* r,
                                int64_t r_row_stride, const void* w, int w_dtype, int w_plus_one,
                                float eps, void* h, int64_t h_row_stride, void* y, int y_dtype,
                                int64_t y_row_stride, int64_t rows, int64_t n, void* stream) {
  clear_error();
  const char* fn = "hgk_add_rms_norm";
  int st = check_common(fn, x, dtype, x_row_stride, w, w_dtype, y, y_dtype, y_row_stride, rows,
                        n, eps);
  if (st) return st;
  if (!r && rows > 0 && n > 0) return fail(HGK_ERR_ARG, "%s: null residual r", fn);
  if (w_plus_one && !w) return fail(HGK_ERR_ARG, "%s: w_plus_one needs a weight", fn);
  if (rows > 1 && (r_row_stride < n || (h && h_row_stride < n)))
    return fail(HGK_ERR_ARG, "%s: r/h row strides (%lld, %lld) smaller than n=%lld", fn,
                (long long)r_row_stride, (long long)h_row_stride, (long long)n);
  if (rows == 0 || n == 0) return HGK_OK;
  const int w_eff = w ? (w_plus_one ? DT_F32 : w_dtype) : dtype;
  const int t_out = promote(dtype, w_eff);
  if (t_out != dtype && t_out != DT_F32)
    return fail(HGK_ERR_UNSUPPORTED, "%s: computation type %s not implemented", fn,
                dtype_name(t_out));
  NormArgs a{};
  // r's rows as groups of one row: row i at i * r_row_stride
  a.x = x; a.xs = x_row_stride; a.z = r; a.zs = r_row_stride; a.zg = 1; a.zgs = r_row_stride;
  a.w = w; a.wdt = w_dtype; a.plus_one = w_plus_one ? 1 : 0;
  a.round_x = (t_out == dtype) ? 1 : 0;
  a.eps = eps; a.inv_n = (float)(1.0 / (double)n);
  a.y = y; a.ys = y_row_stride; a.h = h; a.hs = h_row_stride; a.rows = rows; a.n = (int)n;
  const int vx = 16 / dtype_bytes(dtype);
  const bool vec_ok = aligned16(x) && aligned16(r) && aligned16(y) && (!h || aligned16(h)) &&
                      (!w || aligned16(w)) && n % vx == 0 && x_row_stride % vx == 0 &&
                      r_row_stride % vx == 0 && (!h || h_row_stride % vx == 0) &&
                      (y_row_stride * dtype_bytes(y_dtype)) % 16 == 0 &&
                      (n * dtype_bytes(y_dtype)) % 16 == 0;
  return dispatch<kResid>(a, dtype, y_dtype, vec_ok, as_stream(stream));
}
