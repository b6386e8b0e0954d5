// glu.hip -- SwiGLU (silu(gate) * up) and GeGLU (gelu_tanh(gate) * up) on
// gfx950.
//
// A pure stream: every element of gate and up is read once and every output
// written once. Each thread owns U 16-byte chunks spaced one block-width apart
// (so every load instruction of the block covers a contiguous 4 KB), issues all
// 2U loads before any arithmetic, and writes with non-temporal stores.
//
// SwiGLU arithmetic is MLX's CPU composition, bit for bit:
//   sig = round_T(sigmoid(g)); s = round_T(g * sig); out = round_T(s * u)
// with MLX's sigmoid (y = 1/(1+exp(|g|)); g < 0 ? y : 1-y) and MLX's
// polynomial exp, built from IEEE operations only. That exact sigmoid costs
// ~40 VALU operations per element and would make the kernel compute-bound, so
// for 16-bit inputs the kernel first evaluates the same formula with the
// hardware exp2 and reciprocal, and keeps it only when the result cannot round
// differently: |g| <= 64 (there the fast value is within 3 f32 ulps of the
// exact one, measured over every 16-bit input) and the value is more than
// kTieWindow ulps from a rounding tie of T. Everything else takes the exact
// path. Since a 16-bit input has only 65536 values, the tests check the result
// for all of them.
//
// GeGLU runs in f32 (mlx-rs builds gelu_approximate from f32 scalar arrays,
// which promote a bf16 input): 0.5*g*(1+tanh(k0*(g + k1*g^3))) is evaluated as
// the identical g / (1 + exp(-2*k0*(g + k1*g^3))), using the hardware exp2 and
// reciprocal (relative error ~1e-6), and the product with up is rounded once.
#include <algorithm>

#include "../../include/higgs_hip.h"
#include "hgk_act.h"
#include "hgk_common.h"
#include "hgk_host.h"

namespace hgk {

struct GluArgs {
  const void* g;
  int64_t gs;
  const void* u;
  int64_t us;
  void* o;
  int64_t os;
  uint32_t cpr;    // 16-byte chunks per row
  uint32_t total;  // chunks overall
  int contig;      // all three tensors densely packed
};

// Element offsets of chunk q in gate, up and out (rows of cpr chunks).
template <int V, bool CONTIG>
__device__ inline void glu_offsets(const GluArgs& a, uint32_t q, int64_t& go, int64_t& uo,
                                   int64_t& oo) {
  if constexpr (CONTIG) {
    go = uo = oo = (int64_t)q * V;
  } else {
    const uint32_t row = q / a.cpr, c = q - row * a.cpr;
    go = (int64_t)row * a.gs + (int64_t)c * V;
    uo = (int64_t)row * a.us + (int64_t)c * V;
    oo = (int64_t)row * a.os + (int64_t)c * V;
  }
}

// Chunks past the end are clamped to the last chunk for the loads (so loads
// are never predicated and can all issue before the first wait) and skipped
// at the store.
template <class X, class Y, int ACT, int U, bool CONTIG>
__global__ __launch_bounds__(256) void glu_kernel(GluArgs a) {
  constexpr int V = Vec<X>::N;
  const uint32_t base = blockIdx.x * (256u * U) + threadIdx.x;
  u32x4 gr[U], ur[U];
  int64_t oo[U];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const uint32_t q = base + 256u * k;
    const uint32_t qq = q < a.total ? q : a.total - 1;
    int64_t go, uo;
    glu_offsets<V, CONTIG>(a, qq, go, uo, oo[k]);
    gr[k] = ld16_nt<X>(a.g, go);
    ur[k] = ld16_nt<X>(a.u, uo);
  }
  if constexpr (ACT == HGK_ACT_SILU && X::kBytes == 2) {
    float gv[U * V], uv[U * V], o[U * V];
#pragma unroll
    for (int k = 0; k < U; ++k)
#pragma unroll
      for (int e = 0; e < V; ++e) {
        gv[k * V + e] = elem<X>(gr[k], e);
        uv[k * V + e] = elem<X>(ur[k], e);
      }
    swiglu16<X, U * V>(gv, uv, o);
#pragma unroll
    for (int k = 0; k < U; ++k)
      if (base + 256u * k < a.total) store_elems<Y, V>(a.o, oo[k], o + k * V);
  } else {
#pragma unroll
    for (int k = 0; k < U; ++k) {
      float o[V];
#pragma unroll
      for (int e = 0; e < V; ++e) o[e] = glu1<X, ACT>(elem<X>(gr[k], e), elem<X>(ur[k], e));
      if (base + 256u * k < a.total) store_elems<Y, V>(a.o, oo[k], o);
    }
  }
}

// 16-bit inputs with an f32 output (GeGLU's promoted result): a unit is 4
// elements, read as 8 bytes of gate and of up and written as 16 bytes, so
// every load instruction of a wave covers 512 contiguous bytes and every store
// 1 KB. (With 16-byte input chunks each lane would write 32 bytes in two
// instructions, each covering every other 16 bytes of a 2 KB span.)
template <class X, class Y, int ACT, int U, bool CONTIG>
__global__ __launch_bounds__(256) void glu_wide_kernel(GluArgs a) {
  static_assert(X::kBytes == 2 && Y::kBytes == 4, "16-bit in, f32 out");
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  constexpr int V = 4;
  const uint32_t base = blockIdx.x * (256u * U) + threadIdx.x;
  u32x2 gr[U], ur[U];
  int64_t oo[U];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const uint32_t q = base + 256u * k;
    const uint32_t qq = q < a.total ? q : a.total - 1;
    int64_t go, uo;
    glu_offsets<V, CONTIG>(a, qq, go, uo, oo[k]);
    gr[k] = ld_raw_nt<8>(a.g, go * 2);
    ur[k] = ld_raw_nt<8>(a.u, uo * 2);
  }
  float gv[U * V], uv[U * V], o[U * V];
#pragma unroll
  for (int k = 0; k < U; ++k)
#pragma unroll
    for (int e = 0; e < V; e += 2) {
      gv[k * V + e] = X::lo(gr[k][e / 2]);
      gv[k * V + e + 1] = X::hi(gr[k][e / 2]);
      uv[k * V + e] = X::lo(ur[k][e / 2]);
      uv[k * V + e + 1] = X::hi(ur[k][e / 2]);
    }
  if constexpr (ACT == HGK_ACT_SILU) {
    swiglu16<X, U * V>(gv, uv, o);
  } else {
#pragma unroll
    for (int e = 0; e < U * V; ++e) o[e] = glu1<X, ACT>(gv[e], uv[e]);
  }
#pragma unroll
  for (int k = 0; k < U; ++k)
    if (base + 256u * k < a.total) store_elems<Y, V>(a.o, oo[k], o + k * V);
}

// Any alignment / width: one element per thread per pass of a grid-stride
// loop (the grid is capped, so any element count launches).
template <class X, class Y, int ACT>
__global__ __launch_bounds__(256) void glu_generic_kernel(GluArgs a, int64_t n, int64_t rows) {
  const int64_t total = n * rows;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += stride) {
    const int64_t row = i / n, c = i - row * n;
    const float g = load1<X>(a.g, row * a.gs + c), u = load1<X>(a.u, row * a.us + c);
    store1<Y>(a.o, row * a.os + c, glu1<X, ACT>(g, u));
  }
}

namespace {

template <class X, class Y, int ACT>
void launch(const GluArgs& a0, bool vec_ok, int64_t rows, int64_t n, hipStream_t s) {
  if constexpr (X::kBytes == 2 && Y::kBytes == 4) {
    if (vec_ok && n % 4 == 0 && rows * (n / 4) < ((int64_t)1 << 31)) {
      GluArgs a = a0;  // units of 4 elements
      a.cpr = (uint32_t)(n / 4);
      a.total = (uint32_t)(rows * (n / 4));
      if (a.total >= 256u * 4u * 1024u) {
        const unsigned blocks = (a.total + 1024u - 1u) / 1024u;
        if (a.contig) HGK_LAUNCH((glu_wide_kernel<X, Y, ACT, 4, true>), dim3(blocks), dim3(256), 0, s, a);
        else HGK_LAUNCH((glu_wide_kernel<X, Y, ACT, 4, false>), dim3(blocks), dim3(256), 0, s, a);
      } else {
        const unsigned blocks = (a.total + 511u) / 512u;
        if (a.contig) HGK_LAUNCH((glu_wide_kernel<X, Y, ACT, 2, true>), dim3(blocks), dim3(256), 0, s, a);
        else HGK_LAUNCH((glu_wide_kernel<X, Y, ACT, 2, false>), dim3(blocks), dim3(256), 0, s, a);
      }
      return;
    }
  }
  const GluArgs& a = a0;
  if (vec_ok) {
    // units of 8 elements per thread: 4 from 8M units (the Qwen3-8B prefill's
    // 25M: 183.7 us against 190.7 with 2), 2 below it (the Llama-3.2-1B
    // chain's 4.2M: 32.8 against 34.0 us with 4), 1 below 1M
    if (a.total >= 8u * 1024u * 1024u) {
      const unsigned blocks = (a.total + 1024u - 1u) / 1024u;
      if (a.contig) HGK_LAUNCH((glu_kernel<X, Y, ACT, 4, true>), dim3(blocks), dim3(256), 0, s, a);
      else HGK_LAUNCH((glu_kernel<X, Y, ACT, 4, false>), dim3(blocks), dim3(256), 0, s, a);
    } else if (a.total >= 256u * 4u * 1024u) {
      const unsigned blocks = (a.total + 512u - 1u) / 512u;
      if (a.contig) HGK_LAUNCH((glu_kernel<X, Y, ACT, 2, true>), dim3(blocks), dim3(256), 0, s, a);
      else HGK_LAUNCH((glu_kernel<X, Y, ACT, 2, false>), dim3(blocks), dim3(256), 0, s, a);
    } else {
      const unsigned blocks = (a.total + 255u) / 256u;
      if (a.contig) HGK_LAUNCH((glu_kernel<X, Y, ACT, 1, true>), dim3(blocks), dim3(256), 0, s, a);
      else HGK_LAUNCH((glu_kernel<X, Y, ACT, 1, false>), dim3(blocks), dim3(256), 0, s, a);
    }
    return;
  }
  const int64_t blocks = std::min<int64_t>((n * rows + 255) / 256, (int64_t)1 << 20);
  HGK_LAUNCH((glu_generic_kernel<X, Y, ACT>), dim3((unsigned)blocks), dim3(256), 0, s,
             a, n, rows);
}

template <int ACT>
int dispatch(const GluArgs& a, int xdt, int ydt, bool vec_ok, int64_t rows, int64_t n, hipStream_t s) {
  if (xdt == DT_BF16 && ydt == DT_BF16) launch<BF16, BF16, ACT>(a, vec_ok, rows, n, s);
  else if (xdt == DT_BF16 && ydt == DT_F32) launch<BF16, F32, ACT>(a, vec_ok, rows, n, s);
  else if (xdt == DT_F16 && ydt == DT_F16) launch<F16, F16, ACT>(a, vec_ok, rows, n, s);
  else if (xdt == DT_F16 && ydt == DT_F32) launch<F16, F32, ACT>(a, vec_ok, rows, n, s);
  else if (xdt == DT_F32 && ydt == DT_F32) launch<F32, F32, ACT>(a, vec_ok, rows, n, s);
  else
    return fail(HGK_ERR_UNSUPPORTED, "hgk_glu: output dtype %s for input %s is not implemented",
                dtype_name(ydt), dtype_name(xdt));
  return launch_status("hgk_glu");
}

}  // namespace
}  // namespace hgk

using namespace hgk;

extern "C" int hgk_glu(int act, int dtype, const void* gate, int64_t gate_row_stride,
                       const void* up, int64_t up_row_stride, void* out, int out_dtype,
                       int64_t out_row_stride, int64_t rows, int64_t n, void* stream) {
  clear_error();
  if (act != HGK_ACT_SILU && act != HGK_ACT_GELU_TANH)
    return fail(HGK_ERR_ARG, "hgk_glu: unknown activation %d", act);
  if (!is_float_dtype(dtype) || !is_float_dtype(out_dtype))
    return fail(HGK_ERR_ARG, "hgk_glu: dtypes must be f32, bf16 or f16");
  if (rows < 0 || n < 0) return fail(HGK_ERR_ARG, "hgk_glu: negative shape");
  if ((!gate || !up || !out) && rows > 0 && n > 0) return fail(HGK_ERR_ARG, "hgk_glu: null pointer");
  if (rows > 1 && (gate_row_stride < n || up_row_stride < n || out_row_stride < n))
    return fail(HGK_ERR_ARG, "hgk_glu: row stride smaller than n");
  if (rows == 0 || n == 0) return HGK_OK;
  const int V = 16 / dtype_bytes(dtype);
  const int64_t chunks = (n / V) * rows;
  if (chunks >= ((int64_t)1 << 31) || n * rows >= ((int64_t)1 << 40))
    return fail(HGK_ERR_UNSUPPORTED, "hgk_glu: problem too large");
  GluArgs a{};
  a.g = gate; a.gs = gate_row_stride; a.u = up; a.us = up_row_stride;
  a.o = out; a.os = out_row_stride;
  a.cpr = (uint32_t)(n / V);
  a.total = (uint32_t)chunks;
  a.contig = (rows == 1) || (gate_row_stride == n && up_row_stride == n && out_row_stride == n);
  const int ob = dtype_bytes(out_dtype);
  const bool vec_ok = aligned16(gate) && aligned16(up) && aligned16(out) && n % V == 0 &&
                      gate_row_stride % V == 0 && up_row_stride % V == 0 &&
                      (out_row_stride * ob) % 16 == 0;
  if (act == HGK_ACT_SILU) return dispatch<HGK_ACT_SILU>(a, dtype, out_dtype, vec_ok, rows, n, as_stream(stream));
  return dispatch<HGK_ACT_GELU_TANH>(a, dtype, out_dtype, vec_ok, rows, n, as_stream(stream));
}
