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
// with MLX's sigmoid (1/(1+exp(|g|)), complemented for g >= 0) and MLX's
// polynomial exp, built from IEEE operations only.
// GeGLU runs in f32 (mlx-rs builds gelu_approximate from f32 scalar arrays,
// which promote a bf16 input): 0.5*g*(1+tanh(k0*(g + k1*g^3))) is evaluated as
// the identical g / (1 + exp(-2*k0*(g + k1*g^3))), using the hardware exp2 and
// reciprocal (relative error ~1e-6), and the product with up is rounded once.
//
// Large 16-bit SwiGLU: the exact sigmoid costs ~40 VALU operations per element,
// which would make the kernel compute-bound. But round_T(g * round_T(sig(g)))
// depends only on the 16 bits of g, so a 64K-entry table of it (built once per
// device by the exact code path) is held in LDS (128 KB of gfx950's 160 KB per
// CU) by one 1024-thread block per CU; each element then costs one LDS lookup,
// one multiply and one conversion, bit-identical to the direct path.
#include <mutex>

#include "../../include/higgs_hip.h"
#include "hgk_common.h"
#include "hgk_host.h"

namespace hgk {

// s = round_T(g * round_T(sigmoid(g))) for every 16-bit pattern g.
__device__ uint16_t g_silu_lut_bf16[65536];
__device__ uint16_t g_silu_lut_f16[65536];

template <class X>
__device__ inline uint16_t* silu_lut() {
  if constexpr (X::kCode == DT_BF16) return g_silu_lut_bf16;
  else return g_silu_lut_f16;
}

template <class X>
__global__ __launch_bounds__(256) void silu_lut_init_kernel() {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  const float g = X::lo(i);
  const float sg = X::round(mlx_sigmoid(g));
  const float s = X::round(g * sg);
  silu_lut<X>()[i] = (uint16_t)(X::pack(s, 0.0f) & 0xffffu);
}

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

template <class X, int ACT>
__device__ inline float glu1(float g, float u) {
  if constexpr (ACT == HGK_ACT_SILU) {
    const float sg = X::round(mlx_sigmoid(g));
    const float s = X::round(g * sg);
    return X::round(s * u);
  } else {
    const float k0 = 0.7978845608028654f, k1 = 0.044715f;
    const float g3 = g * g * g;
    const float inner = k0 * (g + k1 * g3);
    const float e = __builtin_amdgcn_exp2f(inner * -2.8853900817779268f);  // exp(-2*inner)
    const float gl = g * __builtin_amdgcn_rcpf(1.0f + e);
    return gl * u;
  }
}

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
    gr[k] = ld16<X>(a.g, go);
    ur[k] = ld16<X>(a.u, uo);
  }
#pragma unroll
  for (int k = 0; k < U; ++k) {
    float o[V];
#pragma unroll
    for (int e = 0; e < V; ++e) o[e] = glu1<X, ACT>(elem<X>(gr[k], e), elem<X>(ur[k], e));
    if (base + 256u * k < a.total) store_elems<Y, V>(a.o, oo[k], o);
  }
}

// Any alignment / width: one element per thread.
template <class X, class Y, int ACT>
__global__ __launch_bounds__(256) void glu_generic_kernel(GluArgs a, int64_t n, int64_t rows) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n * rows) return;
  const int64_t row = i / n, c = i - row * n;
  const float g = load1<X>(a.g, row * a.gs + c), u = load1<X>(a.u, row * a.us + c);
  store1<Y>(a.o, row * a.os + c, glu1<X, ACT>(g, u));
}

constexpr int kLutBlock = 1024;
constexpr int kLutUnroll = 4;

// Persistent SwiGLU for 16-bit X: one 1024-thread block per CU loads the silu
// table into LDS once, then strides over the tensor kLutUnroll chunks per
// thread at a time (all loads of a step issued before any lookup).
template <class X, class Y, bool CONTIG>
__global__ __launch_bounds__(kLutBlock) void swiglu_lut_kernel(GluArgs a) {
  constexpr int V = Vec<X>::N;
  constexpr int U = kLutUnroll;
  __shared__ uint16_t lut[65536];
  const uint32_t per_iter = (uint32_t)kLutBlock * U;
  const uint32_t stride = gridDim.x * per_iter;
  u32x4 gr[U], ur[U];
  int64_t oo[U];
  auto load_step = [&](uint32_t base) {
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const uint32_t q = base + (uint32_t)kLutBlock * k;
      const uint32_t qq = q < a.total ? q : a.total - 1;
      int64_t go, uo;
      glu_offsets<V, CONTIG>(a, qq, go, uo, oo[k]);
      gr[k] = ld16<X>(a.g, go);
      ur[k] = ld16<X>(a.u, uo);
    }
  };
  // the first step's loads go out before the 128 KB table copy
  uint32_t base = blockIdx.x * per_iter + threadIdx.x;
  load_step(base);
  {
    const u32x4* src = reinterpret_cast<const u32x4*>(silu_lut<X>());
    u32x4* dst = reinterpret_cast<u32x4*>(lut);
#pragma unroll
    for (int i = 0; i < 65536 * 2 / 16 / kLutBlock; ++i)
      dst[i * kLutBlock + threadIdx.x] = src[i * kLutBlock + threadIdx.x];
  }
  __syncthreads();
  while (base < a.total) {
#pragma unroll
    for (int k = 0; k < U; ++k) {
      float o[V];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float s0 = X::lo((uint32_t)lut[gr[k][w] & 0xffffu]);
        const float s1 = X::lo((uint32_t)lut[gr[k][w] >> 16]);
        o[2 * w] = s0 * X::lo(ur[k][w]);
        o[2 * w + 1] = s1 * X::hi(ur[k][w]);
        if constexpr (Y::kCode != X::kCode) {  // MLX's result is X; widen after rounding
          o[2 * w] = X::round(o[2 * w]);
          o[2 * w + 1] = X::round(o[2 * w + 1]);
        }
      }
      if (base + (uint32_t)kLutBlock * k < a.total) store_elems<Y, V>(a.o, oo[k], o);
    }
    base += stride;
    if (base < a.total) load_step(base);
  }
}

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_lut_mu;
bool g_lut_ready[2][kMaxDevices];
int g_cu_count[kMaxDevices];

// Build the table for X on the current device once; false when that cannot be
// done right now (stream under graph capture), in which case the caller takes
// the direct path.
template <class X>
bool ensure_silu_lut(hipStream_t s, int* cus) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  const int which = X::kCode == DT_BF16 ? 0 : 1;
  std::lock_guard<std::mutex> lk(g_lut_mu);
  if (!g_cu_count[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      return false;
    g_cu_count[dev] = n;
  }
  *cus = g_cu_count[dev];
  if (g_lut_ready[which][dev]) return true;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return false;
  hipLaunchKernelGGL((silu_lut_init_kernel<X>), dim3(65536 / 256), dim3(256), 0, s);
  if (hipGetLastError() != hipSuccess || hipStreamSynchronize(s) != hipSuccess) return false;
  g_lut_ready[which][dev] = true;
  return true;
}

template <class X, class Y, int ACT>
void launch(const GluArgs& a, bool vec_ok, int64_t rows, int64_t n, hipStream_t s) {
  if constexpr (ACT == HGK_ACT_SILU && X::kBytes == 2) {
    int cus = 0;
    if (vec_ok && a.total >= (1u << 18) && a.total < (1u << 31) && ensure_silu_lut<X>(s, &cus)) {
      const uint32_t per_block = (uint32_t)kLutBlock * kLutUnroll;
      const uint32_t need = (a.total + per_block - 1) / per_block;
      const unsigned blocks = need < (uint32_t)cus ? need : (unsigned)cus;
      if (a.contig) hipLaunchKernelGGL((swiglu_lut_kernel<X, Y, true>), dim3(blocks), dim3(kLutBlock), 0, s, a);
      else hipLaunchKernelGGL((swiglu_lut_kernel<X, Y, false>), dim3(blocks), dim3(kLutBlock), 0, s, a);
      return;
    }
  }
  if (vec_ok) {
    if (a.total >= 256u * 4u * 1024u) {
      const unsigned blocks = (a.total + 1024u - 1u) / 1024u;
      if (a.contig) hipLaunchKernelGGL((glu_kernel<X, Y, ACT, 4, true>), dim3(blocks), dim3(256), 0, s, a);
      else hipLaunchKernelGGL((glu_kernel<X, Y, ACT, 4, false>), dim3(blocks), dim3(256), 0, s, a);
    } else {
      const unsigned blocks = (a.total + 255u) / 256u;
      if (a.contig) hipLaunchKernelGGL((glu_kernel<X, Y, ACT, 1, true>), dim3(blocks), dim3(256), 0, s, a);
      else hipLaunchKernelGGL((glu_kernel<X, Y, ACT, 1, false>), dim3(blocks), dim3(256), 0, s, a);
    }
    return;
  }
  const int64_t blocks = (n * rows + 255) / 256;
  hipLaunchKernelGGL((glu_generic_kernel<X, Y, ACT>), dim3((unsigned)blocks), dim3(256), 0, s,
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
  if (!gate || !up || !out) return fail(HGK_ERR_ARG, "hgk_glu: null pointer");
  if (rows > 1 && (gate_row_stride < n || up_row_stride < n || out_row_stride < n))
    return fail(HGK_ERR_ARG, "hgk_glu: row stride smaller than n");
  if (rows == 0 || n == 0) return HGK_OK;
  const int V = 16 / dtype_bytes(dtype);
  const int64_t chunks = (n / V) * rows;
  if (chunks >= ((int64_t)1 << 32) || n * rows >= ((int64_t)1 << 40))
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
