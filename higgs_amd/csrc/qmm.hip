// qmm.hip -- gather_qmm for 4-bit affine weights (MLX layout) on gfx950: the
// MoE expert projections of crates/higgs-models/src/qwen3_next.rs:294-363,
// 844-904 (SwitchMlpWeights::forward_gather), where every (token, expert)
// pair multiplies one activation row by one expert's weight matrix:
//
//   y[p, n] = sum_k x[row(p), k] * (s[e_p, n, k/g] * q[e_p, n, k] + b[e_p, n, k/g])
//
// with w [E, N, K/8] u32 (8 codes per word, low nibble first), scales and
// biases [E, N, K/g], row(p) = p / x_row_div (or lhs[p]), e_p = experts[p].
// This is transpose=true (weights stored row-major as [N, K]); M = 1 per pair,
// as forward_gather calls it.
//
// Per pair the weights are read once (decode: ~one token per expert, so the
// kernel is bound by the 4-bit weight stream). The arithmetic avoids a full
// dequantization: a code q becomes the bf16 value 128 + q with two bit
// operations (0x4300 | q), v_dot2c_f32_bf16 accumulates x * (128 + q) in f32
// two codes at a time, and per half-group (32 codes) the affine part is
//   s * (sum x*(128+q) - 128 * sum x) + b * sum x
// with the half-group sums of x computed once per block into LDS.
//
// Decode touches ~1.25 pairs per expert, so reading an expert's tile once per
// pair costs ~1.75x the distinct-expert bytes; grouping the pairs by expert
// (sorted order, one block walking an expert's pairs, or a block that lists
// its expert's pairs itself and holds the weights in registers across them:
// 98 against 67 us at 64 sequences x top-10 of 512) measured slower on
// MI355X -- the pairs of one expert run at the same time on different CUs,
// and serialising them costs more than the re-read. At prefill (16 or more
// pairs per expert) the grouped matrix-core kernel in qgemm.hip runs instead.
#include <algorithm>

#include "../../include/higgs_hip.h"
#include "hgk_act.h"
#include "hgk_common.h"
#include "hgk_host.h"
#include "qgemm.h"

namespace hgk {

struct QmmArgs {
  const void* x;
  int64_t xrows;    // rows of x; a pair whose row falls outside gets a zero row
  int64_t xs;       // x row stride (elements)
  int64_t xdiv;     // pair p reads x row p / xdiv (when lhs is null)
  const int32_t* lhs;
  const uint32_t* w;
  const void* sc;
  const void* bi;
  const void* experts;
  int experts_i32;
  int64_t E, N, K;
  int group;
  int gsh;          // log2(group): group is 32, 64 or 128
  int64_t pairs;
  int64_t p0;       // first pair of this launch (launches cover <= 65535 pairs)
  void* y;
  int64_t ys;
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ inline float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

__device__ inline int64_t pair_expert(const QmmArgs& a, int64_t p) {
  if (a.experts == nullptr) return 0;  // quantized_matmul: one weight matrix
  if (a.experts_i32) {
    const int64_t e = reinterpret_cast<const int32_t*>(a.experts)[p];
    return e < 0 ? e + a.E : e;
  }
  return (int64_t)reinterpret_cast<const uint32_t*>(a.experts)[p];
}

// x row of pair p, or -1 when it is outside x (pairs < 2^31, so the
// division is done in 32 bits)
__device__ inline int64_t pair_row(const QmmArgs& a, int64_t p) {
  int64_t r = a.lhs ? (int64_t)a.lhs[p] : (int64_t)((uint32_t)p / (uint32_t)a.xdiv);
  if (a.lhs && r < 0) r += a.xrows;
  return (r >= 0 && r < a.xrows) ? r : -1;
}

// Stage one bf16 x row of K elements in LDS in dot order (the codes of a
// word pair as (0,4) (1,5) (2,6) (3,7)) with its 32-element half-group sums.
// Contains the block's barriers: every thread of the block calls it.
template <int K, int NT = 256>
__device__ inline void qmv_stage_x(const uint16_t* xrow, uint32_t* xs_perm, float* hsum) {
  // thread t handles one word's worth (8 elements) of the row
  for (int wd = threadIdx.x; wd < K / 8; wd += NT) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(xrow + wd * 8);
    // elements 0..7 as lo/hi halves of v[0..3]: e0=v0.lo e1=v0.hi e2=v1.lo ...
    // dot order pairs (e0,e4) (e1,e5) (e2,e6) (e3,e7)
    xs_perm[wd * 4 + 0] = (v[0] & 0xffffu) | (v[2] << 16);
    xs_perm[wd * 4 + 1] = (v[0] >> 16) | (v[2] & 0xffff0000u);
    xs_perm[wd * 4 + 2] = (v[1] & 0xffffu) | (v[3] << 16);
    xs_perm[wd * 4 + 3] = (v[1] >> 16) | (v[3] & 0xffff0000u);
  }
  __syncthreads();
  for (int h = threadIdx.x; h < K / 32; h += NT) {
    float sacc = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; ++q) sacc = dot2_bf16(xs_perm[h * 16 + q], 0x3f803f80u, sacc);
    hsum[h] = sacc;
  }
  __syncthreads();
}

// This lane's share of one output row: its 32 codes per step against the
// staged x, the affine part applied per half group.
template <class S, int STEPS>
__device__ inline float qmv_dot(const u32x4* codes, const uint32_t* sraw, const uint32_t* braw,
                                const uint32_t* xs_perm, const float* hsum, int j) {
  // the nibble mask and the exponent bits of 128 in registers: a
  // three-operand and-or takes no literal on this target, and with literals
  // the compiler splits it into a separate and and or
  uint32_t nib = 0x000f000fu, one = 0x43004300u;
  asm volatile("" : "+v"(nib), "+v"(one));
  float acc = 0.0f;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const u32x4 cs = codes[s];
    const int h = s * 4 + j;  // half group index
    const u32x4 xq0 = *reinterpret_cast<const u32x4*>(&xs_perm[h * 16 + 0]);
    const u32x4 xq1 = *reinterpret_cast<const u32x4*>(&xs_perm[h * 16 + 4]);
    const u32x4 xq2 = *reinterpret_cast<const u32x4*>(&xs_perm[h * 16 + 8]);
    const u32x4 xq3 = *reinterpret_cast<const u32x4*>(&xs_perm[h * 16 + 12]);
    const u32x4 xw[4] = {xq0, xq1, xq2, xq3};
    float d = 0.0f;
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
      const uint32_t c = cs[wi];
      // (128 + q_i, 128 + q_{i+4}) as packed bf16, i = 0..3
      d = dot2_bf16(xw[wi][0], (c & nib) | one, d);
      d = dot2_bf16(xw[wi][1], ((c >> 4) & nib) | one, d);
      d = dot2_bf16(xw[wi][2], ((c >> 8) & nib) | one, d);
      d = dot2_bf16(xw[wi][3], ((c >> 12) & nib) | one, d);
    }
    const float hs = hsum[h];
    const float sv = S::lo(sraw[s]), bv = S::lo(braw[s]);
    acc = __builtin_fmaf(sv, d - 128.0f * hs, acc);
    acc = __builtin_fmaf(bv, hs, acc);
  }
  return acc;
}

// bf16 x: one block = one pair x 64 output rows (4 waves x 16 rows); a row
// is split over 4 lanes, lane j reading 16 bytes (32 codes) per step of 128
// codes, so a wave's load covers 16 rows x 64 contiguous bytes. STEPS = K/128.
// The x row is staged in LDS permuted to the code order of a word (codes 0..7
// of a word pair as (0,4) (1,5) (2,6) (3,7)), with its half-group sums.
template <class S, int STEPS>
__global__ __launch_bounds__(256) void qmv_bf16_kernel(QmmArgs a) {
  constexpr int K = STEPS * 128;
  __shared__ __attribute__((aligned(16))) uint32_t xs_perm[K / 2];  // bf16 pairs in dot order
  __shared__ float hsum[K / 32];       // sum of x over each 32-code half group
  const int64_t p = a.p0 + blockIdx.y;
  const int64_t e = pair_expert(a, p);
  const int64_t xr0 = pair_row(a, p);
  const bool valid = e >= 0 && e < a.E && xr0 >= 0;
  const int64_t xr = xr0 >= 0 ? xr0 : 0;
  const uint16_t* xrow = reinterpret_cast<const uint16_t*>(a.x) + xr * a.xs;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane >> 2, j = lane & 3;
  const int64_t n = (int64_t)blockIdx.x * 64 + wave * 16 + r;
  const bool live = n < a.N && valid;
  const int64_t nc = n < a.N ? n : a.N - 1;
  const int64_t ec = valid ? e : 0;
  const uint32_t* wrow = a.w + (ec * a.N + nc) * (K / 8);
  const int gpr = K >> a.gsh;
  const uint16_t* srow = reinterpret_cast<const uint16_t*>(a.sc) + (ec * a.N + nc) * gpr;
  const uint16_t* brow = reinterpret_cast<const uint16_t*>(a.bi) + (ec * a.N + nc) * gpr;

  // the weight stream goes out first; x is staged while it is in flight (a
  // barrier orders memory operations, so loads issued after the staging
  // barriers would wait for it)
  u32x4 codes[STEPS];
  uint32_t sraw[STEPS], braw[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    codes[s] = *reinterpret_cast<const u32x4*>(wrow + s * 16 + j * 4);
    const int g = (s * 128 + j * 32) >> a.gsh;
    sraw[s] = srow[g];
    braw[s] = brow[g];
  }

  qmv_stage_x<K>(xrow, xs_perm, hsum);
  float acc = qmv_dot<S, STEPS>(codes, sraw, braw, xs_perm, hsum, j);
  // the row's 4 lanes are adjacent: reduce within the quad
  acc += __shfl_xor(acc, 1, 64);
  acc += __shfl_xor(acc, 2, 64);
  if (j == 0 && n < a.N) {
    const float out = live ? acc : 0.0f;
    store1<BF16>(a.y, p * a.ys + n, out);
  }
}

// The gate and up projections of one pair and the SwiGLU between them, in one
// block (SwitchMlpWeights::forward_gather's gate_out, up_out, swiglu): waves
// 0-1 take 32 rows of the gate weights, waves 2-3 the same 32 rows of the up
// weights, all four sharing the staged x row. The up waves pass their
// results, rounded to bf16 as gather_qmm writes them, through LDS, and the
// gate waves write round(round(g * round(sigmoid g)) * u) -- the three
// reference calls' composition, without the gate and up rows ever reaching
// memory. (Blocks of 8 waves over 64 + 64 rows measured 6 % slower.)
template <class S, int STEPS>
__global__ __launch_bounds__(256) void qmv_swiglu_bf16_kernel(QmmArgs a, const uint32_t* wu,
                                                              const void* scu, const void* biu) {
  constexpr int K = STEPS * 128;
  __shared__ __attribute__((aligned(16))) uint32_t xs_perm[K / 2];
  __shared__ float hsum[K / 32];
  __shared__ float upv[32];
  const int64_t p = a.p0 + blockIdx.y;
  const int64_t e = pair_expert(a, p);
  const int64_t xr0 = pair_row(a, p);
  const bool valid = e >= 0 && e < a.E && xr0 >= 0;
  const int64_t xr = xr0 >= 0 ? xr0 : 0;
  const uint16_t* xrow = reinterpret_cast<const uint16_t*>(a.x) + xr * a.xs;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const bool is_up = wave >= 2;  // uniform per wave
  const int r = lane >> 2, j = lane & 3;
  const int slot = (wave & 1) * 16 + r;
  const int64_t n = (int64_t)blockIdx.x * 32 + slot;
  const bool live = n < a.N && valid;
  const int64_t nc = n < a.N ? n : a.N - 1;
  const int64_t ec = valid ? e : 0;
  const uint32_t* wsel = is_up ? wu : a.w;
  const uint16_t* ssel = reinterpret_cast<const uint16_t*>(is_up ? scu : a.sc);
  const uint16_t* bsel = reinterpret_cast<const uint16_t*>(is_up ? biu : a.bi);
  const uint32_t* wrow = wsel + (ec * a.N + nc) * (K / 8);
  const int gpr = K >> a.gsh;
  const uint16_t* srow = ssel + (ec * a.N + nc) * gpr;
  const uint16_t* brow = bsel + (ec * a.N + nc) * gpr;

  u32x4 codes[STEPS];
  uint32_t sraw[STEPS], braw[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    codes[s] = *reinterpret_cast<const u32x4*>(wrow + s * 16 + j * 4);
    const int g = (s * 128 + j * 32) >> a.gsh;
    sraw[s] = srow[g];
    braw[s] = brow[g];
  }

  qmv_stage_x<K>(xrow, xs_perm, hsum);
  float acc = qmv_dot<S, STEPS>(codes, sraw, braw, xs_perm, hsum, j);
  acc += __shfl_xor(acc, 1, 64);
  acc += __shfl_xor(acc, 2, 64);
  const float v = BF16::round(live ? acc : 0.0f);  // the projection's bf16 output
  if (is_up && j == 0) upv[slot] = v;
  __syncthreads();
  if (!is_up && j == 0 && n < a.N) {
    float out;
    const float u = upv[slot];
    swiglu16<BF16, 1>(&v, &u, &out);
    store1<BF16>(a.y, p * a.ys + n, out);
  }
}

// Any shape / dtype: one wave per (pair, output row), f32 arithmetic with
// exact dequantized values, element-strided.
template <class X, class S>
__global__ __launch_bounds__(256) void qmv_generic_kernel(QmmArgs a) {
  // one wave per output element, in a grid-stride loop over the waves (the
  // loop bound is uniform per wave, so the reduction has every lane)
  const int lane = threadIdx.x & 63;
  const int64_t items = a.pairs * a.N;
  const int64_t stride = (int64_t)gridDim.x * 4;
  for (int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); item < items; item += stride) {
    const int64_t p = item / a.N, n = item - p * a.N;
    const int64_t e = pair_expert(a, p);
    const int64_t xr = pair_row(a, p);
    float acc = 0.0f;
    if (e >= 0 && e < a.E && xr >= 0) {
      const int64_t gpr = a.K / a.group;
      for (int64_t k = lane; k < a.K; k += 64) {
        const uint32_t q = (a.w[(e * a.N + n) * (a.K / 8) + k / 8] >> (4 * (k % 8))) & 0xfu;
        const int64_t g = (e * a.N + n) * gpr + k / a.group;
        const float wv = load1<S>(a.sc, g) * (float)q + load1<S>(a.bi, g);
        acc = __builtin_fmaf(load1<X>(a.x, xr * a.xs + k), wv, acc);
      }
    }
    acc = group_sum<64>(acc);
    if (lane == 0) store1<X>(a.y, p * a.ys + n, acc);
  }
}

namespace {

template <class S, int STEPS>
void launch_bf16_k(QmmArgs a, hipStream_t s) {
  // one launch per 65535 pairs (the grid's y extent)
  for (int64_t p0 = 0; p0 < a.pairs; p0 += 65535) {
    a.p0 = p0;
    const int64_t np = a.pairs - p0 < 65535 ? a.pairs - p0 : 65535;
    const dim3 grid((unsigned)((a.N + 63) / 64), (unsigned)np);
    HGK_LAUNCH((qmv_bf16_kernel<S, STEPS>), grid, dim3(256), 0, s, a);
  }
}

template <class S>
bool launch_bf16(const QmmArgs& a, hipStream_t s) {
  switch (a.K) {
    case 512: launch_bf16_k<S, 4>(a, s); return true;
    case 1024: launch_bf16_k<S, 8>(a, s); return true;
    case 2048: launch_bf16_k<S, 16>(a, s); return true;
    case 4096: launch_bf16_k<S, 32>(a, s); return true;
    default: return false;
  }
}

template <int STEPS>
void launch_swiglu_k(QmmArgs a, const uint32_t* wu, const void* su, const void* bu, hipStream_t s) {
  for (int64_t p0 = 0; p0 < a.pairs; p0 += 65535) {
    a.p0 = p0;
    const int64_t np = a.pairs - p0 < 65535 ? a.pairs - p0 : 65535;
    const dim3 grid((unsigned)((a.N + 31) / 32), (unsigned)np);
    HGK_LAUNCH((qmv_swiglu_bf16_kernel<BF16, STEPS>), grid, dim3(256), 0, s, a, wu, su, bu);
  }
}

template <class X, class S>
void launch_generic(const QmmArgs& a, hipStream_t s) {
  const int64_t items = a.pairs * a.N;
  // a grid of at most 2^20 blocks (2^28 work-items), well inside HIP's limit
  const int64_t blocks = std::min<int64_t>((items + 3) / 4, (int64_t)1 << 20);
  HGK_LAUNCH((qmv_generic_kernel<X, S>), dim3((unsigned)blocks), dim3(256), 0, s, a);
}

}  // namespace
}  // namespace hgk

using namespace hgk;

extern "C" int hgk_gather_qmm(int dtype, const void* x, int64_t x_rows, int64_t x_row_stride,
                              int64_t x_row_div,
                              const int32_t* lhs_indices, const uint32_t* w, const void* scales,
                              const void* biases, int scales_dtype, int64_t n_experts, int64_t n,
                              int64_t k, int group_size, int bits, const void* rhs_indices,
                              int rhs_dtype, int64_t pairs, void* y, int64_t y_row_stride,
                              void* stream) {
  clear_error();
  const char* fn = "hgk_gather_qmm";
  if (bits != 4) return fail(HGK_ERR_UNSUPPORTED, "%s: bits=%d (only 4 is implemented)", fn, bits);
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail(HGK_ERR_UNSUPPORTED, "%s: group_size=%d (32, 64 or 128)", fn, group_size);
  if (dtype != DT_BF16 && dtype != DT_F16)
    return fail(HGK_ERR_UNSUPPORTED, "%s: activation dtype must be bf16 or f16", fn);
  if (scales_dtype != dtype)
    return fail(HGK_ERR_UNSUPPORTED, "%s: scales/biases must have the activation dtype", fn);
  if (rhs_dtype != DT_I32 && rhs_dtype != DT_U32)
    return fail(HGK_ERR_ARG, "%s: expert indices must be int32 or uint32", fn);
  if (pairs < 0 || n_experts <= 0 || n <= 0 || k <= 0 || k % group_size || k % 8)
    return fail(HGK_ERR_ARG, "%s: bad shape pairs=%lld E=%lld N=%lld K=%lld (K a multiple of %d)", fn,
                (long long)pairs, (long long)n_experts, (long long)n, (long long)k, group_size);
  if (!lhs_indices && x_row_div <= 0) return fail(HGK_ERR_ARG, "%s: x_row_div must be >= 1", fn);
  if (pairs > 0 && (x_rows <= 0 || (!lhs_indices && (pairs - 1) / (x_row_div > 0 ? x_row_div : 1) >= x_rows)))
    return fail(HGK_ERR_ARG, "%s: %lld pairs with x_row_div %lld need more than %lld rows of x", fn,
                (long long)pairs, (long long)x_row_div, (long long)x_rows);
  if ((x_rows > 1 && x_row_stride < k) || (pairs > 1 && y_row_stride < n))
    return fail(HGK_ERR_ARG, "%s: row strides (%lld, %lld) smaller than K=%lld / N=%lld", fn,
                (long long)x_row_stride, (long long)y_row_stride, (long long)k, (long long)n);
  if (!w || !scales || !biases || ((!x || !rhs_indices || !y) && pairs > 0))
    return fail(HGK_ERR_ARG, "%s: null pointer", fn);
  if (n_experts * n * k >= ((int64_t)1 << 42) || pairs * n >= ((int64_t)1 << 32) || pairs >= ((int64_t)1 << 31))
    return fail(HGK_ERR_UNSUPPORTED, "%s: problem too large", fn);
  if (pairs == 0) return HGK_OK;
  QmmArgs a{};
  a.x = x; a.xrows = x_rows; a.xs = x_row_stride; a.xdiv = x_row_div > 0 ? x_row_div : 1; a.lhs = lhs_indices;
  a.w = w; a.sc = scales; a.bi = biases; a.experts = rhs_indices; a.experts_i32 = rhs_dtype == DT_I32;
  a.E = n_experts; a.N = n; a.K = k; a.group = group_size; a.pairs = pairs; a.y = y;
  a.gsh = group_size == 32 ? 5 : group_size == 64 ? 6 : 7;
  a.ys = y_row_stride;
  const hipStream_t s = as_stream(stream);
  // many pairs per expert (prefill): grouped by expert on the matrix cores
  if (pairs >= kGatherMinPairsPerExpert * n_experts && n_experts < 65535 &&
      gather_grouped_supported(dtype, scales_dtype, group_size, bits, x, x_row_stride, w, k,
                               rhs_indices, pairs)) {
    GatherArgs g{};
    g.x = static_cast<const uint16_t*>(x); g.xrows = x_rows; g.xs = x_row_stride;
    g.xdiv = x_row_div > 0 ? x_row_div : 1; g.lhs = lhs_indices; g.w = w;
    g.sc = static_cast<const uint16_t*>(scales); g.bi = static_cast<const uint16_t*>(biases);
    g.experts = rhs_indices; g.experts_i32 = rhs_dtype == DT_I32; g.E = n_experts; g.N = n; g.K = k;
    g.pairs = pairs; g.y = static_cast<uint16_t*>(y); g.ys = y_row_stride;
    gather_grouped_launch(g, s);
    return launch_status(fn);
  }
  const bool vec_ok = dtype == DT_BF16 && aligned16(x) && x_row_stride % 8 == 0 && aligned16(w) &&
                      (reinterpret_cast<uintptr_t>(scales) & 1) == 0;
  if (vec_ok && launch_bf16<BF16>(a, s)) return launch_status(fn);
  if (dtype == DT_BF16) launch_generic<BF16, BF16>(a, s);
  else launch_generic<F16, F16>(a, s);
  return launch_status(fn);
}

extern "C" int hgk_quantized_matmul(int dtype, const void* x, int64_t m, int64_t x_row_stride,
                                    const uint32_t* w, const void* scales, const void* biases,
                                    int scales_dtype, int64_t n, int64_t k, int group_size,
                                    int bits, void* y, int64_t y_row_stride, void* stream) {
  clear_error();
  const char* fn = "hgk_quantized_matmul";
  if (bits != 4) return fail(HGK_ERR_UNSUPPORTED, "%s: bits=%d (only 4 is implemented)", fn, bits);
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail(HGK_ERR_UNSUPPORTED, "%s: group_size=%d (32, 64 or 128)", fn, group_size);
  if (dtype != DT_BF16 && dtype != DT_F16)
    return fail(HGK_ERR_UNSUPPORTED, "%s: activation dtype must be bf16 or f16", fn);
  if (scales_dtype != dtype)
    return fail(HGK_ERR_UNSUPPORTED, "%s: scales/biases must have the activation dtype", fn);
  if (m < 0 || n <= 0 || k <= 0 || k % group_size || k % 8)
    return fail(HGK_ERR_ARG, "%s: bad shape M=%lld N=%lld K=%lld (K a multiple of %d)", fn,
                (long long)m, (long long)n, (long long)k, group_size);
  if ((m > 1 && x_row_stride < k) || (m > 1 && y_row_stride < n))
    return fail(HGK_ERR_ARG, "%s: row strides (%lld, %lld) smaller than K=%lld / N=%lld", fn,
                (long long)x_row_stride, (long long)y_row_stride, (long long)k, (long long)n);
  if (!w || !scales || !biases || ((!x || !y) && m > 0)) return fail(HGK_ERR_ARG, "%s: null pointer", fn);
  if (n * k >= ((int64_t)1 << 42) || m >= ((int64_t)1 << 31))
    return fail(HGK_ERR_UNSUPPORTED, "%s: problem too large", fn);
  if (m == 0) return HGK_OK;
  const hipStream_t s = as_stream(stream);
  if (m >= kQgemmMinRows &&
      qgemm_supported(dtype, scales_dtype, group_size, bits, x, x_row_stride, w, k) &&
      (m + 127) / 128 <= 65535) {
    QgemmArgs g{};
    g.x = static_cast<const uint16_t*>(x); g.xs = x_row_stride; g.w = w;
    g.sc = static_cast<const uint16_t*>(scales); g.bi = static_cast<const uint16_t*>(biases);
    g.M = m; g.N = n; g.K = k; g.y = static_cast<uint16_t*>(y); g.ys = y_row_stride;
    qgemm_launch(g, s);
    return launch_status(fn);
  }
  if (m * n >= ((int64_t)1 << 32))
    return fail(HGK_ERR_UNSUPPORTED, "%s: M=%lld x N=%lld too large for the per-row path", fn,
                (long long)m, (long long)n);
  // one GEMV per row: the gather kernel with a single weight matrix
  QmmArgs a{};
  a.x = x; a.xrows = m; a.xs = x_row_stride; a.xdiv = 1; a.lhs = nullptr;
  a.w = w; a.sc = scales; a.bi = biases; a.experts = nullptr; a.experts_i32 = 0;
  a.E = 1; a.N = n; a.K = k; a.group = group_size; a.pairs = m; a.y = y; a.ys = y_row_stride;
  a.gsh = group_size == 32 ? 5 : group_size == 64 ? 6 : 7;
  const bool vec_ok = dtype == DT_BF16 && aligned16(x) && x_row_stride % 8 == 0 && aligned16(w) &&
                      (reinterpret_cast<uintptr_t>(scales) & 1) == 0;
  if (vec_ok && launch_bf16<BF16>(a, s)) return launch_status(fn);
  if (dtype == DT_BF16) launch_generic<BF16, BF16>(a, s);
  else launch_generic<F16, F16>(a, s);
  return launch_status(fn);
}

extern "C" int hgk_gather_qmm_swiglu(int dtype, const void* x, int64_t x_rows,
                                     int64_t x_row_stride, int64_t x_row_div,
                                     const int32_t* lhs_indices, const uint32_t* w_gate,
                                     const void* scales_gate, const void* biases_gate,
                                     const uint32_t* w_up, const void* scales_up,
                                     const void* biases_up, int scales_dtype, int64_t n_experts,
                                     int64_t n, int64_t k, int group_size, int bits,
                                     const void* rhs_indices, int rhs_dtype, int64_t pairs,
                                     void* y, int64_t y_row_stride, void* stream) {
  clear_error();
  const char* fn = "hgk_gather_qmm_swiglu";
  if (bits != 4) return fail(HGK_ERR_UNSUPPORTED, "%s: bits=%d (only 4 is implemented)", fn, bits);
  if (dtype != DT_BF16 || scales_dtype != DT_BF16)
    return fail(HGK_ERR_UNSUPPORTED, "%s: bf16 activations and scales only", fn);
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail(HGK_ERR_UNSUPPORTED, "%s: group_size=%d (32, 64 or 128)", fn, group_size);
  if (rhs_dtype != DT_I32 && rhs_dtype != DT_U32)
    return fail(HGK_ERR_ARG, "%s: expert indices must be int32 or uint32", fn);
  if (pairs < 0 || n_experts <= 0 || n <= 0 || k <= 0 || k % group_size || k % 8)
    return fail(HGK_ERR_ARG, "%s: bad shape pairs=%lld E=%lld N=%lld K=%lld", fn, (long long)pairs,
                (long long)n_experts, (long long)n, (long long)k);
  if (k != 512 && k != 1024 && k != 2048 && k != 4096)
    return fail(HGK_ERR_UNSUPPORTED, "%s: K=%lld (512, 1024, 2048 or 4096)", fn, (long long)k);
  if (!lhs_indices && x_row_div <= 0) return fail(HGK_ERR_ARG, "%s: x_row_div must be >= 1", fn);
  if (pairs > 0 && (x_rows <= 0 || (!lhs_indices && (pairs - 1) / (x_row_div > 0 ? x_row_div : 1) >= x_rows)))
    return fail(HGK_ERR_ARG, "%s: %lld pairs with x_row_div %lld need more than %lld rows of x", fn,
                (long long)pairs, (long long)x_row_div, (long long)x_rows);
  if ((x_rows > 1 && x_row_stride < k) || (pairs > 1 && y_row_stride < n))
    return fail(HGK_ERR_ARG, "%s: row strides (%lld, %lld) smaller than K=%lld / N=%lld", fn,
                (long long)x_row_stride, (long long)y_row_stride, (long long)k, (long long)n);
  if (!w_gate || !scales_gate || !biases_gate || !w_up || !scales_up || !biases_up ||
      ((!x || !rhs_indices || !y) && pairs > 0))
    return fail(HGK_ERR_ARG, "%s: null pointer", fn);
  if (pairs == 0) return HGK_OK;
  if (n_experts * n * k >= ((int64_t)1 << 42) || pairs * n >= ((int64_t)1 << 32) || pairs >= ((int64_t)1 << 31))
    return fail(HGK_ERR_UNSUPPORTED, "%s: problem too large", fn);
  const auto odd = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 1) != 0; };
  if (!aligned16(x) || x_row_stride % 8 || !aligned16(w_gate) || !aligned16(w_up) ||
      odd(scales_gate) || odd(biases_gate) || odd(scales_up) || odd(biases_up))
    return fail(HGK_ERR_UNSUPPORTED, "%s: x and the weights must be 16-byte aligned", fn);
  if (pairs >= kGatherMinPairsPerExpert * n_experts) {
    // many pairs per expert (prefill): the grouped matrix-core kernel's fused
    // form, where it applies
    if (pairs > 0 && n_experts < 65535 &&
        gather_grouped_supported(dtype, scales_dtype, group_size, bits, x, x_row_stride, w_gate, k,
                                 rhs_indices, pairs)) {
      GatherArgs g{};
      g.x = static_cast<const uint16_t*>(x); g.xrows = x_rows; g.xs = x_row_stride;
      g.xdiv = x_row_div > 0 ? x_row_div : 1; g.lhs = lhs_indices; g.w = w_gate;
      g.sc = static_cast<const uint16_t*>(scales_gate); g.bi = static_cast<const uint16_t*>(biases_gate);
      g.w2 = w_up; g.sc2 = static_cast<const uint16_t*>(scales_up);
      g.bi2 = static_cast<const uint16_t*>(biases_up);
      g.experts = rhs_indices; g.experts_i32 = rhs_dtype == DT_I32; g.E = n_experts; g.N = n; g.K = k;
      g.pairs = pairs; g.y = static_cast<uint16_t*>(y); g.ys = y_row_stride;
      if (gather_swiglu_grouped_launch(g, as_stream(stream))) return launch_status(fn);
    }
    return fail(HGK_ERR_UNSUPPORTED,
                "%s: %lld pairs over %lld experts is the grouped (prefill) regime and the fused "
                "grouped kernel does not take this call: run gate and up through hgk_gather_qmm and "
                "the activation through hgk_glu",
                fn, (long long)pairs, (long long)n_experts);
  }
  if (pairs == 0) return HGK_OK;
  QmmArgs a{};
  a.x = x; a.xrows = x_rows; a.xs = x_row_stride; a.xdiv = x_row_div > 0 ? x_row_div : 1; a.lhs = lhs_indices;
  a.w = w_gate; a.sc = scales_gate; a.bi = biases_gate; a.experts = rhs_indices;
  a.experts_i32 = rhs_dtype == DT_I32;
  a.E = n_experts; a.N = n; a.K = k; a.group = group_size; a.pairs = pairs; a.y = y;
  a.gsh = group_size == 32 ? 5 : group_size == 64 ? 6 : 7;
  a.ys = y_row_stride;
  const hipStream_t s = as_stream(stream);
  switch (k) {
    case 512: launch_swiglu_k<4>(a, w_up, scales_up, biases_up, s); break;
    case 1024: launch_swiglu_k<8>(a, w_up, scales_up, biases_up, s); break;
    case 2048: launch_swiglu_k<16>(a, w_up, scales_up, biases_up, s); break;
    default: launch_swiglu_k<32>(a, w_up, scales_up, biases_up, s); break;
  }
  return launch_status(fn);
}
