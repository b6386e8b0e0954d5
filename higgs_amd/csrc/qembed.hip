// qembed.hip -- 4-bit affine QuantizedEmbedding gather + dequantize on gfx950.
//
// Table layout (MLX affine quantization, as stored in MLX 4-bit checkpoints):
//   w_q    [vocab, hidden/8]          u32, 8 codes per word, low nibble first
//   scales [vocab, hidden/group]      bf16 or f16
//   biases [vocab, hidden/group]      same dtype as scales
// One wave64 owns one token: each lane reads 16 bytes of packed codes (32
// codes) per step and its group's scale/bias, and writes 64 bytes of output,
// so a token's row (hidden/2 bytes of codes) is one coalesced burst and the
// write (4x larger) is fully vectorised. The table is never dequantized as a
// whole (QEmbedding::forward does that on every call in the reference).
//
// Arithmetic (MLX dequantize, S = scales dtype):
//   v = round_S(round_S(q * s) + b);  optionally v = round_S(v * round_S(scale))
// which is exact to reproduce: no transcendental functions are involved.
#include "../../include/higgs_hip.h"
#include "hgk_common.h"
#include "hgk_host.h"

namespace hgk {

struct QembArgs {
  const void* ids;
  int ids_i32;
  int64_t n;
  const uint32_t* wq;
  const void* sc;
  const void* bi;
  int64_t vocab;
  int wpr;  // words per row = hidden / 8
  int gpr;  // groups per row = hidden / group
  int group;
  float scale;
  int has_scale;
  void* out;
  int64_t os;
  int64_t hidden;
};

__device__ inline int64_t load_id(const QembArgs& a, int64_t t) {
  if (a.ids_i32) {
    int64_t id = reinterpret_cast<const int32_t*>(a.ids)[t];
    return id < 0 ? id + a.vocab : id;
  }
  return (int64_t)reinterpret_cast<const uint32_t*>(a.ids)[t];
}

template <class S>
__device__ inline float deq(uint32_t q, float s, float b) {
  return S::round(S::round((float)q * s) + b);
}

// One wave per token. At step s lane i owns packed word w = s*64 + i (8 codes,
// one group): each load instruction of the wave reads 256 contiguous bytes of
// the row and each store writes 1 KB contiguous, so no cache line is touched
// by more than one instruction.
template <class S, int STEPS>
__global__ __launch_bounds__(256) void qembed_kernel(QembArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x >> 6) +
                    __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (t >= a.n) return;  // whole wave leaves together
  const int64_t id = load_id(a, t);
  const bool valid = id >= 0 && id < a.vocab;
  const int64_t row = valid ? id : 0;
  const float osc = S::round(a.scale);
  const uint32_t* wrow = a.wq + row * a.wpr;
  const int64_t grow = row * a.gpr;

  // every load of the token goes out first, as raw words (converting a value
  // where it is loaded would make the compiler wait for it step by step)
  uint32_t codes[STEPS], sraw[STEPS], braw[STEPS];
  const uint16_t* sc = reinterpret_cast<const uint16_t*>(a.sc);
  const uint16_t* bi = reinterpret_cast<const uint16_t*>(a.bi);
  // (addresses are clamped into the row instead of predicating the loads, so
  // no select has to wait on a loaded value before the next load issues)
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int w = s * 64 + lane;
    const int wc = w < a.wpr ? w : a.wpr - 1;
    const int g = (wc * 8) / a.group;
    codes[s] = wrow[wc];
    sraw[s] = (uint32_t)sc[grow + g];
    braw[s] = (uint32_t)bi[grow + g];
  }
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int w = s * 64 + lane;
    if (w >= a.wpr) continue;
    const float sv = S::lo(sraw[s]), bv = S::lo(braw[s]);
    float v[8];
#pragma unroll
    for (int nib = 0; nib < 8; ++nib) {
      const uint32_t q = (codes[s] >> (4 * nib)) & 0xfu;
      float x = deq<S>(q, sv, bv);
      x = a.has_scale ? S::round(x * osc) : x;
      v[nib] = valid ? x : 0.0f;
    }
    store_elems<S, 8>(a.out, t * a.os + (int64_t)w * 8, v);
  }
}

// Any layout: one output element per thread.
template <class S>
__global__ __launch_bounds__(256) void qembed_generic_kernel(QembArgs a) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.n * a.hidden) return;
  const int64_t t = i / a.hidden, k = i - t * a.hidden;
  const int64_t id = load_id(a, t);
  float x = 0.0f;
  if (id >= 0 && id < a.vocab) {
    const uint32_t q = (a.wq[id * a.wpr + k / 8] >> (4 * (k % 8))) & 0xfu;
    const int64_t g = id * a.gpr + k / a.group;
    x = deq<S>(q, load1<S>(a.sc, g), load1<S>(a.bi, g));
    if (a.has_scale) x = S::round(x * S::round(a.scale));
  }
  store1<S>(a.out, t * a.os + k, x);
}

namespace {

template <class S>
void launch(const QembArgs& a, bool vec_ok, hipStream_t s) {
  const int steps = (a.wpr + 63) / 64;
  if (vec_ok && steps <= 16) {
    const int wpb = a.n >= 1024 ? 4 : 1;
    const unsigned blocks = (unsigned)((a.n + wpb - 1) / wpb);
    const dim3 g(blocks), b(64 * wpb);
    if (steps <= 1) hipLaunchKernelGGL((qembed_kernel<S, 1>), g, b, 0, s, a);
    else if (steps <= 2) hipLaunchKernelGGL((qembed_kernel<S, 2>), g, b, 0, s, a);
    else if (steps <= 4) hipLaunchKernelGGL((qembed_kernel<S, 4>), g, b, 0, s, a);
    else if (steps <= 7) hipLaunchKernelGGL((qembed_kernel<S, 7>), g, b, 0, s, a);
    else if (steps <= 8) hipLaunchKernelGGL((qembed_kernel<S, 8>), g, b, 0, s, a);
    else hipLaunchKernelGGL((qembed_kernel<S, 16>), g, b, 0, s, a);
    return;
  }
  const int64_t blocks = (a.n * a.hidden + 255) / 256;
  hipLaunchKernelGGL((qembed_generic_kernel<S>), dim3((unsigned)blocks), dim3(256), 0, s, a);
}

}  // namespace
}  // namespace hgk

using namespace hgk;

extern "C" int hgk_quantized_embedding(const void* ids, int ids_dtype, int64_t n_ids,
                                       const uint32_t* w_q, const void* scales,
                                       const void* biases, int scales_dtype, int64_t vocab,
                                       int64_t hidden, int group_size, int bits, float out_scale,
                                       void* out, int64_t out_row_stride, void* stream) {
  clear_error();
  const char* fn = "hgk_quantized_embedding";
  if (bits != 4) return fail(HGK_ERR_UNSUPPORTED, "%s: bits=%d (only 4 is implemented)", fn, bits);
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return fail(HGK_ERR_UNSUPPORTED, "%s: group_size=%d (32, 64 or 128)", fn, group_size);
  if (ids_dtype != DT_I32 && ids_dtype != DT_U32)
    return fail(HGK_ERR_ARG, "%s: ids dtype must be int32 or uint32", fn);
  if (scales_dtype != DT_BF16 && scales_dtype != DT_F16)
    return fail(HGK_ERR_UNSUPPORTED, "%s: scales dtype must be bf16 or f16", fn);
  if (n_ids < 0 || vocab <= 0 || hidden <= 0)
    return fail(HGK_ERR_ARG, "%s: bad shape n=%lld vocab=%lld hidden=%lld", fn, (long long)n_ids,
                (long long)vocab, (long long)hidden);
  if (hidden % group_size)
    return fail(HGK_ERR_ARG, "%s: hidden=%lld not a multiple of group_size=%d", fn,
                (long long)hidden, group_size);
  if (n_ids > 1 && out_row_stride < hidden)
    return fail(HGK_ERR_ARG, "%s: out row stride < hidden", fn);
  if (!ids || !w_q || !scales || !biases || !out) return fail(HGK_ERR_ARG, "%s: null pointer", fn);
  if (hidden > (1 << 24) || n_ids * hidden >= ((int64_t)1 << 40))
    return fail(HGK_ERR_UNSUPPORTED, "%s: problem too large", fn);
  if (n_ids == 0) return HGK_OK;
  QembArgs a{};
  a.ids = ids; a.ids_i32 = ids_dtype == DT_I32; a.n = n_ids; a.wq = w_q; a.sc = scales;
  a.bi = biases; a.vocab = vocab; a.wpr = (int)(hidden / 8); a.gpr = (int)(hidden / group_size);
  a.group = group_size; a.scale = out_scale; a.has_scale = out_scale != 0.0f;
  a.out = out; a.os = out_row_stride; a.hidden = hidden;
  const bool vec_ok = (reinterpret_cast<uintptr_t>(w_q) & 3u) == 0 && aligned16(out) &&
                      hidden % 8 == 0 && out_row_stride % 8 == 0;
  if (scales_dtype == DT_BF16) launch<BF16>(a, vec_ok, as_stream(stream));
  else launch<F16>(a, vec_ok, as_stream(stream));
  return launch_status(fn);
}
