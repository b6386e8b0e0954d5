// qembed.hip -- 4-bit affine QuantizedEmbedding gather + dequantize on gfx950.
//
// Table layout (MLX affine quantization, as stored in MLX 4-bit checkpoints):
//   w_q    [vocab, hidden/8]          u32, 8 codes per word, low nibble first
//   scales [vocab, hidden/group]      bf16 or f16
//   biases [vocab, hidden/group]      same dtype as scales
// One wave64 owns one token: at step s lane i reads packed word s*64 + i
// (8 codes) and its group's scale/bias and writes those 8 outputs, so every
// load instruction reads 256 contiguous bytes of the row and every store
// writes 1 KB contiguous (a lane owning 16 contiguous bytes of codes and
// 64 bytes of output measured 2.5x slower: each instruction then touched
// every line of the row). The table is never dequantized as a whole
// (QEmbedding::forward does that on every call in the reference).
//
// Arithmetic (MLX dequantize, S = scales dtype):
//   v = round_S(round_S(q * s) + b);  optionally v = round_S(v * round_S(scale))
// which is exact to reproduce: no transcendental functions are involved.
//
// The fused form also applies the first layer's input RMSNorm to the row it
// has just built (the wave holds the whole row in registers), writing the
// embedding h (the residual stream) and y = rms_norm(h) in one pass: the
// `embed_tokens.forward(ids)` then `input_layernorm.forward(&h)` pair of
// transformer.rs:494 and 407.
#include <algorithm>
#include <cmath>

#include "../../include/higgs_hip.h"
#include "hgk_common.h"
#include "hgk_host.h"

namespace hgk {

// Dequantize with dot2 products where the row's scales and biases allow it
// (0 keeps the element-by-element form everywhere, for comparisons).
#ifndef HGK_QEMB_DOT2
#define HGK_QEMB_DOT2 1
#endif

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
  int fast_scale_ok;  // no output scale, or an output scale in [2^-19, 2^19]
  void* out;  // h (may be null in the fused form)
  int64_t os;
  int64_t hidden;
  // fused RMSNorm (qembed_norm_kernel only)
  const void* nw;
  int nwdt;
  int plus_one;
  int round_x;
  float eps;
  float inv_n;
  void* y;
  int64_t ys;
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

// The same dequantization of one packed word (8 codes, one group) from the
// packed forms, with dot2 products: a code enters as the 16-bit number
// K + q (K = 128 for bf16, 1024 for f16: two bit operations per pair of
// codes), and
//   q s         = dot2((K + q_i, K + q_i+4), (s, 0)) - K s     (exact in f32)
//   round(q s) + b = dot2(P, (1, 0)) + b                        (P = the rounded pair)
//   round(v) * o   = dot2(V, (o, 0)) - 0                        (o = the output scale)
// Each product has at most 22 significant bits and each sum is exact, so
// every value is the IEEE one before its rounding to S; the roundings are
// the packing conversions. About half the VALU work of unpacking and
// multiplying element by element. A dot2 also multiplies the pair's other
// element by zero, so every intermediate must stay finite and normal: the
// scale and bias ranges of deq_fast_ok guarantee that (bf16: 2^-100 <= |s| <
// 2^100, b = +-0 or 2^-100 <= |b| < 2^126; f16: normal |s| < 2^12, |b| <
// 2^11), the host admits positive output scales in [2^-19, 2^19] only (a
// negative one would turn a +0 element into -0 * (+0) + (+0) = +0 where the
// reference has round(+0 * o) = -0), and a negative scale beside a bias of -0
// is excluded (q = 0 would give +0 where the reference has -0). Rows with any
// other group take deq() instead.
template <class S> struct DeqK;
template <> struct DeqK<BF16> {
  static constexpr uint32_t kMagic = 0x43004300u;  // bf16 128 in each half
  static constexpr float kOff = 128.0f;
  static constexpr uint32_t kOne = 0x3f80u;
};
template <> struct DeqK<F16> {
  static constexpr uint32_t kMagic = 0x64006400u;  // f16 1024 in each half
  static constexpr float kOff = 1024.0f;
  static constexpr uint32_t kOne = 0x3c00u;
};

template <class S>
__device__ inline bool deq_fast_ok(uint32_t s16, uint32_t b16) {
  const bool neg_zero = (s16 & 0x8000u) && b16 == 0x8000u;
  if constexpr (DeqK<S>::kOff == 128.0f) {  // bf16: exponent field e, |x| ~ 2^(e - 127)
    const uint32_t se = (s16 >> 7) & 0xffu, be = (b16 >> 7) & 0xffu;
    const bool s_ok = se >= 27u && se <= 226u;
    const bool b_ok = (b16 & 0x7fffu) == 0u || (be >= 27u && be <= 252u);
    return s_ok && b_ok && !neg_zero;
  } else {  // f16: exponent field e, |x| ~ 2^(e - 15)
    const uint32_t se = (s16 >> 10) & 0x1fu, be = (b16 >> 10) & 0x1fu;
    return se >= 1u && se <= 26u && be <= 25u && !neg_zero;
  }
}

// Constants of the dot2 form, held in registers for the whole kernel (made
// once by DeqRegs::make): (1, 0) and (0, 1), the code mask and magic, and -0.
// Given 0x00003f80 as an immediate, this compiler encodes it as the inline
// constant 1.0, which the hardware reads in a dot2 as a different pair
// (measured: the product then took the high element); a three-operand
// and-or takes no literal here, so the mask and magic in registers let the
// code extraction be one v_and_or_b32.
struct DeqRegs {
  uint32_t one_lo, one_hi, mask, magic;
  float nzero;
  template <class S>
  __device__ static inline DeqRegs make() {
    DeqRegs r{DeqK<S>::kOne, DeqK<S>::kOne << 16, 0x000f000fu, DeqK<S>::kMagic, -0.0f};
    asm volatile("" : "+v"(r.one_lo), "+v"(r.one_hi), "+v"(r.mask), "+v"(r.magic), "+v"(r.nzero));
    return r;
  }
};

// One word's 8 outputs, packed in S (out[k] = elements 2k, 2k + 1); HS: the
// output scale o16 applies.
template <class S, bool HS>
__device__ inline u32x4 deq_word_fast(uint32_t c, uint32_t s16, float sv, float bv, uint32_t o16,
                                      const DeqRegs& R) {
  const uint32_t slo = s16, shi = s16 << 16, olo = o16, ohi = o16 << 16;
  const float nks = -DeqK<S>::kOff * sv;
  float v[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t q = ((c >> (4 * k)) & R.mask) | R.magic;  // codes k, k + 4
    const uint32_t p = S::pack(dot2_16<S>(q, slo, nks), dot2_16<S>(q, shi, nks));
    float v0 = dot2_16<S>(p, R.one_lo, bv), v1 = dot2_16<S>(p, R.one_hi, bv);
    if constexpr (HS) {
      const uint32_t w = S::pack(v0, v1);
      v0 = dot2_16<S>(w, olo, R.nzero);
      v1 = dot2_16<S>(w, ohi, R.nzero);
    }
    v[k] = v0;
    v[k + 4] = v1;
  }
  u32x4 o;
#pragma unroll
  for (int k = 0; k < 4; ++k) o[k] = S::pack(v[2 * k], v[2 * k + 1]);
  return o;
}

// The loads of one token's row, issued together and kept as raw words until
// used (converting a value where it is loaded would make the compiler wait for
// it step by step). At step s lane i owns packed word w = s*64 + i (8 codes,
// one group): each code load instruction of the wave reads 256 contiguous
// bytes of the row. Addresses are clamped into the row instead of predicating
// the loads, so no select has to wait on a loaded value before the next load
// issues.
//  PERM: the row's scales and biases (gpr even, gpr <= 64) come in with one
//        32-bit load per lane -- lane l < gpr/2 holds scale pair l, lane
//        gpr/2 + l bias pair l -- and each step takes its group's pair from
//        the owning lane by a cross-lane permute: 1 load instruction per row
//        instead of 2 per step (each of which read 16 useful bytes).
//  else: one 16-bit scale and bias load per step.
template <class S, int STEPS, bool PERM>
struct QembRow {
  uint32_t codes[STEPS];
  uint32_t sraw[PERM ? 1 : STEPS], braw[PERM ? 1 : STEPS];
  bool valid;

  __device__ inline void load(const QembArgs& a, int64_t t, int lane) {
    load_row(a, load_id(a, t), lane);
  }

  __device__ inline void load_row(const QembArgs& a, int64_t id, int lane) {
    valid = id >= 0 && id < a.vocab;
    const int64_t row = valid ? id : 0;
    const uint32_t* wrow = a.wq + row * a.wpr;
    const uint16_t* sc = reinterpret_cast<const uint16_t*>(a.sc) + row * a.gpr;
    const uint16_t* bi = reinterpret_cast<const uint16_t*>(a.bi) + row * a.gpr;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int w = s * 64 + lane;
      codes[s] = wrow[w < a.wpr ? w : a.wpr - 1];
    }
    if constexpr (PERM) {
      const int half = a.gpr >> 1;
      const int l = lane < a.gpr ? lane : a.gpr - 1;
      const uint16_t* p = l < half ? sc + 2 * l : bi + 2 * (l - half);
      sraw[0] = *reinterpret_cast<const uint32_t*>(p);
    } else {
#pragma unroll
      for (int s = 0; s < STEPS; ++s) {
        const int w = s * 64 + lane;
        const int g = ((w < a.wpr ? w : a.wpr - 1) * 8) / a.group;
        sraw[s] = (uint32_t)sc[g];
        braw[s] = (uint32_t)bi[g];
      }
    }
  }

  // The scale and bias of step s's group, as f32 and as their 16-bit codes.
  __device__ inline void group_affine(const QembArgs& a, int s, int lane, float& sv, float& bv,
                                      uint32_t& s16, uint32_t& b16) const {
    if constexpr (PERM) {
      const int w = s * 64 + lane;
      int g = (w * 8) / a.group;
      g = g < a.gpr ? g : a.gpr - 1;
      const uint32_t sw = (uint32_t)__shfl((int)sraw[0], g >> 1);
      const uint32_t bw = (uint32_t)__shfl((int)sraw[0], (a.gpr >> 1) + (g >> 1));
      s16 = (g & 1) ? sw >> 16 : sw & 0xffffu;
      b16 = (g & 1) ? bw >> 16 : bw & 0xffffu;
    } else {
      s16 = sraw[s] & 0xffffu;
      b16 = braw[s] & 0xffffu;
    }
    sv = S::lo(s16);
    bv = S::lo(b16);
  }

  // Whether every group of the row takes deq_word_fast (uniform over the
  // wave; PERM rows only, whose lanes hold all of the row's scales and biases).
  __device__ inline bool fast_row(const QembArgs& a, int lane) const {
    if constexpr (PERM) {
      const int half = a.gpr >> 1;
      // lane l < half holds scale pair l; its biases are in lane half + l
      const uint32_t bw = (uint32_t)__shfl((int)sraw[0], (lane < half ? lane : 0) + half);
      bool ok = true;
      if (lane < half)
        ok = deq_fast_ok<S>(sraw[0] & 0xffffu, bw & 0xffffu) && deq_fast_ok<S>(sraw[0] >> 16, bw >> 16);
      return __builtin_amdgcn_ballot_w64(!ok) == 0;
    } else {
      return false;
    }
  }
};

// Persistent waves over the tokens (wave w takes tokens w, w + W, w + 2W, ...
// for W waves in the grid, sized to what the chip holds resident), software
// pipelined: the next token's loads are issued before the current token's
// row is dequantized and stored, so every wave keeps one row of reads in
// flight under its stores. Each store writes 1 KB contiguous.
template <class S, int STEPS, bool PERM>
__global__ __launch_bounds__(256) void qembed_kernel(QembArgs a) {
  const int lane = threadIdx.x & 63;
  const int wpb = blockDim.x >> 6;
  const int64_t nw = (int64_t)gridDim.x * wpb;
  int64_t t = (int64_t)blockIdx.x * wpb + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (t >= a.n) return;  // whole wave leaves together
  const float osc = S::round(a.scale);
  const uint32_t o16 = S::pack(osc, 0.0f) & 0xffffu;
  const DeqRegs R = DeqRegs::make<S>();
  QembRow<S, STEPS, PERM> cur, nxt;
  cur.load(a, t, lane);
  for (;;) {
    const int64_t tn = t + nw;
    const bool more = tn < a.n;
    if (more) nxt.load(a, tn, lane);
    const bool fast = HGK_QEMB_DOT2 && a.fast_scale_ok && cur.fast_row(a, lane);
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      float sv, bv;
      uint32_t s16, b16;
      cur.group_affine(a, s, lane, sv, bv, s16, b16);  // (a permute: every lane takes part)
      const int w = s * 64 + lane;
      if (w >= a.wpr) continue;
      char* op = reinterpret_cast<char*>(a.out) + (t * a.os + (int64_t)w * 8) * S::kBytes;
      if (fast) {
        u32x4 o = a.has_scale ? deq_word_fast<S, true>(cur.codes[s], s16, sv, bv, o16, R)
                              : deq_word_fast<S, false>(cur.codes[s], s16, sv, bv, o16, R);
        if (!cur.valid) o = u32x4{0u, 0u, 0u, 0u};
        __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(op));
        continue;
      }
      float v[8];
#pragma unroll
      for (int nib = 0; nib < 8; ++nib) {
        const uint32_t q = (cur.codes[s] >> (4 * nib)) & 0xfu;
        float x = deq<S>(q, sv, bv);
        x = a.has_scale ? S::round(x * osc) : x;
        v[nib] = cur.valid ? x : 0.0f;
      }
      store_elems<S, 8>(a.out, t * a.os + (int64_t)w * 8, v);
    }
    if (!more) break;
    t = tn;
    cur = nxt;
  }
}

// Many tokens (at least four per wave over half the resident waves): TPW
// tokens per wave, t = w + k * W for W waves; lane k fetches token k's id, and
// every one of the wave's TPW rows is loaded before the first row is stored,
// so the wave keeps TPW rows of reads in flight (with one token in flight per
// wave, the reads of 16384 random rows come back too slowly to keep the write
// stream busy).
template <class S, int STEPS, int TPW, bool HS>
__global__ __launch_bounds__(256) void qembed_rows_kernel(QembArgs a, int64_t nwaves) {
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * (blockDim.x >> 6) +
                    __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (w >= nwaves) return;  // whole wave leaves together
  int64_t id = 0;
  {
    int64_t t = w + (int64_t)(lane < TPW ? lane : TPW - 1) * nwaves;
    t = t < a.n ? t : a.n - 1;
    id = load_id(a, t);
  }
  const float osc = S::round(a.scale);
  const uint32_t o16 = S::pack(osc, 0.0f) & 0xffffu;
  const DeqRegs R = DeqRegs::make<S>();
  QembRow<S, STEPS, true> rows[TPW];
#pragma clang loop unroll(full)
  for (int k = 0; k < TPW; ++k) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)id, k);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)id >> 32), k);
    rows[k].load_row(a, (int64_t)(((uint64_t)hi << 32) | lo), lane);
  }
#pragma clang loop unroll(full)
  for (int k = 0; k < TPW; ++k) {
    const int64_t t = w + (int64_t)k * nwaves;
    const bool live = t < a.n;  // uniform over the wave
    const QembRow<S, STEPS, true>& cur = rows[k];
    if (!cur.valid) {  // an id outside the table: a row of zeros (uniform over the wave)
#pragma clang loop unroll(full)
      for (int s = 0; s < STEPS; ++s) {
        const int wd = s * 64 + lane;
        if (live && wd < a.wpr)
          __builtin_nontemporal_store(u32x4{0u, 0u, 0u, 0u},
                                      reinterpret_cast<u32x4*>(reinterpret_cast<char*>(a.out) +
                                                               (t * a.os + (int64_t)wd * 8) * S::kBytes));
      }
      continue;
    }
    const bool fast = HGK_QEMB_DOT2 && a.fast_scale_ok && cur.fast_row(a, lane);
#pragma clang loop unroll(full)
    for (int s = 0; s < STEPS; ++s) {
      float sv, bv;
      uint32_t s16, b16;
      cur.group_affine(a, s, lane, sv, bv, s16, b16);  // (a permute: every lane takes part)
      const int wd = s * 64 + lane;
      if (!live || wd >= a.wpr) continue;
      char* op = reinterpret_cast<char*>(a.out) + (t * a.os + (int64_t)wd * 8) * S::kBytes;
      if (fast) {
        const u32x4 o = deq_word_fast<S, HS>(cur.codes[s], s16, sv, bv, o16, R);
        __builtin_nontemporal_store(o, reinterpret_cast<u32x4*>(op));
        continue;
      }
      float v[8];
#pragma unroll
      for (int nib = 0; nib < 8; ++nib) {
        const uint32_t q = (cur.codes[s] >> (4 * nib)) & 0xfu;
        float x = deq<S>(q, sv, bv);
        x = HS ? S::round(x * osc) : x;
        v[nib] = x;
      }
      store_elems<S, 8>(a.out, t * a.os + (int64_t)wd * 8, v);
    }
  }
}

// Any layout: one output element per thread per pass of a grid-stride loop
// (the grid is capped, so any element count launches).
template <class S>
__global__ __launch_bounds__(256) void qembed_generic_kernel(QembArgs a) {
  const int64_t total = a.n * a.hidden;
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += stride) {
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
}

// Gather + dequantize + RMSNorm: one wave per token, as qembed_kernel. The
// row's values are kept packed in S (they are exactly S values) while the f64
// sum of squares is reduced across the wave; the norm weights (W = S or f32)
// are loaded with the codes. Computation type T = promote(S, w'), as in
// rms_norm_kernel; Y is S or f32.
template <class S, int STEPS, class W, class Y>
__global__ __launch_bounds__(256) void qembed_norm_kernel(QembArgs a) {
  constexpr int WW = 8 * W::kBytes / 4;  // 32-bit words of weights per packed word
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
  const uint16_t* sc = reinterpret_cast<const uint16_t*>(a.sc);
  const uint16_t* bi = reinterpret_cast<const uint16_t*>(a.bi);

  uint32_t codes[STEPS], sraw[STEPS], braw[STEPS], wr[STEPS][WW];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int w = s * 64 + lane;
    const int wc = w < a.wpr ? w : a.wpr - 1;
    const int g = (wc * 8) / a.group;
    codes[s] = wrow[wc];
    sraw[s] = (uint32_t)sc[grow + g];
    braw[s] = (uint32_t)bi[grow + g];
#pragma unroll
    for (int q = 0; q < WW / 4; ++q) {
      const u32x4 tw = ld16<W>(a.nw, (int64_t)wc * 8 + q * Vec<W>::N);
#pragma unroll
      for (int k = 0; k < 4; ++k) wr[s][4 * q + k] = tw[k];
    }
  }
  // dequantize; h values are S values, kept packed two per word
  uint32_t hp[STEPS][4];
  double ss = 0.0;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const float sv = S::lo(sraw[s]), bv = S::lo(braw[s]);
    const bool own = s * 64 + lane < a.wpr;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float v[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const uint32_t q = (codes[s] >> (4 * (2 * k + e))) & 0xfu;
        float x = deq<S>(q, sv, bv);
        x = a.has_scale ? S::round(x * osc) : x;
        v[e] = (valid && own) ? x : 0.0f;
        ss = __builtin_fma((double)v[e], (double)v[e], ss);
      }
      hp[s][k] = S::pack(v[0], v[1]);
    }
  }
  ss = group_sum<64>(ss);
  const float rr = rms_scale(ss, a.inv_n, a.eps);
  const bool rx = a.round_x != 0;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int w = s * 64 + lane;
    if (w >= a.wpr) continue;
    if (a.out) {
      u32x4 hv;
#pragma unroll
      for (int k = 0; k < 4; ++k) hv[k] = hp[s][k];
      __builtin_nontemporal_store(
          hv, reinterpret_cast<u32x4*>(reinterpret_cast<char*>(a.out) +
                                       (t * a.os + (int64_t)w * 8) * S::kBytes));
    }
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      float n0 = S::lo(hp[s][e / 2]) * rr, n1 = S::hi(hp[s][e / 2]) * rr;
      if (rx) round2<S>(n0, n1);
      float w0 = elem<W>(wr[s], e), w1 = elem<W>(wr[s], e + 1);
      if (a.plus_one) {
        w0 = w0 + 1.0f;
        w1 = w1 + 1.0f;
      }
      n0 = n0 * w0;
      n1 = n1 * w1;
      if constexpr (Y::kCode != S::kCode) {
        if (rx) round2<S>(n0, n1);
      }
      o[e] = n0;
      o[e + 1] = n1;
    }
    store_elems<Y, 8>(a.y, t * a.ys + (int64_t)w * 8, o);
  }
}

// Fused form, any layout: one wave per token, two passes (the second
// dequantizes again), element-strided.
template <class S, class Y>
__global__ __launch_bounds__(256) void qembed_norm_generic_kernel(QembArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= a.n) return;  // whole wave leaves together
  const int64_t id = load_id(a, t);
  const bool valid = id >= 0 && id < a.vocab;
  auto value = [&](int64_t k) {
    if (!valid) return 0.0f;
    const uint32_t q = (a.wq[id * a.wpr + k / 8] >> (4 * (k % 8))) & 0xfu;
    const int64_t g = id * a.gpr + k / a.group;
    float x = deq<S>(q, load1<S>(a.sc, g), load1<S>(a.bi, g));
    return a.has_scale ? S::round(x * S::round(a.scale)) : x;
  };
  double ss = 0.0;
  for (int64_t k = lane; k < a.hidden; k += 64) {
    const double v = (double)value(k);
    ss = __builtin_fma(v, v, ss);
  }
  ss = group_sum<64>(ss);
  const float rr = rms_scale(ss, a.inv_n, a.eps);
  for (int64_t k = lane; k < a.hidden; k += 64) {
    const float hv = value(k);
    if (a.out) store1<S>(a.out, t * a.os + k, hv);
    float nv = hv * rr;
    nv = a.round_x ? S::round(nv) : nv;
    float we = load1_dt(a.nw, a.nwdt, k);
    we = a.plus_one ? we + 1.0f : we;
    nv = nv * we;
    nv = a.round_x ? S::round(nv) : nv;
    store1<Y>(a.y, t * a.ys + k, nv);
  }
}

namespace {

template <class S, int TPW, bool HS>
void launch_rows(const QembArgs& a, int steps, hipStream_t s) {
  const int64_t nwaves = (a.n + TPW - 1) / TPW;
  const dim3 g((unsigned)((nwaves + 3) / 4)), b(256);
  if (steps <= 1) HGK_LAUNCH((qembed_rows_kernel<S, 1, TPW, HS>), g, b, 0, s, a, nwaves);
  else if (steps <= 2) HGK_LAUNCH((qembed_rows_kernel<S, 2, TPW, HS>), g, b, 0, s, a, nwaves);
  else if (steps <= 4) HGK_LAUNCH((qembed_rows_kernel<S, 4, TPW, HS>), g, b, 0, s, a, nwaves);
  else if (steps <= 7) HGK_LAUNCH((qembed_rows_kernel<S, 7, TPW, HS>), g, b, 0, s, a, nwaves);
  else HGK_LAUNCH((qembed_rows_kernel<S, 8, TPW, HS>), g, b, 0, s, a, nwaves);
}

template <class S, bool PERM>
void launch_fast(const QembArgs& a, int steps, hipStream_t s) {
  // waves: one per token up to what the chip keeps resident (8 per SIMD)
  const int wpb = a.n >= 1024 ? 4 : 1;
  const int64_t waves = std::min<int64_t>(a.n, (int64_t)resident_waves());
  const dim3 g((unsigned)((waves + wpb - 1) / wpb)), b(64 * wpb);
  if (steps <= 1) HGK_LAUNCH((qembed_kernel<S, 1, PERM>), g, b, 0, s, a);
  else if (steps <= 2) HGK_LAUNCH((qembed_kernel<S, 2, PERM>), g, b, 0, s, a);
  else if (steps <= 4) HGK_LAUNCH((qembed_kernel<S, 4, PERM>), g, b, 0, s, a);
  else if (steps <= 7) HGK_LAUNCH((qembed_kernel<S, 7, PERM>), g, b, 0, s, a);
  else if (steps <= 8) HGK_LAUNCH((qembed_kernel<S, 8, PERM>), g, b, 0, s, a);
  else HGK_LAUNCH((qembed_kernel<S, 16, PERM>), g, b, 0, s, a);
}

template <class S>
void launch(const QembArgs& a, bool vec_ok, bool perm_ok, hipStream_t s) {
  const int steps = (a.wpr + 63) / 64;
  // four rows in flight per wave where that still leaves half the resident
  // waves (measured at 16384 tokens of 256000 x 3584: 6 % faster than one
  // token in flight; at 4096 tokens, with 1024 waves, 45 % slower)
  if (vec_ok && perm_ok && steps <= 8 && a.n >= 2 * (int64_t)resident_waves()) {
    if (a.has_scale) launch_rows<S, 4, true>(a, steps, s);
    else launch_rows<S, 4, false>(a, steps, s);
    return;
  }
  if (vec_ok && steps <= 16) {
    if (perm_ok) launch_fast<S, true>(a, steps, s);
    else launch_fast<S, false>(a, steps, s);
    return;
  }
  const int64_t blocks = std::min<int64_t>((a.n * a.hidden + 255) / 256, (int64_t)1 << 20);
  HGK_LAUNCH((qembed_generic_kernel<S>), dim3((unsigned)blocks), dim3(256), 0, s, a);
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
  // the dot2 form takes positive output scales in [2^-19, 2^19]: every
  // product stays normal, and no +0 element changes sign (a negative scale
  // takes the element-by-element form, which gives the reference's -0)
  a.fast_scale_ok = !a.has_scale || (out_scale >= 0x1p-19f && out_scale <= 0x1p19f);
  a.out = out; a.os = out_row_stride; a.hidden = hidden;
  const bool vec_ok = (reinterpret_cast<uintptr_t>(w_q) & 3u) == 0 && aligned16(out) &&
                      hidden % 8 == 0 && out_row_stride % 8 == 0;
  // one 32-bit load per lane brings a row's scales and biases when they fit
  // one register across the wave and every row's pairs are 4-byte aligned
  const bool perm_ok = a.gpr % 2 == 0 && a.gpr <= 64 &&
                       ((reinterpret_cast<uintptr_t>(scales) | reinterpret_cast<uintptr_t>(biases)) & 3u) == 0;
  if (scales_dtype == DT_BF16) launch<BF16>(a, vec_ok, perm_ok, as_stream(stream));
  else launch<F16>(a, vec_ok, perm_ok, as_stream(stream));
  return launch_status(fn);
}

namespace hgk {
namespace {

template <class S, class W, class Y>
bool launch_norm_fast(const QembArgs& a, hipStream_t s) {
  const int steps = (a.wpr + 63) / 64;
  const int wpb = a.n >= 1024 ? 4 : 1;
  const dim3 g((unsigned)((a.n + wpb - 1) / wpb)), b(64 * wpb);
  if (steps <= 1) HGK_LAUNCH((qembed_norm_kernel<S, 1, W, Y>), g, b, 0, s, a);
  else if (steps <= 2) HGK_LAUNCH((qembed_norm_kernel<S, 2, W, Y>), g, b, 0, s, a);
  else if (steps <= 4) HGK_LAUNCH((qembed_norm_kernel<S, 4, W, Y>), g, b, 0, s, a);
  else if (steps <= 7) HGK_LAUNCH((qembed_norm_kernel<S, 7, W, Y>), g, b, 0, s, a);
  else if (steps <= 8) HGK_LAUNCH((qembed_norm_kernel<S, 8, W, Y>), g, b, 0, s, a);
  else if (steps <= 16) HGK_LAUNCH((qembed_norm_kernel<S, 16, W, Y>), g, b, 0, s, a);
  else return false;
  return true;
}

template <class S, class Y>
void launch_norm(const QembArgs& a, bool vec_ok, hipStream_t s) {
  if (vec_ok) {
    if (a.nwdt == S::kCode && launch_norm_fast<S, S, Y>(a, s)) return;
    if (a.nwdt == DT_F32 && launch_norm_fast<S, F32, Y>(a, s)) return;
  }
  const int wpb = a.n >= 1024 ? 4 : 1;
  HGK_LAUNCH((qembed_norm_generic_kernel<S, Y>), dim3((unsigned)((a.n + wpb - 1) / wpb)),
             dim3(64 * wpb), 0, s, a);
}

}  // namespace
}  // namespace hgk

extern "C" int hgk_quantized_embedding_rms_norm(
    const void* ids, int ids_dtype, int64_t n_ids, const uint32_t* w_q, const void* scales,
    const void* biases, int scales_dtype, int64_t vocab, int64_t hidden, int group_size, int bits,
    float out_scale, void* h, int64_t h_row_stride, const void* norm_w, int norm_w_dtype,
    int w_plus_one, float eps, void* y, int y_dtype, int64_t y_row_stride, void* stream) {
  clear_error();
  const char* fn = "hgk_quantized_embedding_rms_norm";
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
  if (n_ids > 1 && ((h && h_row_stride < hidden) || y_row_stride < hidden))
    return fail(HGK_ERR_ARG, "%s: h/y row stride < hidden", fn);
  if (!ids || !w_q || !scales || !biases || !norm_w || !y)
    return fail(HGK_ERR_ARG, "%s: null pointer", fn);
  if (!is_float_dtype(norm_w_dtype) || !is_float_dtype(y_dtype))
    return fail(HGK_ERR_ARG, "%s: norm weight / y dtype must be f32, bf16 or f16", fn);
  if (!(eps >= 0.0f)) return fail(HGK_ERR_ARG, "%s: eps must be >= 0", fn);
  if (hidden > (1 << 24) || n_ids * hidden >= ((int64_t)1 << 40))
    return fail(HGK_ERR_UNSUPPORTED, "%s: problem too large", fn);
  const int w_eff = w_plus_one ? DT_F32 : norm_w_dtype;
  const int t_out = promote(scales_dtype, w_eff);
  if (t_out != scales_dtype && t_out != DT_F32)
    return fail(HGK_ERR_UNSUPPORTED, "%s: computation type %s not implemented", fn,
                dtype_name(t_out));
  if (y_dtype != scales_dtype && y_dtype != DT_F32)
    return fail(HGK_ERR_UNSUPPORTED, "%s: y dtype must be the scales dtype or f32", fn);
  if (n_ids == 0) return HGK_OK;
  QembArgs a{};
  a.ids = ids; a.ids_i32 = ids_dtype == DT_I32; a.n = n_ids; a.wq = w_q; a.sc = scales;
  a.bi = biases; a.vocab = vocab; a.wpr = (int)(hidden / 8); a.gpr = (int)(hidden / group_size);
  a.group = group_size; a.scale = out_scale; a.has_scale = out_scale != 0.0f;
  a.out = h; a.os = h_row_stride; a.hidden = hidden;
  a.nw = norm_w; a.nwdt = norm_w_dtype; a.plus_one = w_plus_one ? 1 : 0;
  a.round_x = t_out == scales_dtype ? 1 : 0; a.eps = eps; a.inv_n = (float)(1.0 / (double)hidden);
  a.y = y; a.ys = y_row_stride;
  const bool vec_ok = (reinterpret_cast<uintptr_t>(w_q) & 3u) == 0 && hidden % 8 == 0 &&
                      (!h || (aligned16(h) && h_row_stride % 8 == 0)) && aligned16(y) &&
                      (y_row_stride * dtype_bytes(y_dtype)) % 16 == 0 && aligned16(norm_w);
  const hipStream_t st = as_stream(stream);
  if (scales_dtype == DT_BF16) {
    if (y_dtype == DT_BF16) launch_norm<BF16, BF16>(a, vec_ok, st);
    else launch_norm<BF16, F32>(a, vec_ok, st);
  } else {
    if (y_dtype == DT_F16) launch_norm<F16, F16>(a, vec_ok, st);
    else launch_norm<F16, F32>(a, vec_ok, st);
  }
  return launch_status(fn);
}
