// qembed.hip -- 4-bit affine QuantizedEmbedding gather + dequantize on gfx950.
//
// Table layout (MLX affine quantization, as stored in MLX 4-bit checkpoints):
//   w_q    [vocab, hidden/8]          u32, 8 codes per word, low nibble first
//   scales [vocab, hidden/group]      bf16 or f16
//   biases [vocab, hidden/group]      same dtype as scales
// One wave64 owns one token: at step s lane i reads packed word s*64 + i
// (8 codes) and writes those 8 outputs, so every load instruction reads 256
// contiguous bytes of the row and every store writes 1 KB contiguous (a lane
// owning 16 contiguous bytes of codes and 64 bytes of output measured 2.5x
// slower: each instruction then touched every line of the row). The table is
// never dequantized as a whole (QEmbedding::forward does that on every call
// in the reference).
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
  int group_shift;  // log2(group / 8): packed words per group
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

// The gather: one wave per token, through a table of the row's values.
//
// A 4-bit code takes 16 values, so each group of the row has 16 possible
// outputs. The wave first builds them -- lane g computes group g's 16 values
// with the exact element formula deq() (and the output scale), 8 pairs with
// one packed rounding each -- and writes them to its region of LDS (32 bytes
// per group). Each element is then one 16-bit LDS read at the address
// region + 32 g + 2 q: per packed word of 8 codes, two shift/and-or
// operations leave 2q in the low bits of each byte, with (g mod 8) * 32
// merged into the same bytes (the region is 256-byte aligned, so the low byte
// of an entry's address is (g mod 8) * 32 + 2q and the rest is region +
// 256 (g / 8)), and one byte permute per element splices that byte into the
// address. About 17 VALU operations per word against ~64 for computing the 8
// values directly (and the tables cost 16 values per group of 64 elements).
// Every value is the one deq() gives, for any scale, bias and output scale.
//
// At step s lane i reads packed word s*64 + i of the row (each load
// instruction of the wave reads 256 contiguous bytes) and writes its 8
// outputs with one 16-byte store (1 KB contiguous per instruction). The
// scales and biases come first (the tables need them), then the codes.
//  GSH: log2(group / 8) (words per group) when known at compile time (group
//       64: 3), else 0 and the group's shift is read from the arguments;
//  TG:  groups the wave's table region holds (64 or 256).
typedef __attribute__((address_space(3))) uint16_t lds_u16;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

constexpr int kLutWaves = 4;  // waves per workgroup

// Lane g's share of a row's table: the 16 values of groups g, g + 64, ...
// (GPL of them) from their scales and biases, written at tb + 32 g.
template <class S, int GPL>
__device__ inline void lut_build(const QembArgs& a, const uint32_t* sr, const uint32_t* br,
                                 float osc, uint32_t tb, int lane) {
#pragma unroll
  for (int j = 0; j < GPL; ++j) {
    if (64 * j >= a.gpr) break;  // uniform
    const float sv = S::lo(sr[j]), bv = S::lo(br[j]);
    uint32_t e[8];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      float p0 = (float)(2 * m) * sv, p1 = (float)(2 * m + 1) * sv;
      round2<S>(p0, p1);
      p0 += bv;
      p1 += bv;
      if (a.has_scale) {
        round2<S>(p0, p1);
        p0 *= osc;
        p1 *= osc;
      }
      e[m] = S::pack(p0, p1);
    }
    if (lane + 64 * j < a.gpr) {
      lds_u32x4* dst = (lds_u32x4*)(size_t)(tb + (uint32_t)(lane + 64 * j) * 32u);
      dst[0] = u32x4{e[0], e[1], e[2], e[3]};
      dst[1] = u32x4{e[4], e[5], e[6], e[7]};
    }
  }
  // the wave's own LDS accesses are performed in order; these keep the
  // compiler from moving the table reads above the writes
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// The 8 values of packed word wd (codes c) from the wave's table at tb:
// out[j] = values 2j, 2j + 1. sel: the permute selectors 0x07060500 | j.
template <int GSH>
__device__ inline u32x4 lut_word(uint32_t c, int wd, int gsh, uint32_t tb, const uint32_t* sel) {
  const uint32_t g = (uint32_t)wd >> (GSH ? GSH : gsh);
  const uint32_t lo8 = ((g & 7u) << 5) * 0x01010101u;
  const uint32_t hb = tb + ((g >> 3) << 8);
  const uint32_t ev = ((c << 1) & 0x1e1e1e1eu) | lo8;  // byte j: entry of code 2j
  const uint32_t od = ((c >> 3) & 0x1e1e1e1eu) | lo8;  // byte j: entry of code 2j + 1
  u32x4 o;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    u16x2 v;
    v.x = *(const lds_u16*)(size_t)__builtin_amdgcn_perm(hb, ev, sel[j]);
    v.y = *(const lds_u16*)(size_t)__builtin_amdgcn_perm(hb, od, sel[j]);
    o[j] = __builtin_bit_cast(uint32_t, v);
  }
  return o;
}

template <class S, int STEPS, int GSH, int TG>
__global__ __launch_bounds__(64 * kLutWaves) void qembed_lut_kernel(QembArgs a) {
  __shared__ __align__(256) uint16_t lut[kLutWaves][TG * 16];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x >> 6) + wv;
  if (t >= a.n) return;  // whole wave leaves together
  const int64_t id = load_id(a, t);
  const bool valid = id >= 0 && id < a.vocab;
  const int64_t row = valid ? id : 0;
  constexpr int GPL = TG / 64;  // groups per lane in the table
  uint32_t sr[GPL], br[GPL], codes[STEPS];
  const uint16_t* sc = reinterpret_cast<const uint16_t*>(a.sc) + row * a.gpr;
  const uint16_t* bi = reinterpret_cast<const uint16_t*>(a.bi) + row * a.gpr;
#pragma unroll
  for (int j = 0; j < GPL; ++j) {
    const int g = lane + 64 * j;
    const int gc = g < a.gpr ? g : a.gpr - 1;
    sr[j] = sc[gc];
    br[j] = bi[gc];
  }
  const uint32_t* wrow = a.wq + row * a.wpr;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int wd = s * 64 + lane;
    codes[s] = wrow[wd < a.wpr ? wd : a.wpr - 1];
  }
  char* obase = reinterpret_cast<char*>(a.out) + (t * a.os + (int64_t)lane * 8) * S::kBytes;
  if (!valid) {  // an id outside the table: a row of zeros (uniform over the wave)
#pragma unroll
    for (int s = 0; s < STEPS; ++s)
      if (s * 64 + lane < a.wpr)
        __builtin_nontemporal_store(u32x4{0u, 0u, 0u, 0u},
                                    reinterpret_cast<u32x4*>(obase + s * 512 * S::kBytes));
    return;
  }
  const float osc = S::round(a.scale);
  const uint32_t tb = (uint32_t)(size_t)(lds_u16*)&lut[wv][0];
  lut_build<S, GPL>(a, sr, br, osc, tb, lane);
  const int gsh = GSH ? GSH : a.group_shift;
  // byte selectors of the permute (byte j of the code bytes, then the
  // address's upper three bytes), in registers
  uint32_t sel[4] = {0x07060500u, 0x07060501u, 0x07060502u, 0x07060503u};
  asm volatile("" : "+v"(sel[0]), "+v"(sel[1]), "+v"(sel[2]), "+v"(sel[3]));
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int wd = s * 64 + lane;
    if (wd >= a.wpr) continue;
    __builtin_nontemporal_store(lut_word<GSH>(codes[s], wd, gsh, tb, sel),
                                reinterpret_cast<u32x4*>(obase + s * 512 * S::kBytes));
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

// Gather + dequantize + RMSNorm: one wave per token, as the gather. The
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
    const int g = wc >> a.group_shift;
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

// The fused form through the row's lookup table (group 64, up to 64 groups a
// row): the gather's table build and lookups give the row's values packed in
// S, then the f64 sum of squares and the norm as above.
template <class S, int STEPS, class W, class Y>
__global__ __launch_bounds__(64 * kLutWaves) void qembed_norm_lut_kernel(QembArgs a) {
  constexpr int WW = 8 * W::kBytes / 4;  // 32-bit words of weights per packed word
  __shared__ __align__(256) uint16_t lut[kLutWaves][64 * 16];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t t = (int64_t)blockIdx.x * (blockDim.x >> 6) + wv;
  if (t >= a.n) return;  // whole wave leaves together
  const int64_t id = load_id(a, t);
  const bool valid = id >= 0 && id < a.vocab;
  const int64_t row = valid ? id : 0;
  uint32_t sr[1], br[1], codes[STEPS], wr[STEPS][WW];
  {
    const int gc = lane < a.gpr ? lane : a.gpr - 1;
    sr[0] = reinterpret_cast<const uint16_t*>(a.sc)[row * a.gpr + gc];
    br[0] = reinterpret_cast<const uint16_t*>(a.bi)[row * a.gpr + gc];
  }
  const uint32_t* wrow = a.wq + row * a.wpr;
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int w = s * 64 + lane;
    const int wc = w < a.wpr ? w : a.wpr - 1;
    codes[s] = wrow[wc];
#pragma unroll
    for (int q = 0; q < WW / 4; ++q) {
      const u32x4 tw = ld16<W>(a.nw, (int64_t)wc * 8 + q * Vec<W>::N);
#pragma unroll
      for (int k = 0; k < 4; ++k) wr[s][4 * q + k] = tw[k];
    }
  }
  // h values are S values, kept packed two per word (zeros past the row and
  // for an id outside the table)
  uint32_t hp[STEPS][4];
#pragma unroll
  for (int s = 0; s < STEPS; ++s)
#pragma unroll
    for (int k = 0; k < 4; ++k) hp[s][k] = 0u;
  if (valid) {  // uniform over the wave
    const uint32_t tb = (uint32_t)(size_t)(lds_u16*)&lut[wv][0];
    lut_build<S, 1>(a, sr, br, S::round(a.scale), tb, lane);
    uint32_t sel[4] = {0x07060500u, 0x07060501u, 0x07060502u, 0x07060503u};
    asm volatile("" : "+v"(sel[0]), "+v"(sel[1]), "+v"(sel[2]), "+v"(sel[3]));
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int wd = s * 64 + lane;
      if (wd < a.wpr) {
        const u32x4 o = lut_word<3>(codes[s], wd, 3, tb, sel);
#pragma unroll
        for (int k = 0; k < 4; ++k) hp[s][k] = o[k];
      }
    }
  }
  double ss = 0.0;
#pragma unroll
  for (int s = 0; s < STEPS; ++s)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const double d0 = (double)S::lo(hp[s][k]), d1 = (double)S::hi(hp[s][k]);
      ss = __builtin_fma(d0, d0, ss);
      ss = __builtin_fma(d1, d1, ss);
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

template <class S, int GSH>
bool launch_lut(const QembArgs& a, hipStream_t s) {
  const int steps = (a.wpr + 63) / 64;
  // four waves per workgroup once there are enough tokens to fill the chip;
  // fewer tokens spread one per workgroup over more CUs
  const int wpb = a.n >= 1024 ? kLutWaves : 1;
  const dim3 g((unsigned)((a.n + wpb - 1) / wpb)), b(64 * wpb);
  const bool wide = a.gpr > 64;
  // Four-wave workgroups ask for a quarter of the CU's LDS (dynamic shared
  // memory the kernel leaves unused), so a CU holds at most four of them: 16
  // waves rather than 32. At 16384 ids of 256000 x 3584 that took 26.4 us
  // against 27.5 at 32 waves per CU, 26.7 at 20, 27.5 at 12 and 31.3 at 8:
  // fewer rows read at random at once run faster, until too few waves hide
  // the latency. (Walking several tokens per wave in a grid of that size
  // instead took 29.5 us.)
  const size_t table = (size_t)kLutWaves * (wide ? 256 : 64) * 32;
  const size_t quarter = (size_t)lds_per_cu() / kLutWaves;
  const size_t pad = wpb == kLutWaves && quarter > table ? quarter - table : 0;
  if (steps <= 1) HGK_LAUNCH((qembed_lut_kernel<S, 1, GSH, 64>), g, b, pad, s, a);
  else if (steps <= 2) HGK_LAUNCH((qembed_lut_kernel<S, 2, GSH, 64>), g, b, pad, s, a);
  else if (steps <= 4) HGK_LAUNCH((qembed_lut_kernel<S, 4, GSH, 64>), g, b, pad, s, a);
  else if (steps <= 7 && !wide) HGK_LAUNCH((qembed_lut_kernel<S, 7, GSH, 64>), g, b, pad, s, a);
  else if (steps <= 7) HGK_LAUNCH((qembed_lut_kernel<S, 7, GSH, 256>), g, b, pad, s, a);
  else if (steps <= 8 && !wide) HGK_LAUNCH((qembed_lut_kernel<S, 8, GSH, 64>), g, b, pad, s, a);
  else if (steps <= 8) HGK_LAUNCH((qembed_lut_kernel<S, 8, GSH, 256>), g, b, pad, s, a);
  else if (steps <= 16 && !wide) HGK_LAUNCH((qembed_lut_kernel<S, 16, GSH, 64>), g, b, pad, s, a);
  else if (steps <= 16 && a.gpr <= 256) HGK_LAUNCH((qembed_lut_kernel<S, 16, GSH, 256>), g, b, pad, s, a);
  else return false;
  return true;
}

template <class S>
void launch(const QembArgs& a, bool vec_ok, hipStream_t s) {
  if (vec_ok) {
    if (a.group == 64 ? launch_lut<S, 3>(a, s) : launch_lut<S, 0>(a, s)) return;
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
  if (!w_q || !scales || !biases || ((!ids || !out) && n_ids > 0))
    return fail(HGK_ERR_ARG, "%s: null pointer", fn);
  if (hidden > (1 << 24) || n_ids * hidden >= ((int64_t)1 << 40))
    return fail(HGK_ERR_UNSUPPORTED, "%s: problem too large", fn);
  if (n_ids == 0) return HGK_OK;
  QembArgs a{};
  a.ids = ids; a.ids_i32 = ids_dtype == DT_I32; a.n = n_ids; a.wq = w_q; a.sc = scales;
  a.bi = biases; a.vocab = vocab; a.wpr = (int)(hidden / 8); a.gpr = (int)(hidden / group_size);
  a.group = group_size; a.scale = out_scale; a.has_scale = out_scale != 0.0f;
  a.group_shift = group_size == 32 ? 2 : group_size == 64 ? 3 : 4;
  a.out = out; a.os = out_row_stride; a.hidden = hidden;
  const bool vec_ok = (reinterpret_cast<uintptr_t>(w_q) & 3u) == 0 && aligned16(out) &&
                      hidden % 8 == 0 && out_row_stride % 8 == 0;
  if (scales_dtype == DT_BF16) launch<BF16>(a, vec_ok, as_stream(stream));
  else launch<F16>(a, vec_ok, as_stream(stream));
  return launch_status(fn);
}

namespace hgk {
namespace {

template <class S, class W, class Y>
bool launch_norm_lut(const QembArgs& a, hipStream_t s) {
  const int steps = (a.wpr + 63) / 64;
  if (a.group != 64 || a.gpr > 64) return false;
  const int wpb = a.n >= 1024 ? kLutWaves : 1;
  const dim3 g((unsigned)((a.n + wpb - 1) / wpb)), b(64 * wpb);
  if (steps <= 1) HGK_LAUNCH((qembed_norm_lut_kernel<S, 1, W, Y>), g, b, 0, s, a);
  else if (steps <= 2) HGK_LAUNCH((qembed_norm_lut_kernel<S, 2, W, Y>), g, b, 0, s, a);
  else if (steps <= 4) HGK_LAUNCH((qembed_norm_lut_kernel<S, 4, W, Y>), g, b, 0, s, a);
  else if (steps <= 7) HGK_LAUNCH((qembed_norm_lut_kernel<S, 7, W, Y>), g, b, 0, s, a);
  else if (steps <= 8) HGK_LAUNCH((qembed_norm_lut_kernel<S, 8, W, Y>), g, b, 0, s, a);
  else return false;
  return true;
}

template <class S, class W, class Y>
bool launch_norm_fast(const QembArgs& a, hipStream_t s) {
  if (launch_norm_lut<S, W, Y>(a, s)) return true;
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
  if (!w_q || !scales || !biases || !norm_w || ((!ids || !y) && n_ids > 0))
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
  a.group_shift = group_size == 32 ? 2 : group_size == 64 ? 3 : 4;
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
