// rope.hip -- RoPE (default / explicit-frequency e.g. llama3 / partial rotary,
// per-sequence offsets) with an optional fused per-head RMSNorm (Qwen3
// q_norm/k_norm), for q and k in one launch, on gfx950.
//
// Work split: a block owns `tpb` consecutive tokens (token = b*L + l) and
// every head row of q and k for those tokens.
//  phase A: the block fills an LDS table of cos/sin for its tokens x dims/2
//           frequencies (computed once per (token, frequency) and shared by all
//           heads), rounded to the activation dtype as MLX's fallback does.
//  phase B: a lane group owns one head row, in one of two layouts:
//           - two chunks per lane (rows of >= 256 bytes, full rotation):
//             LPR = head_dim/(2*V) lanes, lane j holds the rotation pair
//             (j, j+R) when j < R = dims/(2*V), else the pass-through chunks
//             (2j, 2j+1); each store instruction still covers whole lines;
//           - one chunk per lane (rows under 256 bytes): LPR =
//             head_dim/V lanes, lane j holds chunk j and fetches its rotation
//             partner j ^ R from the partner lane (DPP within a 16-lane row),
//             so every load and store instruction moves whole rows.
//           The row is read once, optionally normalised (group shuffle
//           reduction), rotated and written once to an arbitrary (b, l, h)
//           layout, which folds the [B,L,H,D] -> [B,H,L,D] transpose into the
//           store.
//
// Arithmetic (MLX CPU fallback of fast::rope, T = activation dtype):
//   pos = (f32(l) + offset_b) * scale;  th = pos * inv_freq[i]
//   c = round_T(cos th), s = round_T(sin th)
//   y1 = round_T(round_T(x1*c) - round_T(x2*s))
//   y2 = round_T(round_T(x1*s) + round_T(x2*c))
// cos/sin are evaluated in f64 and rounded to f32 (cos_sin_f32: within 3 f64
// ulps of the true values at any |th| < 2^20), then to T.
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
  uint32_t hsum_magic;  // ceil(2^32 / hsum) for hsum >= 2: r / hsum = mulhi(r, magic)
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
    float c, s;
    cos_sin_f32(pos * a.inv_freq[i], c, s);
    cs[e] = X::round(c);
    sn[e] = X::round(s);
  }
}

// Head rows a lane group keeps in flight, and a fixed tokens-per-block count
// (0: derived from the shape). Compile-time so that sweeps can rebuild with
// other values.
#ifndef HGK_ROPE_RB
#define HGK_ROPE_RB 4
#endif
#ifndef HGK_ROPE_TPB
#define HGK_ROPE_TPB 0
#endif
constexpr int kRopeBatch = HGK_ROPE_RB;

// Row r of the block's rows (token-major: tk = r / hsum, head = r % hsum).
struct RopeRow {
  int64_t xb, yb;
  int tk;
  bool isk;
};

// The q and k tensor descriptors, read once into wave-uniform registers so a
// row's q/k choice is a register select rather than a per-lane load from the
// kernel-argument segment (such loads would sit in the same in-order memory
// counter as the data loads and drain them at every wait).
struct RopePair {
  const void* x[2];
  void* y[2];
  int64_t xs0[2], xs1[2], xs2[2], ys0[2], ys1[2], ys2[2];
  int qheads;
};

__device__ inline RopePair rope_pair(const RopeArgs& a) {
  RopePair p;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    p.x[i] = a.t[i].x;
    p.y[i] = a.t[i].y;
    p.xs0[i] = a.t[i].xs0; p.xs1[i] = a.t[i].xs1; p.xs2[i] = a.t[i].xs2;
    p.ys0[i] = a.t[i].ys0; p.ys1[i] = a.t[i].ys1; p.ys2[i] = a.t[i].ys2;
  }
  p.qheads = a.t[0].heads;
  return p;
}

__device__ inline RopeRow rope_row(const RopeArgs& a, const RopePair& p, uint32_t t0, int r) {
  RopeRow o;
  o.tk = r / a.hsum;
  const int h = r - o.tk * a.hsum;
  o.isk = h >= p.qheads;
  const int hh = o.isk ? h - p.qheads : h;
  const uint32_t tok = t0 + o.tk;
  const uint32_t b = tok / a.L, l = tok - b * a.L;
  o.xb = (int64_t)b * (o.isk ? p.xs0[1] : p.xs0[0]) + (int64_t)l * (o.isk ? p.xs1[1] : p.xs1[0]) +
         (int64_t)hh * (o.isk ? p.xs2[1] : p.xs2[0]);
  o.yb = (int64_t)b * (o.isk ? p.ys0[1] : p.ys0[0]) + (int64_t)l * (o.isk ? p.ys1[1] : p.ys1[0]) +
         (int64_t)hh * (o.isk ? p.ys2[1] : p.ys2[0]);
  return o;
}

// The block's rows relative to its first token (b0, l0), for launches where
// the host has checked that every row's element offset from that token fits
// in 32 bits and that a block spans at most two sequences (L >= tokens per
// block): no division and no 64-bit multiply per row.
struct RopeBlock {
  const char* x[2];
  char* y[2];
  int32_t xs1[2], xs2[2], xw[2], ys1[2], ys2[2], yw[2];  // xw = xs0 - L*xs1 (a wrap)
  uint32_t l0;
};

template <class X>
__device__ inline RopeBlock rope_block(const RopeArgs& a, uint32_t t0) {
  RopeBlock o;
  const uint32_t b0 = t0 / a.L;
  o.l0 = t0 - b0 * a.L;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const RopeTensor& T = a.t[i];
    o.x[i] = reinterpret_cast<const char*>(T.x) + ((int64_t)b0 * T.xs0 + (int64_t)o.l0 * T.xs1) * X::kBytes;
    o.y[i] = reinterpret_cast<char*>(T.y) + ((int64_t)b0 * T.ys0 + (int64_t)o.l0 * T.ys1) * X::kBytes;
    o.xs1[i] = (int32_t)T.xs1; o.xs2[i] = (int32_t)T.xs2;
    o.xw[i] = (int32_t)(T.xs0 - (int64_t)a.L * T.xs1);
    o.ys1[i] = (int32_t)T.ys1; o.ys2[i] = (int32_t)T.ys2;
    o.yw[i] = (int32_t)(T.ys0 - (int64_t)a.L * T.ys1);
  }
  return o;
}

// Row r of the block: (token tk, head) with the element offsets of its q or
// k row from the block's first token.
struct RopeRow32 {
  int32_t xo, yo;
  int tk;
  bool isk;
};

__device__ inline RopeRow32 rope_row32(const RopeArgs& a, const RopeBlock& bb, int qheads, int r) {
  RopeRow32 o;
  o.tk = a.hsum == 1 ? r : (int)__umulhi((uint32_t)r, a.hsum_magic);
  const int h = r - o.tk * a.hsum;
  o.isk = h >= qheads;
  const int hh = o.isk ? h - qheads : h;
  const int i = o.isk ? 1 : 0;
  const bool wrap = bb.l0 + (uint32_t)o.tk >= a.L;
  o.xo = o.tk * bb.xs1[i] + hh * bb.xs2[i] + (wrap ? bb.xw[i] : 0);
  o.yo = o.tk * bb.ys1[i] + hh * bb.ys2[i] + (wrap ? bb.yw[i] : 0);
  return o;
}

template <class X, int LPR, bool NORM, bool FAST>
__global__ __launch_bounds__(256) void rope_kernel(RopeArgs a) {
  constexpr int V = Vec<X>::N;
  constexpr int RB = kRopeBatch;
  constexpr int slots = 256 / LPR;
  // the square root and division of a batch's four rows are done once per
  // quad of lanes (lane j finishes row j % 4) and broadcast by DPP
  constexpr bool SHARED = NORM && RB == 4 && LPR >= 4;
  extern __shared__ __align__(16) float smem[];
  float* cs = smem;
  float* sn = smem + a.tpb * a.half;
  const uint32_t t0 = blockIdx.x * (uint32_t)a.tpb;
  const int ntok = (int)min((uint32_t)a.tpb, a.tokens - t0);
  const int rows = ntok * a.hsum;
  const int slot = threadIdx.x / LPR;
  const int j = threadIdx.x % LPR;
  const bool rot = j < a.R;
  const int c0 = rot ? j : 2 * j;
  const int c1 = rot ? j + a.R : 2 * j + 1;

  // norm weights of q and k, packed, staged in LDS after the table ([2][D / V]
  // chunks, read per row): held in registers for the whole kernel they cost
  // the 16 VGPRs that decide between 3 and 4 waves per SIMD
  u32x4* wl = reinterpret_cast<u32x4*>(sn + a.tpb * a.half);
  const int nch = a.D / V;
  if constexpr (NORM) {
    for (int e = threadIdx.x; e < 2 * nch; e += blockDim.x) {
      const int which = e >= nch ? 1 : 0;
      const void* nw = a.t[which].nw;
      wl[e] = nw ? ld16<X>(nw, (e - which * nch) * V) : u32x4{0u, 0u, 0u, 0u};
    }
  }

  const RopePair pr = rope_pair(a);
  RopeBlock bb;
  if constexpr (FAST) bb = rope_block<X>(a, t0);
  u32x4 d0[RB], d1[RB];
  struct {
    char* y;  // the row's first output element
    int tk;
    bool isk;
  } rw[RB];
  auto load_batch = [&](int base) {
#pragma unroll
    for (int k = 0; k < RB; ++k) {
      // rows past the block's last are clamped to it (loaded, never stored)
      const int r = base + k * slots;
      const int rc = r < rows ? r : rows - 1;
      const char* xp;
      if constexpr (FAST) {
        const RopeRow32 o = rope_row32(a, bb, pr.qheads, rc);
        xp = (o.isk ? bb.x[1] : bb.x[0]) + (int64_t)o.xo * X::kBytes;
        rw[k].y = (o.isk ? bb.y[1] : bb.y[0]) + (int64_t)o.yo * X::kBytes;
        rw[k].tk = o.tk;
        rw[k].isk = o.isk;
      } else {
        const RopeRow o = rope_row(a, pr, t0, rc);
        xp = reinterpret_cast<const char*>(o.isk ? pr.x[1] : pr.x[0]) + o.xb * X::kBytes;
        rw[k].y = reinterpret_cast<char*>(o.isk ? pr.y[1] : pr.y[0]) + o.yb * X::kBytes;
        rw[k].tk = o.tk;
        rw[k].isk = o.isk;
      }
      if constexpr (LPR >= 8) {  // each load instruction reads whole 128-byte lines
        d0[k] = ld16_nt<X>(xp, c0 * V);
        d1[k] = ld16_nt<X>(xp, c1 * V);
      } else {  // half lines: the default policy keeps the line for its other half
        d0[k] = ld16<X>(xp, c0 * V);
        d1[k] = ld16<X>(xp, c1 * V);
      }
    }
  };

  // the first batch's loads go out before the block builds its table
  load_batch(slot);
  fill_table<X>(a, cs, sn, t0, ntok);
  __syncthreads();

  for (int base = slot;;) {
    // the batch's rms scales: every lane holds every row's sum; with SHARED,
    // lane j of each quad finishes row j % 4 and the quad shares the results
    float rsk[RB];
    if constexpr (NORM) {
      double ssk[RB];
#pragma unroll
      for (int k = 0; k < RB; ++k) {
        double ss = 0.0;
#pragma unroll
        for (int e = 0; e < V; ++e) {
          const double v = (double)elem<X>(d0[k], e);
          ss = __builtin_fma(v, v, ss);
        }
#pragma unroll
        for (int e = 0; e < V; ++e) {
          const double v = (double)elem<X>(d1[k], e);
          ss = __builtin_fma(v, v, ss);
        }
        ssk[k] = group_sum<LPR>(ss);
      }
      if constexpr (SHARED) {
        const int q = j & 3;
        double mine = ssk[0];
        mine = q == 1 ? ssk[1] : mine;
        mine = q == 2 ? ssk[2] : mine;
        mine = q == 3 ? ssk[3] : mine;
        const float r = rms_scale(mine, a.inv_d, a.eps);
        const int ri = __builtin_bit_cast(int, r);
        rsk[0] = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ri, 0x00, 0xF, 0xF, true));
        rsk[1] = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ri, 0x55, 0xF, 0xF, true));
        rsk[2] = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ri, 0xAA, 0xF, 0xF, true));
        rsk[3] = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, ri, 0xFF, 0xF, 0xF, true));
      } else {
#pragma unroll
        for (int k = 0; k < RB; ++k) rsk[k] = rms_scale(ssk[k], a.inv_d, a.eps);
      }
    }
#pragma unroll
    for (int k = 0; k < RB; ++k) {
      const int r = base + k * slots;
      if (r >= rows) break;
      const bool isk = rw[k].isk;
      float v0[V], v1[V];
#pragma unroll
      for (int e = 0; e < V; ++e) {
        v0[e] = elem<X>(d0[k], e);
        v1[e] = elem<X>(d1[k], e);
      }
      if constexpr (NORM) {
        const bool has = isk ? (a.t[1].nw != nullptr) : (a.t[0].nw != nullptr);
        if (has) {  // uniform across the row's lane group
          const float rs = rsk[k];
          const u32x4 wa = wl[(isk ? nch : 0) + c0], wb = wl[(isk ? nch : 0) + c1];
#pragma unroll
          for (int e = 0; e < V; e += 2) {  // roundings paired: one conversion per two
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
      }
      if (rot) {
        // y1 = round(round(x1*c) - round(x2*s)), y2 = round(round(x1*s) + round(x2*c));
        // the outer rounding happens in the store's packing conversion
        const float* cp = cs + rw[k].tk * a.half + j * V;
        const float* sp = sn + rw[k].tk * a.half + j * V;
#pragma unroll
        for (int e = 0; e < V; e += 2) {
          const float c0 = cp[e], s0 = sp[e], c1 = cp[e + 1], s1 = sp[e + 1];
          const float x10 = v0[e], x20 = v1[e], x11 = v0[e + 1], x21 = v1[e + 1];
          float a0 = x10 * c0, a1 = x11 * c1, b0 = x20 * s0, b1 = x21 * s1;
          float d0 = x10 * s0, d1 = x11 * s1, f0 = x20 * c0, f1 = x21 * c1;
          round2<X>(a0, a1);
          round2<X>(b0, b1);
          round2<X>(d0, d1);
          round2<X>(f0, f1);
          v0[e] = a0 - b0;
          v0[e + 1] = a1 - b1;
          v1[e] = d0 + f0;
          v1[e + 1] = d1 + f1;
        }
      }
      store_elems<X, V>(rw[k].y, c0 * V, v0);
      store_elems<X, V>(rw[k].y, c1 * V, v1);
    }
    base += slots * RB;
    if (base >= rows) break;
    load_batch(base);
  }
}

// The same chunk (16 bytes) of lane j ^ R, for aligned groups of 2R lanes.
// R <= 8 stays inside a 16-lane row and uses DPP; R = 4 composes the
// half-row mirror (j -> 7 - j) with a quad reversal (j -> 3 - j), which
// together map j to j ^ 4. Wider partners go through the LDS crossbar.
template <int R>
__device__ inline u32x4 xor_partner(u32x4 v) {
  u32x4 o;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int s = (int)v[k];
    int t;
    if constexpr (R == 1) t = __builtin_amdgcn_update_dpp(0, s, 0xB1, 0xF, 0xF, true);
    else if constexpr (R == 2) t = __builtin_amdgcn_update_dpp(0, s, 0x4E, 0xF, 0xF, true);
    else if constexpr (R == 4)
      t = __builtin_amdgcn_update_dpp(
          0, __builtin_amdgcn_update_dpp(0, s, 0x141, 0xF, 0xF, true), 0x1B, 0xF, 0xF, true);
    else if constexpr (R == 8) t = __builtin_amdgcn_update_dpp(0, s, 0x128, 0xF, 0xF, true);
    else t = __shfl_xor(s, R, 64);
    o[k] = (uint32_t)t;
  }
  return o;
}

// Rows a lane group of the one-chunk layout keeps in flight. At the Llama
// chain's 4096 tokens x 40 heads of 64 (4 tokens, 160 rows per block, 5 per
// lane group) 6 measured 8.91 us, 5 8.96, 8 9.21 and 4 10.79 (one call).
#ifndef HGK_ROPE_LRB
#define HGK_ROPE_LRB 6
#endif
constexpr int kRopeLaneBatch = HGK_ROPE_LRB;

// One chunk per lane: a group of LPR = head_dim / V lanes owns a head row and
// lane j holds chunk j, so each load and each store instruction moves whole
// rows (whole 128-byte lines for rows of >= 128 bytes). The rotation partner
// of chunk j < 2R is chunk j ^ R (R = dims / (2V), a power of two), fetched
// from the partner lane after the optional norm. Both halves of a pair use
// the same two rounded products: a = round(x * c), b = round(p * s), with
// y = a - b in the first half (x = x1, p = x2) and y = a + b in the second
// (x = x2, p = x1), which is y2 = round(x1 * s) + round(x2 * c) reordered.
// A row's partner lanes and norm-reduction lanes all sit in its own aligned
// group, so a group that leaves the batch early (its next row is past the
// block's last) never feeds a cross-lane move of a group still running.
template <class X, int LPR, int R, bool NORM, bool FAST>
__global__ __launch_bounds__(256) void rope_lane_kernel(RopeArgs a) {
  constexpr int V = Vec<X>::N;
  constexpr int RB = kRopeLaneBatch;
  constexpr int slots = 256 / LPR;
  static_assert(2 * R <= LPR, "rotated chunks within the row");
  extern __shared__ __align__(16) float smem[];
  float* cs = smem;
  float* sn = smem + a.tpb * a.half;
  const uint32_t t0 = blockIdx.x * (uint32_t)a.tpb;
  const int ntok = (int)min((uint32_t)a.tpb, a.tokens - t0);
  const int rows = ntok * a.hsum;
  const int slot = threadIdx.x / LPR;
  const int j = threadIdx.x % LPR;
  const bool rot = j < 2 * R;
  const bool first = j < R;
  const int f0 = (j & (R - 1)) * V;  // this lane's first frequency index

  // norm weights of q and k, packed, in LDS after the table ([2][D / V] chunks)
  u32x4* wl = reinterpret_cast<u32x4*>(sn + a.tpb * a.half);
  if constexpr (NORM) {
    for (int e = threadIdx.x; e < 2 * LPR; e += blockDim.x) {
      const int which = e >= LPR ? 1 : 0;
      const void* nw = a.t[which].nw;
      wl[e] = nw ? ld16<X>(nw, (e - which * LPR) * V) : u32x4{0u, 0u, 0u, 0u};
    }
  }

  const RopePair pr = rope_pair(a);
  RopeBlock bb;
  if constexpr (FAST) bb = rope_block<X>(a, t0);
  u32x4 d[RB];
  struct {
    char* y;
    int tk;
    bool isk;
  } rw[RB];
  auto load_batch = [&](int base) {
#pragma unroll
    for (int k = 0; k < RB; ++k) {
      const int r = base + k * slots;
      const int rc = r < rows ? r : rows - 1;
      const char* xp;
      if constexpr (FAST) {
        const RopeRow32 o = rope_row32(a, bb, pr.qheads, rc);
        xp = (o.isk ? bb.x[1] : bb.x[0]) + (int64_t)o.xo * X::kBytes;
        rw[k].y = (o.isk ? bb.y[1] : bb.y[0]) + (int64_t)o.yo * X::kBytes;
        rw[k].tk = o.tk;
        rw[k].isk = o.isk;
      } else {
        const RopeRow o = rope_row(a, pr, t0, rc);
        xp = reinterpret_cast<const char*>(o.isk ? pr.x[1] : pr.x[0]) + o.xb * X::kBytes;
        rw[k].y = reinterpret_cast<char*>(o.isk ? pr.y[1] : pr.y[0]) + o.yb * X::kBytes;
        rw[k].tk = o.tk;
        rw[k].isk = o.isk;
      }
      if constexpr (LPR * 16 >= 128) d[k] = ld16_nt<X>(xp, j * V);
      else d[k] = ld16<X>(xp, j * V);
    }
  };

  load_batch(slot);
  fill_table<X>(a, cs, sn, t0, ntok);
  __syncthreads();

  for (int base = slot;;) {
#pragma unroll
    for (int k = 0; k < RB; ++k) {
      const int r = base + k * slots;
      if (r >= rows) break;
      const bool isk = rw[k].isk;
      float v[V];
#pragma unroll
      for (int e = 0; e < V; ++e) v[e] = elem<X>(d[k], e);
      u32x4 own = d[k];
      if constexpr (NORM) {
        const bool has = isk ? (a.t[1].nw != nullptr) : (a.t[0].nw != nullptr);
        if (has) {  // uniform across the row's lane group
          double ss = 0.0;
#pragma unroll
          for (int e = 0; e < V; ++e) ss = __builtin_fma((double)v[e], (double)v[e], ss);
          ss = group_sum<LPR>(ss);
          const float rs = rms_scale(ss, a.inv_d, a.eps);
          const u32x4 w = wl[(isk ? LPR : 0) + j];
#pragma unroll
          for (int e = 0; e < V; e += 2) {
            float p0 = v[e] * rs, p1 = v[e + 1] * rs;
            round2<X>(p0, p1);
            p0 = p0 * elem<X>(w, e);
            p1 = p1 * elem<X>(w, e + 1);
            round2<X>(p0, p1);
            v[e] = p0;
            v[e + 1] = p1;
          }
          // the normalised values are representable in X: pack them exactly
          if constexpr (X::kBytes == 2) {
#pragma unroll
            for (int q = 0; q < 4; ++q) own[q] = X::pack(v[2 * q], v[2 * q + 1]);
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) own[q] = f2u(v[q]);
          }
        }
      }
      const u32x4 pt = xor_partner<R>(own);
      if (rot) {
        const float* cp = cs + rw[k].tk * a.half + f0;
        const float* sp = sn + rw[k].tk * a.half + f0;
#pragma unroll
        for (int e = 0; e < V; e += 2) {
          float a0 = v[e] * cp[e], a1 = v[e + 1] * cp[e + 1];
          float b0 = elem<X>(pt, e) * sp[e], b1 = elem<X>(pt, e + 1) * sp[e + 1];
          round2<X>(a0, a1);
          round2<X>(b0, b1);
          v[e] = first ? a0 - b0 : a0 + b0;
          v[e + 1] = first ? a1 - b1 : a1 + b1;
        }
      }
      store_elems<X, V>(rw[k].y, j * V, v);
    }
    base += slots * RB;
    if (base >= rows) break;
    load_batch(base);
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
        float c, s;
        cos_sin_f32(pos * a.inv_freq[d], c, s);
        const float cf = X::round(c), sf = X::round(s);
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


// Whether the 32-bit row offsets of rope_row32 are exact for this launch.
bool fast_index_ok(const RopeArgs& a) {
  if ((uint32_t)a.tpb > a.L || a.hsum >= 16384) return false;
  const int64_t lim = ((int64_t)1 << 31) - 1;
  for (int i = 0; i < 2; ++i) {
    const RopeTensor& T = a.t[i];
    if (T.heads == 0) continue;
    const int64_t st[2][3] = {{T.xs0, T.xs1, T.xs2}, {T.ys0, T.ys1, T.ys2}};
    for (const auto& v : st) {
      const int64_t wrap = v[0] - (int64_t)a.L * v[1];
      const int64_t span = (int64_t)a.tpb * v[1] + (int64_t)T.heads * v[2] + (wrap < 0 ? -wrap : wrap);
      if (v[1] > lim || v[2] > lim || span > lim) return false;
    }
  }
  return true;
}

template <class X, int LPR, bool NORM>
void launch_fast(RopeArgs& a, hipStream_t s) {
  // as many tokens per block as keep every lane group's rows in one batch of
  // loads, but enough blocks to fill the chip
  const int slots = 256 / LPR;
  // (stepping down one token at a time: halving from 6 to 3 at the Llama
  // chain's 4096 tokens x 40 heads measured 8% slower than 4)
  int tpb = std::max(1, std::min((slots * kRopeBatch) / a.hsum, kMaxTpb));
  while (tpb > 1 && (a.tokens + tpb - 1) / tpb < 1024u) --tpb;
  if (HGK_ROPE_TPB > 0) tpb = std::min(HGK_ROPE_TPB, kMaxTpb);
  a.tpb = tpb;
  a.hsum_magic = a.hsum >= 2 ? (uint32_t)((((uint64_t)1 << 32) + a.hsum - 1) / a.hsum) : 0u;
  const unsigned blocks = (a.tokens + tpb - 1) / tpb;
  // the cos/sin table, then the packed norm weights of q and k
  const size_t shmem = 2u * tpb * a.half * sizeof(float) + 2u * a.D * X::kBytes;
  if (fast_index_ok(a))
    HGK_LAUNCH((rope_kernel<X, LPR, NORM, true>), dim3(blocks), dim3(256), shmem, s, a);
  else
    HGK_LAUNCH((rope_kernel<X, LPR, NORM, false>), dim3(blocks), dim3(256), shmem, s, a);
}

template <class X, int LPR, int R, bool NORM>
void launch_lane(RopeArgs& a, hipStream_t s) {
  const int slots = 256 / LPR;
  int tpb = std::max(1, std::min((slots * kRopeLaneBatch) / a.hsum, kMaxTpb));
  while (tpb > 1 && (a.tokens + tpb - 1) / tpb < 1024u) --tpb;
  if (HGK_ROPE_TPB > 0) tpb = std::min(HGK_ROPE_TPB, kMaxTpb);
  a.tpb = tpb;
  a.hsum_magic = a.hsum >= 2 ? (uint32_t)((((uint64_t)1 << 32) + a.hsum - 1) / a.hsum) : 0u;
  const unsigned blocks = (a.tokens + tpb - 1) / tpb;
  const size_t shmem = 2u * tpb * a.half * sizeof(float) + 2u * a.D * X::kBytes;
  if (fast_index_ok(a))
    HGK_LAUNCH((rope_lane_kernel<X, LPR, R, NORM, true>), dim3(blocks), dim3(256), shmem, s, a);
  else
    HGK_LAUNCH((rope_lane_kernel<X, LPR, R, NORM, false>), dim3(blocks), dim3(256), shmem, s, a);
}

template <class X, int LPR, bool NORM>
bool launch_lane_r(RopeArgs& a, int R, hipStream_t s) {
  switch (R) {
    case 1: if constexpr (LPR >= 2) { launch_lane<X, LPR, 1, NORM>(a, s); return true; } break;
    case 2: if constexpr (LPR >= 4) { launch_lane<X, LPR, 2, NORM>(a, s); return true; } break;
    case 4: if constexpr (LPR >= 8) { launch_lane<X, LPR, 4, NORM>(a, s); return true; } break;
    case 8: if constexpr (LPR >= 16) { launch_lane<X, LPR, 8, NORM>(a, s); return true; } break;
    case 16: if constexpr (LPR >= 32) { launch_lane<X, LPR, 16, NORM>(a, s); return true; } break;
    case 32: if constexpr (LPR >= 64) { launch_lane<X, LPR, 32, NORM>(a, s); return true; } break;
    default: break;
  }
  return false;
}

// Which layout runs a vectorisable shape: one chunk per lane (whole-row
// loads and stores, a cross-lane move for the rotation partner) when the
// two-chunk layout's store instructions would cover less than a 128-byte line
// per row (rows under 256 bytes: at head_dim 64 in bf16 the two-chunk layout
// wrote 1.21x the output bytes to HBM, the one-chunk layout exactly 1.00x);
// else two chunks per lane, which needs no cross-lane move (at head_dim 128
// and 256 it measured 15 % and 9 % faster, and at the 64-sequence partial
// rotation of head_dim 256 also faster). HGK_ROPE_LANE = 0 / 2 forces the
// two-chunk / one-chunk layout wherever it applies (the one-chunk layout
// only for rows of up to 8 lanes).
#ifndef HGK_ROPE_LANE
#define HGK_ROPE_LANE 1
#endif

template <class X, bool NORM>
bool try_lane(RopeArgs& a, hipStream_t s) {
  constexpr int V = Vec<X>::N;
  const int lpr = a.D / V;
  const int R = a.dims / (2 * V);
  const bool narrow = a.D * X::kBytes < 256;
  if (HGK_ROPE_LANE == 0 || (HGK_ROPE_LANE == 1 && !narrow)) return false;
  switch (lpr) {  // rows under 256 bytes: at most 8 lanes
    case 2: return launch_lane_r<X, 2, NORM>(a, R, s);
    case 4: return launch_lane_r<X, 4, NORM>(a, R, s);
    case 8: return launch_lane_r<X, 8, NORM>(a, R, s);
    default: return false;
  }
}

template <class X, bool NORM>
void launch_x(RopeArgs& a, bool vec_ok, hipStream_t s) {
  constexpr int V = Vec<X>::N;
  const bool shape_ok = a.D % (2 * V) == 0 && a.dims % (2 * V) == 0;
  const int lpr = a.D / (2 * V);
  if (vec_ok && shape_ok) {
    a.R = a.dims / (2 * V);
    if (try_lane<X, NORM>(a, s)) return;
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
  HGK_LAUNCH((rope_generic_kernel<X, NORM>), dim3((unsigned)((rows + wpb - 1) / wpb)),
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
  if (B > 0 && L > 0 && qh > 0) {
    if ((st = check_strides(fn, "q", q, qs)) || (st = check_strides(fn, "q_out", qo, qos))) return st;
  }
  if (B > 0 && L > 0 && kh > 0) {
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
