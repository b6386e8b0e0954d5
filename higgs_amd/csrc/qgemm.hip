// qgemm.hip -- quantized_matmul(x, w, scales, biases, transpose = true, 64, 4)
// on gfx950 MFMA: QLinear::forward (crates/higgs-models/src/qwen3_next.rs:
// 174-221), y[m, n] = sum_k x[m, k] * (s[n, k/64] * q[n, k] + b[n, k/64]),
// with w [N, K/8] u32 (8 codes per word, low nibble first) and scales/biases
// [N, K/64] in the activation dtype (bf16).
//
// Three kernels: the exact-product kernel below (M <= 512), the decode kernel
// for M <= 64 with K a multiple of 512 and the hi/lo-plane kernel for M > 512
// (further down).
//
// Exact products, one group at a time. A code q enters the matrix core as
// the bf16 number 128 + q (two bit operations per pair of codes), x as
// itself, so every product x * (128 + q) is exact and the MFMA sums them in
// f32. Per 64-code group g the block has C_g[m, n] = sum x (128 + q) and the
// row sums Sx_g[m] = sum x, and the affine part is applied once per group in
// f32:   acc += s[n, g] * C_g + (b[n, g] - 128 s[n, g]) * Sx_g[m].
// No weight is ever rounded to bf16, so the result is the exact contraction
// up to f32 summation error, rounded to bf16 once at the end.
//
// Layout: a block computes BM x 128 of y with 4 waves (2 x 2), each a
// (BM/2) x 64 tile of 16 x 16 MFMA tiles (v_mfma_f32_16x16x32_bf16: lane l
// supplies row l%16 of A and column l%16 of B, 8 k-values each; it receives
// rows 4(l/16)+r of column l%16). The k-order inside an MFMA is free as long
// as A and B agree: lane group j = l/16 supplies, for the two MFMAs of a
// group, words 2j and 2j+1 of the group's 8 code words (16 consecutive k).
// So a lane's B operand is read straight from global memory as one 8-byte
// load per column and group (no LDS), and x is staged in LDS as it is,
// together with its per-group row sums (dot products with ones). The x tile
// is double-buffered in LDS (one barrier per group) and the next group's x,
// codes, scales and biases are loaded while the current group's MFMAs run.
#include "../../include/higgs_hip.h"
#include "hgk_act.h"
#include "hgk_common.h"
#include "hgk_host.h"
#include "qgemm.h"

namespace hgk {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));


constexpr int kQgBN = 128;   // output columns per block
constexpr int kQgPitch = 72; // LDS row pitch of the x tile (64 + 8 elements)
constexpr int kCUs = 256;     // compute units of an MI355X

// 8 codes of one word (code i at bits 4i) -> the 8 bf16 values 128 + q_i in
// order: the low and high nibbles of each byte are split apart, v_perm_b32
// pairs byte j of each into one word, and the exponent bits of 128 are OR-ed
// in.
__device__ inline bf16x8_t expand_codes(uint32_t c) {
  const uint32_t lo = c & 0x0f0f0f0fu;          // q0 q2 q4 q6
  const uint32_t hi = (c >> 4) & 0x0f0f0f0fu;   // q1 q3 q5 q7
  u32x4 v;
  v[0] = __builtin_amdgcn_perm(hi, lo, 0x0c040c00u) | 0x43004300u;  // (q0, q1)
  v[1] = __builtin_amdgcn_perm(hi, lo, 0x0c050c01u) | 0x43004300u;  // (q2, q3)
  v[2] = __builtin_amdgcn_perm(hi, lo, 0x0c060c02u) | 0x43004300u;  // (q4, q5)
  v[3] = __builtin_amdgcn_perm(hi, lo, 0x0c070c03u) | 0x43004300u;  // (q6, q7)
  return __builtin_bit_cast(bf16x8_t, v);
}

// 8 codes of one word -> the bf16 numbers 128 + q in the order (q0, q4),
// (q1, q5), (q2, q6), (q3, q7): for x stored in the same order, each pair is
// one shift and one and-or (7 operations per word against 11 above).
// The two masks are passed in registers (x4_masks): a three-operand and-or
// takes no literal on this target, and with literals the compiler splits it
// into a separate and and or.
struct X4Masks {
  uint32_t nib, one;  // 0x000f000f, 0x43004300
};
__device__ inline X4Masks x4_masks() {
  X4Masks m{0x000f000fu, 0x43004300u};
  asm volatile("" : "+v"(m.nib), "+v"(m.one));
  return m;
}
__device__ inline bf16x8_t expand_codes_x4(uint32_t c, X4Masks m) {
  u32x4 v;
  v[0] = (c & m.nib) | m.one;
  v[1] = ((c >> 4) & m.nib) | m.one;
  v[2] = ((c >> 8) & m.nib) | m.one;
  v[3] = ((c >> 12) & m.nib) | m.one;
  return __builtin_bit_cast(bf16x8_t, v);
}

// A 16-byte piece of 8 bf16 values (x0 .. x7) reordered to (x0, x4),
// (x1, x5), (x2, x6), (x3, x7), the order expand_codes_x4 gives the codes.
__device__ inline u32x4 order_x4(u32x4 w) {
  u32x4 v;
  v[0] = __builtin_amdgcn_perm(w[2], w[0], 0x05040100u);
  v[1] = __builtin_amdgcn_perm(w[2], w[0], 0x07060302u);
  v[2] = __builtin_amdgcn_perm(w[3], w[1], 0x05040100u);
  v[3] = __builtin_amdgcn_perm(w[3], w[1], 0x07060302u);
  return v;
}

typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));

__device__ inline float dot2_ones(uint32_t w, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, w),
                                         __builtin_bit_cast(bf16x2_v, 0x3f803f80u), c, false);
}

// Sum of the 8 bf16 values of a 16-byte piece: four dot products with (1, 1).
// The words are taken out of the vector one by one into plain registers
// first (with the vector element feeding the builtin directly, this compiler
// read the first word four times).
__device__ inline float sum8_bf16(u32x4 v) {
  uint32_t w0 = v[0], w1 = v[1], w2 = v[2], w3 = v[3];
  asm volatile("" : "+v"(w0), "+v"(w1), "+v"(w2), "+v"(w3));
  float s = dot2_ones(w0, 0.0f);
  s = dot2_ones(w1, s);
  s = dot2_ones(w2, s);
  return dot2_ones(w3, s);
}

// Sum over the 8 lanes of a DPP half-row.
__device__ inline float sum8_lanes(float v) {
  v += u2f((uint32_t)__builtin_amdgcn_update_dpp(0, (int)f2u(v), 0xB1, 0xF, 0xF, true));
  v += u2f((uint32_t)__builtin_amdgcn_update_dpp(0, (int)f2u(v), 0x4E, 0xF, 0xF, true));
  v += u2f((uint32_t)__builtin_amdgcn_update_dpp(0, (int)f2u(v), 0x141, 0xF, 0xF, true));
  return v;
}

template <int BM>
__global__ __launch_bounds__(256) void qgemm_kernel(QgemmArgs a) {
  constexpr int MT = BM / 32;          // 16-row MFMA tiles per wave
  constexpr int NT = 4;                // 16-column MFMA tiles per wave
  constexpr int XCH = BM * 8 / 256;    // 16-byte x chunks per thread per group
  static_assert(XCH >= 1, "BM >= 32");
  __shared__ __align__(16) uint16_t xs[2][BM][kQgPitch];
  __shared__ __align__(16) float sx[2][BM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l16 = lane & 15, lg = lane >> 4;
  const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * kQgBN;
  const int KW = (int)(a.K / 8), G = (int)(a.K / 64);

  // this thread's x chunks: chunk c = tid + 256 i -> row c / 8, word c % 8
  const uint16_t* xrow[XCH];
#pragma unroll
  for (int i = 0; i < XCH; ++i) {
    const int64_t r = m0 + (tid + 256 * i) / 8;
    xrow[i] = a.x + (r < a.M ? r : a.M - 1) * a.xs + ((tid + 256 * i) & 7) * 8;
  }
  // this lane's weight columns (one per 16-column tile)
  const uint32_t* wcol[NT];
  const uint16_t* scol[NT];
  const uint16_t* bcol[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int64_t n = n0 + wn * 64 + t * 16 + l16;
    const int64_t nc = n < a.N ? n : a.N - 1;
    wcol[t] = a.w + nc * KW + 2 * lg;
    scol[t] = a.sc + nc * G;
    bcol[t] = a.bi + nc * G;
  }

  u32x4 xr[XCH];
  u32x2_t wr[NT];
  uint32_t sr[NT], br[NT];
  auto fetch = [&](int g) {
#pragma unroll
    for (int i = 0; i < XCH; ++i) xr[i] = *reinterpret_cast<const u32x4*>(xrow[i] + g * 64);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      wr[t] = *reinterpret_cast<const u32x2_t*>(wcol[t] + g * 8);
      sr[t] = scol[t][g];
      br[t] = bcol[t][g];
    }
  };

  f32x4_t acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[i][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  fetch(0);
  for (int g = 0; g < G; ++g) {
    const int buf = g & 1;
    // publish this group's x (permuted) and its row sums
#pragma unroll
    for (int i = 0; i < XCH; ++i) {
      const int c = tid + 256 * i;
      *reinterpret_cast<u32x4*>(&xs[buf][c / 8][(c & 7) * 8]) = xr[i];
      const float s8 = sum8_lanes(sum8_bf16(xr[i]));
      if ((c & 7) == 0) sx[buf][c / 8] = s8;
    }
    // this group's codes, scales and biases stay in registers for the MFMAs
    bf16x8_t bw[NT][2];
    float s[NT], bp[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      bw[t][0] = expand_codes(wr[t][0]);
      bw[t][1] = expand_codes(wr[t][1]);
      s[t] = BF16::lo(sr[t]);
      bp[t] = BF16::lo(br[t]) - 128.0f * s[t];
    }
    __syncthreads();
    if (g + 1 < G) fetch(g + 1);

#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int row = wm * (BM / 2) + i * 16;
      const bf16x8_t a0 = *reinterpret_cast<const bf16x8_t*>(&xs[buf][row + l16][(2 * lg) * 8]);
      const bf16x8_t a1 = *reinterpret_cast<const bf16x8_t*>(&xs[buf][row + l16][(2 * lg + 1) * 8]);
      const f32x4_t sxr = *reinterpret_cast<const f32x4_t*>(&sx[buf][row + 4 * lg]);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        f32x4_t c = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bw[t][0], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bw[t][1], c, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc[i][t][r] = __builtin_fmaf(s[t], c[r], __builtin_fmaf(bp[t], sxr[r], acc[i][t][r]));
      }
    }
  }

  // y: lane holds rows 4 lg + r of column l16 of each tile
#pragma unroll
  for (int i = 0; i < MT; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t m = m0 + wm * (BM / 2) + i * 16 + 4 * lg + r;
      if (m >= a.M) continue;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int64_t n = n0 + wn * 64 + t * 16 + l16;
        if (n < a.N) a.y[m * a.ys + n] = (uint16_t)(BF16::pack(acc[i][t][r], 0.0f) & 0xffffu);
      }
    }
  }
}

// ---------------------------------------------------------------- decode
// Few rows (M <= 64, the decode step of a batch; K a multiple of 512): the
// weights are read once and x (at most 64 rows) is read by every block. A
// block is 8 waves over 16 NT columns and all rows (or, with MS = 2, one half
// of the rows: the two blocks of a column tile each read the tile's codes and
// half of x), and walks K in chunks of
// 32 groups, each split into 4 sub-chunks of 8 groups. All 512 threads load
// the chunk's codes, scales and biases with coalesced loads (512 contiguous
// bytes of codes per wave instruction), sub-chunk by sub-chunk in issue
// order, and publish each sub-chunk to LDS as it lands (one barrier per
// sub-chunk), so the MFMAs of sub-chunk s run while later sub-chunks are
// still arriving. Wave w takes group 8 s + w of sub-chunk s and reads its x
// straight from global memory into its MFMA A registers (the waves read
// disjoint slices of x; each A fragment serves NT column tiles). Per group a
// wave runs the exact-product MFMAs C_g = x . (128 + q) of its MT x NT tiles
// (B from LDS) and acc += s C_g; two more MFMAs of ones against x^T give the
// row sums Sx_g (every output of lane (l16, lg) is the sum of row l16). The
// bias term sum_g (b - 128 s)[n, g] Sx_g[m] of a chunk's four sub-chunks is
// one f32 MFMA (16 x 16 x 4) per tile, with k = the sub-chunk. The partial
// sums of the 8 waves meet in LDS at the end and are added in wave order.
// (Staging x through LDS as well, with contiguous 1 KB loads, measured no
// faster: the per-sub-chunk load volume, mostly x re-read by every CU, and
// not the access pattern, sets the pace.)
//
// Global loads are buffer loads (a uniform descriptor, a fixed 32-bit offset
// per lane), all unconditional: a sub-chunk past the last group loads through
// a descriptor of zero size, which returns zeros without touching memory. So
// the sequence of loads is the same on every path and the waits stay exact.
constexpr int kDecWaves = 8;
constexpr int kDecThreads = 64 * kDecWaves;
constexpr int kDecSubs = 4;                       // sub-chunks of 8 groups per chunk
constexpr int kDecCG = 8 * kDecSubs;              // groups per chunk
constexpr int kDecPitch = kDecCG * 32 + 16;       // LDS bytes per code row (conflict-free reads)
constexpr int kBufWord3 = 0x00020000;             // raw buffer, 32-bit data format
// Code loads of the decode kernel are non-temporal (each block reads its
// columns' codes once): 12.68 against 12.89 us at M 64, N 12288, K 2048.
// The grouped prefill kernel keeps the default policy: a lane reads 8 bytes
// of a 128-byte code line per group, and the line serves four groups.
constexpr int kDecNt = 2;

template <int MT>
struct DecX {
  u32x4 x[MT][2];
};

__device__ inline __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kBufWord3);
}

template <int MT, int NT, int MS>
__global__ __launch_bounds__(kDecThreads) void qgemm_decode_kernel(QgemmArgs a) {
  constexpr int ROWS = 16 * NT;
  constexpr int WB = ROWS * kDecPitch;             // codes of a chunk
  constexpr int SB = ROWS * kDecCG * 2;            // scales of a chunk (biases again)
  constexpr int RB = kDecWaves * MT * NT * 256 * 4;  // partial sums of the 8 waves
  constexpr int LB = WB + 2 * SB > RB ? WB + 2 * SB : RB;
  // code pieces of PB bytes (16 where the sub-chunk divides evenly into
  // 16-byte pieces over the block's threads, else 8), WP per thread
  constexpr int PB = (ROWS * 16) % kDecThreads == 0 ? 16 : 8;
  constexpr int PR = 256 / PB;                      // pieces per row of a sub-chunk
  constexpr int WP = ROWS * PR / kDecThreads;
  static_assert(WP * kDecThreads == ROWS * PR, "even split");
  typedef typename RawVec<PB>::type piece_t;
  __shared__ __align__(16) unsigned char lds[LB];
  unsigned char* const sct = lds + WB;
  unsigned char* const bit = lds + WB + SB;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  // MS = 2: the rows are split in two halves of 16 MT, and the two blocks of
  // a column tile are 8 apart in launch order, so that both run on the same
  // XCD (blocks are dealt to the 8 XCDs in turn) and share its L2 for the
  // tile's codes.
  int bt = blockIdx.x, half = 0;
  if constexpr (MS == 2) {
    half = (bt >> 3) & 1;
    bt = ((bt >> 4) << 3) | (bt & 7);
  }
  const int64_t n0 = (int64_t)bt * ROWS;
  if (n0 >= a.N) return;  // a padding block of the split grid (whole block)
  const int m0 = half * 16 * MT;
  const int KW = (int)(a.K / 8), G = (int)(a.K / 64);

  const uint32_t xbytes = (uint32_t)(((int64_t)(a.M - 1) * a.xs + a.K) * 2);
  const uint32_t wbytes = (uint32_t)(a.N * a.K / 2), sbytes = (uint32_t)(a.N * G * 2);

  // lane (l16, lg) supplies row l16 of each 16-row tile and, to the group's
  // two MFMAs f = 0, 1, k = 32 f + 8 lg .. 32 f + 8 lg + 7 (code words lg and
  // 4 + lg), so the four lanes of a row read 64 contiguous bytes of x per load
  uint32_t xo[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int r = m0 + i * 16 + l16;
    xo[i] = (uint32_t)((r < a.M ? r : a.M - 1) * a.xs * 2) + 16u * lg;
  }
  // this thread's share of a sub-chunk: code piece c = tid + 512 i is row
  // c / PR, bytes PB (c % PR) of the sub-chunk's 256; each row's 16 bytes of
  // scales and of biases are loaded by one lane (below)
  uint32_t wgo[WP];
#pragma unroll
  for (int i = 0; i < WP; ++i) {
    const int c = tid + kDecThreads * i;
    const int64_t n = n0 + c / PR < a.N ? n0 + c / PR : a.N - 1;
    wgo[i] = (uint32_t)(n * KW * 4) + (uint32_t)(PB * (c % PR));
  }
  // waves 0 .. SW-1 stage the scales (row 64 w + lane), the next SW waves
  // the biases
  constexpr int SW = (ROWS + 63) / 64;
  static_assert(2 * SW <= kDecWaves, "scale and bias staging waves");
  const int srow = 64 * (wave % SW) + lane;
  const bool sbl = wave < 2 * SW && srow < ROWS;
  const bool sct_w = wave < SW;
  const uint32_t sgo = (uint32_t)((n0 + srow < a.N ? n0 + srow : a.N - 1) * G * 2);

  f32x4_t acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[i][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});

  for (int c0 = 0; c0 < G; c0 += kDecCG) {
    if (c0 > 0) __syncthreads();  // the previous chunk's readers are done

    // sub-chunk s covers groups c0 + 8 s .. c0 + 8 s + 7 (live when c0 + 8 s < G)
    piece_t wv[kDecSubs][WP];
    u32x4 sbv[kDecSubs];
    auto load_sub = [&](int s) {
      const uint32_t live = c0 + 8 * s < G ? 0xffffffffu : 0u;
      const int g0 = (c0 + 8 * s) & (int)live;
      const __amdgpu_buffer_rsrc_t bw = buf_rsrc(a.w, wbytes & live);
#pragma unroll
      for (int i = 0; i < WP; ++i)
        if constexpr (PB == 16)
          wv[s][i] = __builtin_bit_cast(piece_t, __builtin_amdgcn_raw_buffer_load_b128(bw, wgo[i], g0 * 32, kDecNt));
        else
          wv[s][i] = __builtin_bit_cast(piece_t, __builtin_amdgcn_raw_buffer_load_b64(bw, wgo[i], g0 * 32, kDecNt));
      const __amdgpu_buffer_rsrc_t bs = buf_rsrc(sct_w ? a.sc : a.bi, wave < 2 * SW ? sbytes & live : 0u);
      sbv[s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(bs, sgo, g0 * 2, 0));
      asm volatile("" ::: "memory");
    };
    auto publish_sub = [&](int s) {
#pragma unroll
      for (int i = 0; i < WP; ++i) {
        const int c = tid + kDecThreads * i;
        *reinterpret_cast<piece_t*>(lds + (c / PR) * kDecPitch + s * 256 + PB * (c % PR)) = wv[s][i];
      }
      if (sbl) *reinterpret_cast<u32x4*>((sct_w ? sct : bit) + srow * (kDecCG * 2) + s * 16) = sbv[s];
    };
    // this wave's group of sub-chunk s: x (zeros, without a memory access,
    // past the last group)
    auto fetch_x = [&](DecX<MT>& q, int s) {
      const bool live = c0 + 8 * s < G;
      const int g = live ? c0 + 8 * s + wave : 0;
      const __amdgpu_buffer_rsrc_t bx = buf_rsrc(a.x, live ? xbytes : 0u);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        q.x[i][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(bx, xo[i], g * 128, 0));
        q.x[i][1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(bx, xo[i] + 64, g * 128, 0));
      }
      asm volatile("" ::: "memory");
    };
    // the row sums of this wave's group in each sub-chunk, row l16 of each
    // 16-row tile (the bias term is applied once per chunk, below)
    float sxs[kDecSubs][MT];
    auto compute = [&](const DecX<MT>& q, int s) {
      const int gl = 8 * s + wave;  // group within the chunk
      bf16x8_t bw[NT][2];
      float sc[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int row = t * 16 + l16;
        const unsigned char* wp = lds + row * kDecPitch + gl * 32 + lg * 4;
        uint32_t w0 = *reinterpret_cast<const uint32_t*>(wp), w1 = *reinterpret_cast<const uint32_t*>(wp + 16);
        asm volatile("" : "+v"(w0), "+v"(w1));
        bw[t][0] = expand_codes(w0);
        bw[t][1] = expand_codes(w1);
        sc[t] = BF16::lo(*reinterpret_cast<const uint16_t*>(sct + row * (kDecCG * 2) + gl * 2));
      }
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const bf16x8_t a0 = __builtin_bit_cast(bf16x8_t, q.x[i][0]);
        const bf16x8_t a1 = __builtin_bit_cast(bf16x8_t, q.x[i][1]);
        // ones . x^T: every output of lane (l16, lg) is the row sum of row l16
        f32x4_t sx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, a0, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
        sx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, a1, sx, 0, 0, 0);
        sxs[s][i] = sx[0];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          f32x4_t c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bw[t][0], f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
          c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bw[t][1], c, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][t][r] = __builtin_fmaf(sc[t], c[r], acc[i][t][r]);
        }
        // the tile row's update completes here (otherwise every MFMA result
        // of the group is held at once)
#pragma unroll
        for (int t = 0; t < NT; ++t) asm volatile("" : "+v"(acc[i][t]));
      }
    };

    // two sub-chunks in flight: sub-chunk s + 2 is requested once the MFMAs
    // of sub-chunk s are done, so those run while s + 1 is still arriving
    DecX<MT> xr[2];
    load_sub(0);
    fetch_x(xr[0], 0);
    load_sub(1);
    fetch_x(xr[1], 1);
#pragma unroll
    for (int s = 0; s < kDecSubs; ++s) {
      publish_sub(s);
      __syncthreads();
      if (c0 + 8 * s < G) {
        compute(xr[s & 1], s);
      } else {
#pragma unroll
        for (int i = 0; i < MT; ++i) sxs[s][i] = 0.0f;
      }
      if (s + 2 < kDecSubs) {
        load_sub(s + 2);
        fetch_x(xr[s & 1], s + 2);
      }
    }
    // bias term of the wave's 4 groups, sum_g (b - 128 s)[n, g] Sx_g[m], as one
    // f32 MFMA (16 x 16 x 4) per tile: k = the sub-chunk, lane (l16, lg)
    // supplies Sx of row l16 and (b - 128 s) of column l16 for sub-chunk lg
    // (zero past the last group: x and the scales read zeros there)
    const int glb = 8 * lg + wave;
    float bsel[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int row = t * 16 + l16;
      const float sv = BF16::lo(*reinterpret_cast<const uint16_t*>(sct + row * (kDecCG * 2) + glb * 2));
      bsel[t] = BF16::lo(*reinterpret_cast<const uint16_t*>(bit + row * (kDecCG * 2) + glb * 2)) - 128.0f * sv;
    }
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const float asel = lg == 0 ? sxs[0][i] : lg == 1 ? sxs[1][i] : lg == 2 ? sxs[2][i] : sxs[3][i];
#pragma unroll
      for (int t = 0; t < NT; ++t)
        acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(asel, bsel[t], acc[i][t], 0, 0, 0);
    }
  }

  // partial sums -> LDS (over the chunk buffers), one 16-byte tile fragment
  // per lane: fragment f = (i NT + t) 64 + lane
  __syncthreads();
  f32x4_t* red = reinterpret_cast<f32x4_t*>(lds);
  constexpr int F = MT * NT * 64;
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < NT; ++t) red[wave * F + (i * NT + t) * 64 + lane] = acc[i][t];
  __syncthreads();
  for (int f = tid; f < F; f += kDecThreads) {
    f32x4_t v = red[f];
#pragma unroll
    for (int w = 1; w < kDecWaves; ++w) v += red[w * F + f];
    const int ln = f & 63, it = f >> 6;
    const int t = it % NT, i = it / NT;
    const int64_t n = n0 + t * 16 + (ln & 15);
    if (n >= a.N) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t m = m0 + i * 16 + 4 * (ln >> 4) + r;
      if (m < a.M) a.y[m * a.ys + n] = (uint16_t)(BF16::pack(v[r], 0.0f) & 0xffffu);
    }
  }
}

// ---------------------------------------------------------------- hi/lo
// Many rows (prefill): the matrix cores are the bound, and the per-group f32
// epilogue of the exact form costs as much VALU time as the MFMAs take. Here
// each block dequantizes its 128-column weight tile once per group into LDS
// as two bf16 planes, w = s*q + b (one f32 rounding) = hi + lo with
// hi = the top 16 bits of w and lo = bf16(w - hi) (|error| <= 2^-17 |w|),
// and the MFMAs run over both planes straight into the accumulators (no
// epilogue, no row sums). A block is 8 waves (4 x 2) of 64 x 64 tiles:
// 256 rows x 128 columns; x and the two planes are double-buffered in LDS,
// one barrier per group, and the next group's x, codes, scales and biases
// are loaded while the current group's MFMAs run.
constexpr int kHlBM = 256, kHlBN = 128;
// groups of loads in flight (4 measured no faster than 2: this kernel is
// bound by LDS traffic and issue, not by load latency)
constexpr int kHlDepth = 2;

// two f32 -> packed bf16 pair by truncation (the hi plane) and by rounding
__device__ inline uint32_t pack_hi(float a, float b) {
  return (f2u(a) >> 16) | (f2u(b) & 0xffff0000u);
}

// Ask the scheduler to spread the next group's publish (dequantization VALU
// and LDS writes) between this group's MFMAs instead of after them: with the
// waves of a SIMD in step (one barrier per group), a publish placed after the
// MFMAs leaves the matrix core idle while it runs.
// The operand reads go first (the A fragments of the MT row tiles and the
// first column tile's B fragments), each later column tile's B fragments one
// tile ahead; per column tile the MT x 4 MFMAs alternate with the VALU and LDS
// writes of the publish (about 100 VALU per group and wave). The grouped
// gather kernel (2 row tiles per wave) measured 3% slower with it and keeps
// the compiler's order.
template <int MT>
__device__ inline void hl_interleave() {
  __builtin_amdgcn_sched_group_barrier(0x100, 2 * MT + 4, 0);  // LDS reads
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    if (t < 3) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // next tile's B
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);           // 4 MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 40 / MT, 0);     // VALU (6 and 8 measured slower)
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);           // 1 LDS write
    }
  }
}

// WM x 2 waves, each (16 MT) x 64: WM * 16 * MT = 256 rows.
template <int WM, int MT>
__global__ __launch_bounds__(WM * 128) void qgemm_hl_kernel(QgemmArgs a) {
  constexpr int NT = 4, T = WM * 128;
  static_assert(WM * 16 * MT == kHlBM, "256-row blocks");
  constexpr int XP = kHlBM * 8 / T;   // 16-byte x pieces per thread per group
  constexpr int WPT = kHlBN * 8 / T;  // code words per thread per group (2 or 4)
  __shared__ __align__(16) uint16_t xs[2][kHlBM][kQgPitch];
  __shared__ __align__(16) uint16_t wh[2][kHlBN][kQgPitch];
  __shared__ __align__(16) uint16_t wl[2][kHlBN][kQgPitch];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l16 = lane & 15, lg = lane >> 4;
  const int64_t m0 = (int64_t)blockIdx.y * kHlBM, n0 = (int64_t)blockIdx.x * kHlBN;
  const int KW = (int)(a.K / 8), G = (int)(a.K / 64);

  // x: 256 rows x 8 pieces of 16 B per group; piece c = tid + T i
  const uint16_t* xrow[XP];
#pragma unroll
  for (int i = 0; i < XP; ++i) {
    const int c = tid + T * i;
    const int64_t r = m0 + c / 8;
    xrow[i] = a.x + (r < a.M ? r : a.M - 1) * a.xs + (c & 7) * 8;
  }
  // weights: column tid / (8 / WPT) of the tile, WPT consecutive words
  const int wcn = tid / (8 / WPT), wpart = tid % (8 / WPT);
  const int64_t wn_ = n0 + wcn < a.N ? n0 + wcn : a.N - 1;
  const uint32_t* wsrc = a.w + wn_ * KW + WPT * wpart;
  const uint16_t* ssrc = a.sc + wn_ * G;
  const uint16_t* bsrc = a.bi + wn_ * G;

  // a ring of kHlDepth groups' loads in registers (slot g % kHlDepth)
  struct Stage {
    u32x4 x[XP];
    uint32_t w[WPT];
    uint32_t s, b;
  };
  Stage st[kHlDepth];
  auto fetch = [&](Stage& q, int g) {
#pragma unroll
    for (int i = 0; i < XP; ++i) q.x[i] = *reinterpret_cast<const u32x4*>(xrow[i] + g * 64);
    if constexpr (WPT == 4) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(wsrc + g * 8);
#pragma unroll
      for (int h = 0; h < 4; ++h) q.w[h] = v[h];
    } else {
      const u32x2_t v = *reinterpret_cast<const u32x2_t*>(wsrc + g * 8);
      q.w[0] = v[0];
      q.w[1] = v[1];
    }
    q.s = ssrc[g];
    q.b = bsrc[g];
  };
  // write a fetched group into LDS buffer `buf`: x as it is, weights as the
  // hi and lo planes of s * q + b
  auto publish = [&](const Stage& q, int buf) {
#pragma unroll
    for (int i = 0; i < XP; ++i) {
      const int c = tid + T * i;
      *reinterpret_cast<u32x4*>(&xs[buf][c / 8][(c & 7) * 8]) = q.x[i];
    }
    const float sc = BF16::lo(q.s), bi = BF16::lo(q.b);
#pragma unroll
    for (int h = 0; h < WPT; ++h) {
      const uint32_t c = q.w[h];
      float w[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) w[k] = __builtin_fmaf(sc, (float)((c >> (4 * k)) & 15u), bi);
      u32x4 hi, lo;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        hi[k] = pack_hi(w[2 * k], w[2 * k + 1]);
        const float h0 = u2f(f2u(w[2 * k]) & 0xffff0000u), h1 = u2f(f2u(w[2 * k + 1]) & 0xffff0000u);
        lo[k] = BF16::pack(w[2 * k] - h0, w[2 * k + 1] - h1);
      }
      *reinterpret_cast<u32x4*>(&wh[buf][wcn][(WPT * wpart + h) * 8]) = hi;
      *reinterpret_cast<u32x4*>(&wl[buf][wcn][(WPT * wpart + h) * 8]) = lo;
    }
  };

  f32x4_t acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[i][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  auto compute = [&](int buf) {
    bf16x8_t av[MT][2];
#pragma unroll
    for (int i = 0; i < MT; ++i) {
      const int row = wm * 16 * MT + i * 16 + l16;
      av[i][0] = *reinterpret_cast<const bf16x8_t*>(&xs[buf][row][(2 * lg) * 8]);
      av[i][1] = *reinterpret_cast<const bf16x8_t*>(&xs[buf][row][(2 * lg + 1) * 8]);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int col = wn * 64 + t * 16 + l16;
      const bf16x8_t h0 = *reinterpret_cast<const bf16x8_t*>(&wh[buf][col][(2 * lg) * 8]);
      const bf16x8_t h1 = *reinterpret_cast<const bf16x8_t*>(&wh[buf][col][(2 * lg + 1) * 8]);
      const bf16x8_t o0 = *reinterpret_cast<const bf16x8_t*>(&wl[buf][col][(2 * lg) * 8]);
      const bf16x8_t o1 = *reinterpret_cast<const bf16x8_t*>(&wl[buf][col][(2 * lg + 1) * 8]);
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i][0], h0, acc[i][t], 0, 0, 0);
        acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i][1], h1, acc[i][t], 0, 0, 0);
        acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i][0], o0, acc[i][t], 0, 0, 0);
        acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i][1], o1, acc[i][t], 0, 0, 0);
      }
    }
  };

  // every fetch is unconditional (past the last group it re-reads the last
  // group), so the count of loads in flight is the same on every path and a
  // publish waits only for its own group's loads
#pragma unroll
  for (int d = 0; d < kHlDepth; ++d) fetch(st[d], d < G ? d : G - 1);
  publish(st[0], 0);
  for (int g0 = 0; g0 < G; g0 += kHlDepth) {
#pragma unroll
    for (int d = 0; d < kHlDepth; ++d) {
      const int g = g0 + d;
      if (g >= G) break;
      __syncthreads();  // buffer g&1 is complete; buffer (g+1)&1 is no longer read
      fetch(st[d], g + kHlDepth < G ? g + kHlDepth : G - 1);
      compute(g & 1);
      // (after the last group this publishes a repeat of it into the buffer
      // that is no longer read: unconditional, so the MFMAs and the publish
      // share one scheduling region)
      publish(st[(d + 1) % kHlDepth], (g + 1) & 1);
      hl_interleave<MT>();
    }
  }

#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t m = m0 + wm * 16 * MT + i * 16 + 4 * lg + r;
      if (m >= a.M) continue;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int64_t n = n0 + wn * 64 + t * 16 + l16;
        if (n < a.N) a.y[m * a.ys + n] = (uint16_t)(BF16::pack(acc[i][t][r], 0.0f) & 0xffffu);
      }
    }
}

// ---------------------------------------------------------------- gather
// gather_qmm grouped by expert (forward_gather at prefill: hundreds of pairs
// per expert). The caller's indices are unsorted (the reference passes
// sorted = false) and the library allocates nothing, so block (n-tile, e)
// finds expert e's pairs itself: it scans the expert ids 4096 at a time,
// each wave compacting its matches with a ballot and one LDS atomic, into an
// LDS list of up to kGaCap pairs (a round's id loads all go out before any
// is compared). The listed pairs are then run 128 rows at a
// time through the hi/lo-plane MFMA pipeline of the prefill kernel with x
// rows gathered through the list (8 waves of 32 x 64 tiles; each group's
// x, codes, scales and biases are loaded four groups ahead into a register
// ring); a full list is drained and the scan resumes. Block row e = E writes the zero rows of pairs whose expert is out
// of range (x rows out of range are staged as zeros, giving zero rows too).
constexpr int kGaBM = 128, kGaDepth = 4;
constexpr int kGaRoundIds = 4096;  // expert ids per block per scan round
constexpr int kGaCap = 6144;       // listed pairs (a round adds at most kGaRoundIds)
// A pass's first round starts from an empty list, so it always runs and fits:
// every pass advances the scan.
static_assert(kGaCap >= kGaRoundIds, "a round must fit in an empty list");

__device__ inline int64_t ga_expert(const GatherArgs& a, int64_t p) {
  if (a.experts_i32) {
    const int64_t e = reinterpret_cast<const int32_t*>(a.experts)[p];
    return e < 0 ? e + a.E : e;
  }
  return (int64_t)reinterpret_cast<const uint32_t*>(a.experts)[p];
}

__device__ inline int64_t ga_row(const GatherArgs& a, int64_t p) {
  int64_t r = a.lhs ? (int64_t)a.lhs[p] : p / a.xdiv;
  if (a.lhs && r < 0) r += a.xrows;
  return (r >= 0 && r < a.xrows) ? r : -1;
}

// One listing phase of the grouped kernels: the ids from pair `scan` on are
// read kGaRoundIds per round (RND per thread, two rounds in flight: the next
// round's ids are requested before the current round is compared, into the
// other of two arrays, so no register copy waits for them) and expert e's
// pairs appended to the LDS list, until the ids run out or the list could
// overflow on the next round. Each id slot's matches are one ballot per
// wave; one LDS atomic per wave reserves the wave's slots and each match
// takes its place from scalar popcounts and its lane's mbcnt rank. This
// replaced a wave-wide prefix sum of per-thread counts (six dependent lane
// shuffles per round): gate 188.3 -> 183.8 us, down 210.8 -> 206.5 and the
// fused gate + up + SwiGLU 327.2 -> 322.7 at the 4096-token Qwen3-Next MoE
// prefill. The list order is free: every listed pair's output row is
// computed on its own.
// Contains barriers: every thread of the block calls it. Returns the count.
template <int RND>
__device__ inline int ga_list_phase(const GatherArgs& a, __amdgpu_buffer_rsrc_t rid, int64_t e,
                                    int64_t& scan, int tid, int* cnt, int32_t* list) {
  const int lane = tid & 63;
  // raw ids equal to e (and, for int32 ids, to e - E, which wraps to e)
  const uint32_t e1 = (uint32_t)e, e2 = a.experts_i32 ? (uint32_t)(e - a.E) : (uint32_t)e;
  const uint32_t pairs = (uint32_t)a.pairs;
  auto load_round = [&](uint32_t (&r)[RND], int64_t base) {
    const bool live = base < a.pairs;
#pragma unroll
    for (int c = 0; c < RND / 4; ++c) {
      const uint32_t off = live ? (uint32_t)((base + RND * tid + 4 * c) * 4) : 0x80000000u;
      const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rid, off, 0, 0));
#pragma unroll
      for (int k = 0; k < 4; ++k) r[4 * c + k] = v[k];
    }
  };
  auto round = [&](const uint32_t (&ids)[RND]) {
    const uint32_t p0 = (uint32_t)scan + RND * tid;
    // one ballot per id slot: a wave's matches are counted and placed with
    // scalar popcounts and mbcnt (no cross-lane prefix sum)
    uint64_t bal[RND];
    int tot = 0;
#pragma unroll
    for (int i = 0; i < RND; ++i) {
      bal[i] = __ballot(p0 + i < pairs && (ids[i] == e1 || ids[i] == e2));
      tot += __popcll(bal[i]);
    }
    if (tot > 0) {  // uniform per wave
      int base = 0;
      if (lane == 0) base = atomicAdd(cnt, tot);
      base = __builtin_amdgcn_readfirstlane(base);
#pragma unroll
      for (int i = 0; i < RND; ++i) {
        if (bal[i]) {  // uniform
          const uint32_t lo = (uint32_t)bal[i], hi = (uint32_t)(bal[i] >> 32);
          const int rank = (int)__builtin_amdgcn_mbcnt_hi(hi, __builtin_amdgcn_mbcnt_lo(lo, 0u));
          if ((bal[i] >> lane) & 1u) list[base + rank] = (int32_t)(p0 + i);
          base += __popcll(bal[i]);
        }
      }
    }
    scan += kGaRoundIds;
    __syncthreads();
  };
  uint32_t ra[RND], rb[RND];
  load_round(ra, scan);
  __syncthreads();
  if (tid == 0) *cnt = 0;
  __syncthreads();
  while (scan < a.pairs) {
    if (*cnt > kGaCap - kGaRoundIds) break;  // uniform: read after the round's barrier
    load_round(rb, scan + kGaRoundIds);
    round(ra);
    if (scan >= a.pairs || *cnt > kGaCap - kGaRoundIds) break;
    load_round(ra, scan + kGaRoundIds);
    round(rb);
  }
  return *cnt;
}

template <int WAVES>
__global__ __launch_bounds__(WAVES * 64) void gather_hl_kernel(GatherArgs a) {
  // WAVES = 4: 2 x 2 waves of 64 x 64; WAVES = 8: 4 x 2 waves of 32 x 64
  constexpr int T = WAVES * 64, MT = 16 / WAVES, NT = 4;
  constexpr int RND = kGaRoundIds / T;  // ids per thread per scan round
  constexpr int XP = kGaBM * 8 / T;   // 4 x pieces per thread per group
  constexpr int WPT = kHlBN * 8 / T;  // 4 code words per thread per group
  __shared__ __align__(16) uint16_t xs[2][kGaBM][kQgPitch];
  __shared__ __align__(16) uint16_t wh[2][kHlBN][kQgPitch];
  __shared__ __align__(16) uint16_t wl[2][kHlBN][kQgPitch];
  __shared__ int32_t list[kGaCap];
  __shared__ int32_t cnt;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int l16 = lane & 15, lg = lane >> 4;
  // this block: expert blockIdx.y, column tiles blockIdx.x * tpg .. + tpg
  const int64_t e = blockIdx.y;
  const int ntiles = (int)((a.N + kHlBN - 1) / kHlBN);
  const int tpg = (ntiles + (int)gridDim.x - 1) / (int)gridDim.x;
  const int nt0 = (int)blockIdx.x * tpg, nt1 = nt0 + tpg < ntiles ? nt0 + tpg : ntiles;
  const int KW = (int)(a.K / 8), G = (int)(a.K / 64);

  if (e == a.E) {
    // pairs whose expert is out of range: zero rows (this block's columns)
    const int64_t c0 = (int64_t)nt0 * kHlBN, c1 = (int64_t)nt1 * kHlBN < a.N ? (int64_t)nt1 * kHlBN : a.N;
    for (int64_t p0 = 0; p0 < a.pairs; p0 += T) {
      const int64_t p = p0 + tid;
      const int64_t ep = p < a.pairs ? ga_expert(a, p) : 0;
      if (p < a.pairs && (ep < 0 || ep >= a.E))
        for (int64_t c = c0; c < c1; ++c) a.y[p * a.ys + c] = 0;
    }
    return;
  }
  const int wcn = tid / (8 / WPT), wpart = tid % (8 / WPT);

  // the expert ids as stored (converted where compared); thread tid reads ids
  // base + RND tid .. + RND - 1 of a round with 16-byte buffer loads (ids past
  // the last pair read zeros and are never listed)
  static_assert(RND % 4 == 0, "whole 16-byte id loads");
  const __amdgpu_buffer_rsrc_t rid = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(a.experts), (short)0, (int)(a.pairs * 4), 0x00020000);
  int64_t scan = 0;
  while (scan < a.pairs) {
    // ---- fill the list from `scan` (stop before overflow)
    const int rows = ga_list_phase<RND>(a, rid, e, scan, tid, &cnt, list);

    // ---- the listed pairs, kGaBM at a time, for each of this block's column tiles
    for (int nt = nt0; nt < nt1; ++nt)
    for (int t0 = 0; t0 < rows; t0 += kGaBM) {
      const int64_t n0 = (int64_t)nt * kHlBN;
      // this thread's weight column and words (expert e)
      const int64_t wn_ = n0 + wcn < a.N ? n0 + wcn : a.N - 1;
      const uint32_t* wsrc = a.w + (e * a.N + wn_) * KW + WPT * wpart;
      const uint16_t* ssrc = a.sc + (e * a.N + wn_) * G;
      const uint16_t* bsrc = a.bi + (e * a.N + wn_) * G;
      const uint16_t* xrow[XP];
      bool xok[XP];
#pragma unroll
      for (int i = 0; i < XP; ++i) {
        const int c = tid + T * i, r = t0 + c / 8;
        const int64_t xr = r < rows ? ga_row(a, list[r]) : -1;
        xok[i] = xr >= 0;
        xrow[i] = a.x + (xr >= 0 ? xr : 0) * a.xs + (c & 7) * 8;
      }
      // a ring of kGaDepth groups' loads in registers (slot g % kGaDepth)
      struct Stage {
        u32x4 x[XP];
        uint32_t w[WPT];
        uint32_t s, b;
      };
      Stage st[kGaDepth];
      auto fetch = [&](Stage& q, int g) {
        // unconditional loads (an invalid row reads row 0 and is zeroed at
        // publish), so the number of loads in flight is the same on every path
#pragma unroll
        for (int i = 0; i < XP; ++i) q.x[i] = *reinterpret_cast<const u32x4*>(xrow[i] + g * 64);
        if constexpr (WPT == 4) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(wsrc + g * 8);
#pragma unroll
          for (int h = 0; h < 4; ++h) q.w[h] = v[h];
        } else {
          const u32x2_t v = *reinterpret_cast<const u32x2_t*>(wsrc + g * 8);
          q.w[0] = v[0];
          q.w[1] = v[1];
        }
        q.s = ssrc[g];
        q.b = bsrc[g];
      };
      auto publish = [&](const Stage& q, int buf) {
#pragma unroll
        for (int i = 0; i < XP; ++i) {
          const int c = tid + T * i;
          const uint32_t m = xok[i] ? 0xffffffffu : 0u;
          *reinterpret_cast<u32x4*>(&xs[buf][c / 8][(c & 7) * 8]) =
              u32x4{q.x[i][0] & m, q.x[i][1] & m, q.x[i][2] & m, q.x[i][3] & m};
        }
        const float sc = BF16::lo(q.s), bi = BF16::lo(q.b);
#pragma unroll
        for (int h = 0; h < WPT; ++h) {
          const uint32_t c = q.w[h];
          float w[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) w[k] = __builtin_fmaf(sc, (float)((c >> (4 * k)) & 15u), bi);
          u32x4 hi, lo;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            hi[k] = pack_hi(w[2 * k], w[2 * k + 1]);
            const float h0 = u2f(f2u(w[2 * k]) & 0xffff0000u), h1 = u2f(f2u(w[2 * k + 1]) & 0xffff0000u);
            lo[k] = BF16::pack(w[2 * k] - h0, w[2 * k + 1] - h1);
          }
          *reinterpret_cast<u32x4*>(&wh[buf][wcn][(WPT * wpart + h) * 8]) = hi;
          *reinterpret_cast<u32x4*>(&wl[buf][wcn][(WPT * wpart + h) * 8]) = lo;
        }
      };

      f32x4_t acc[MT][NT];
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[i][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

      auto compute = [&](int buf) {
        bf16x8_t av[MT][2];
#pragma unroll
        for (int i = 0; i < MT; ++i) {
          const int row = wm * 16 * MT + i * 16 + l16;
          av[i][0] = *reinterpret_cast<const bf16x8_t*>(&xs[buf][row][(2 * lg) * 8]);
          av[i][1] = *reinterpret_cast<const bf16x8_t*>(&xs[buf][row][(2 * lg + 1) * 8]);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const int col = wn * 64 + t * 16 + l16;
          const bf16x8_t h0 = *reinterpret_cast<const bf16x8_t*>(&wh[buf][col][(2 * lg) * 8]);
          const bf16x8_t h1 = *reinterpret_cast<const bf16x8_t*>(&wh[buf][col][(2 * lg + 1) * 8]);
          const bf16x8_t o0 = *reinterpret_cast<const bf16x8_t*>(&wl[buf][col][(2 * lg) * 8]);
          const bf16x8_t o1 = *reinterpret_cast<const bf16x8_t*>(&wl[buf][col][(2 * lg + 1) * 8]);
#pragma unroll
          for (int i = 0; i < MT; ++i) {
            acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i][0], h0, acc[i][t], 0, 0, 0);
            acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i][1], h1, acc[i][t], 0, 0, 0);
            acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i][0], o0, acc[i][t], 0, 0, 0);
            acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[i][1], o1, acc[i][t], 0, 0, 0);
          }
        }
      };

      __syncthreads();  // the previous tile's LDS reads are done
      // every fetch is unconditional (past the last group it re-reads the
      // last group), so the count of loads in flight is the same on every
      // path and a publish waits only for its own group's loads
#pragma unroll
      for (int d = 0; d < kGaDepth; ++d) fetch(st[d], d < G ? d : G - 1);
      publish(st[0], 0);
      // group g: its loads were issued kGaDepth - 1 groups earlier into slot
      // g % kGaDepth; the loop is unrolled by the ring depth so the slots are
      // fixed registers
      for (int g0 = 0; g0 < G; g0 += kGaDepth) {
#pragma unroll
        for (int d = 0; d < kGaDepth; ++d) {
          const int g = g0 + d;
          if (g >= G) break;
          __syncthreads();
          fetch(st[d], g + kGaDepth < G ? g + kGaDepth : G - 1);
          compute(g & 1);
          if (g + 1 < G) publish(st[(d + 1) % kGaDepth], (g + 1) & 1);
        }
      }

#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int lr = t0 + wm * 16 * MT + i * 16 + 4 * lg + r;
          if (lr >= rows) continue;
          const int64_t p = list[lr];
#pragma unroll
          for (int t = 0; t < NT; ++t) {
            const int64_t n = n0 + wn * 64 + t * 16 + l16;
            if (n < a.N) a.y[p * a.ys + n] = (uint16_t)(BF16::pack(acc[i][t][r], 0.0f) & 0xffffu);
          }
        }
    }
  }
}

// ---------------------------------------------------------------- grouped, exact
// The prefill form of gather_qmm with no weight plane in LDS. A block is one
// expert and 8 waves side by side over 512 columns (64 each, 4 column tiles);
// its rows are the expert's listed pairs, up to 16 RT per pass. Per group a
// wave loads its codes straight into B-operand registers, one 8-byte buffer
// load per column tile (lane group j supplies code words 2j and 2j + 1, i.e.
// k = 16 j .. 16 j + 15 of the group), and expands each word to the bf16
// numbers 128 + q in the order (q0, q4), (q1, q5), (q2, q6), (q3, q7), which
// x is stored in as well (7 operations per word). The MFMAs C = x . (128 + q)
// are exact products summed in f32, with acc += s C per group from four
// independent MFMA chains (one per column tile). The bias term
// sum_g (b - 128 s)[n, g] Sx_g[m] is one f32 MFMA (16 x 16 x 4) per tile and
// 4 groups. LDS holds x (four groups' buffers, one barrier per two groups),
// its per-group row sums, the block's scales and biases (8 groups at a time,
// double-buffered) and the pair list. Global loads are buffer loads at fixed
// per-lane offsets; a row past the pass's last reads zeros through an
// out-of-range offset, so the load sequence is the same on every path.
// Measured at a 4096-token Qwen3-Next MoE prefill (40,960 pairs, top-10 of
// 512): gate 184 us against 342 for the hi/lo kernel, down 207-212 against
// 414. Passes of 112 rows (7 row tiles) rather than 96 took gate from 218 to
// 190 us and down from 261 to 224. An expert holds about 80 pairs here, but
// with 96 rows per pass those holding more than 96 took a second pass, and
// the CUs running them set the launch's end. 128-row passes measured 191 us
// for gate. (One barrier per group instead of per two: 234 and 280 at 96
// rows.)
// Non-temporal x loads, requesting all scan rounds' ids at once, and issuing
// the next pass's first loads before a pass's stores all measured slower.
constexpr int kXpXB = 4;  // x buffers in LDS (two groups per barrier)
constexpr int kXpWaves = 8, kXpT = 64 * kXpWaves;
constexpr int kXpBN = 64 * kXpWaves;  // columns per block pass

// SW: the fused gate + up + SwiGLU form. Waves 0-3 run the gate projection
// and waves 4-7 the up projection of the same 256 columns; after a pass the
// up waves leave their bf16 results in LDS and the gate waves write
// swiglu(gate, up), rounded as the reference's three calls round it.
template <int RT, bool SW>
__global__ __launch_bounds__(kXpT) void gather_xp_kernel(GatherArgs a) {
  constexpr int BM = 16 * RT, NT = 4;
  constexpr int BNO = SW ? kXpBN / 2 : kXpBN;  // output columns per pass
  constexpr int XP = (BM * 8 + kXpT - 1) / kXpT;  // 16-byte x pieces per thread per group
  constexpr int RND = kGaRoundIds / kXpT;  // ids per thread per scan round
  __shared__ __align__(16) uint16_t xs[kXpXB][BM][kQgPitch];
  __shared__ float sxs[8][BM];              // row sums, ring of 8 groups
  // scales and biases of 8 groups per column (double-buffered per 8 groups)
  __shared__ __align__(16) u32x4 ssb[2][kXpBN], bsb[2][kXpBN];
  __shared__ int32_t list[kGaCap];
  __shared__ int32_t cnt;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int64_t e = blockIdx.y;
  const int ntiles = (int)((a.N + BNO - 1) / BNO);
  const int tpg = (ntiles + (int)gridDim.x - 1) / (int)gridDim.x;
  const int nt0 = (int)blockIdx.x * tpg, nt1 = nt0 + tpg < ntiles ? nt0 + tpg : ntiles;
  const int G = (int)(a.K / 64);

  if (e == a.E) {
    // pairs whose expert is out of range: zero rows (this block's columns)
    const int64_t c0 = (int64_t)nt0 * BNO, c1 = (int64_t)nt1 * BNO < a.N ? (int64_t)nt1 * BNO : a.N;
    for (int64_t p0 = 0; p0 < a.pairs; p0 += kXpT) {
      const int64_t p = p0 + tid;
      const int64_t ep = p < a.pairs ? ga_expert(a, p) : 0;
      if (p < a.pairs && (ep < 0 || ep >= a.E))
        for (int64_t c = c0; c < c1; ++c) a.y[p * a.ys + c] = 0;
    }
    return;
  }

  static_assert(RND % 4 == 0, "whole 16-byte id loads");
  const __amdgpu_buffer_rsrc_t rid = buf_rsrc(a.experts, (uint32_t)(a.pairs * 4));

  const uint32_t xbytes = (uint32_t)(((a.xrows - 1) * a.xs + a.K) * 2);
  const __amdgpu_buffer_rsrc_t rx = buf_rsrc(a.x, xbytes);
  // the up waves (SW, waves 4-7: also the threads staging the up columns'
  // scales) read the up projection's arrays
  const bool upw = SW && wave >= 4;
  const __amdgpu_buffer_rsrc_t rw = buf_rsrc(upw ? a.w2 : a.w, (uint32_t)(a.E * a.N * a.K / 2));
  const __amdgpu_buffer_rsrc_t rs = buf_rsrc(upw ? a.sc2 : a.sc, (uint32_t)(a.E * a.N * G * 2));
  const __amdgpu_buffer_rsrc_t rb = buf_rsrc(upw ? a.bi2 : a.bi, (uint32_t)(a.E * a.N * G * 2));
  const int C8 = G / 8;
  const int wcol = SW ? (wave & 3) : wave;  // the wave's 64-column slice of the pass
  // whole 16-byte output pieces: 8-column rows, 16-byte aligned
  const bool yvec = a.N % 8 == 0 && a.ys % 8 == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0;

  // ---- per-pass addressing and loads (a pass: column chunk nt, rows t0 .. t0 + rp)
  uint32_t wo[NT], so, xo[XP];
  // this lane's columns of chunk nt: codes (words 2 lg, 2 lg + 1 of each
  // group); this thread's column of the block's scale/bias staging
  auto set_cols = [&](int nt) {
    const int64_t n0 = (int64_t)nt * BNO + 64 * wcol;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int64_t n = n0 + 16 * t + l16;
      const int64_t nc = n < a.N ? n : a.N - 1;
      wo[t] = (uint32_t)((e * a.N + nc) * (a.K / 2)) + 8u * lg;
    }
    const int64_t sn = (int64_t)nt * BNO + (SW ? (tid & (BNO - 1)) : tid);
    so = (uint32_t)((e * a.N + (sn < a.N ? sn : a.N - 1)) * G * 2);
  };
  // this thread's x pieces: piece c = tid + 512 i is row c / 8, bytes 16 (c % 8)
  // of the group's 128 (out of range past the pass's rows)
  auto set_rows = [&](int t0, int rp) {
#pragma unroll
    for (int i = 0; i < XP; ++i) {
      const int c = tid + kXpT * i, r = c / 8;
      const int64_t xr = r < rp && c < BM * 8 ? ga_row(a, list[t0 + r]) : -1;
      xo[i] = xr >= 0 ? (uint32_t)(xr * a.xs * 2) + 16u * (c & 7) : 0x80000000u;
    }
  };
  u32x2_t cw[2][NT];   // codes of two groups in flight
  u32x4 cx[2][XP];     // x pieces of two groups in flight
  u32x4 sreg, breg;    // scales and biases of 8 groups of this thread's column
  auto fetch_w = [&](u32x2_t (&q)[NT], int g) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
      q[t] = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(rw, wo[t], g * 32, 0));
    asm volatile("" ::: "memory");
  };
  auto fetch_x = [&](u32x4 (&q)[XP], int g) {
#pragma unroll
    for (int i = 0; i < XP; ++i)
      q[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, xo[i], g * 128, 0));
    asm volatile("" ::: "memory");
  };
  auto fetch_sb = [&](int c8) {
    sreg = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, so, c8 * 16, 0));
    breg = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, so, c8 * 16, 0));
    asm volatile("" ::: "memory");
  };
  auto publish_sb = [&](int buf) {
    ssb[buf][tid] = sreg;
    bsb[buf][tid] = breg;
  };
  auto publish_x = [&](const u32x4 (&q)[XP], int g) {
    const int buf = g & (kXpXB - 1);
#pragma unroll
    for (int i = 0; i < XP; ++i) {
      const int c = tid + kXpT * i;
      if (c < BM * 8) {  // whole waves (BM * 8 is a multiple of 64)
        *reinterpret_cast<u32x4*>(&xs[buf][c / 8][(c & 7) * 8]) = order_x4(q[i]);
        const float s8 = sum8_lanes(sum8_bf16(q[i]));
        if ((c & 7) == 0) sxs[g & 7][c / 8] = s8;
      }
    }
  };
  // element j (0..7) of a column's staged scales or biases
  auto stage_elem = [&](const u32x4 (&st)[kXpBN], int col, int j) {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(&st[col]);
    return BF16::lo((uint32_t)p[j]);
  };
  const X4Masks xm = x4_masks();

  int64_t scan = 0;
  while (scan < a.pairs) {
    // ---- list this expert's pairs from `scan` (stop before overflow)
    const int rows = ga_list_phase<RND>(a, rid, e, scan, tid, &cnt, list);

    for (int nt = nt0; nt < nt1; ++nt)
    for (int t0 = 0; t0 < rows; t0 += BM) {
      const int rp = rows - t0 < BM ? rows - t0 : BM;  // rows of this pass
      const int rt = (rp + 15) >> 4;                   // live row tiles
      const int64_t n0 = (int64_t)nt * BNO + 64 * wcol;
      set_cols(nt);
      set_rows(t0, rp);
      fetch_sb(0);
      fetch_x(cx[0], 0);
      fetch_w(cw[0], 0);
      fetch_x(cx[1], 1);
      fetch_w(cw[1], 1);

      f32x4_t acc[RT][NT];
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[i][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

      // group g: its codes in cw[g & 1], its scales in stage (g / 8) & 1
      auto compute = [&](const u32x2_t (&q)[NT], int g) {
        const int sb = (g >> 3) & 1, j = g & 7;
        bf16x8_t bw[NT][2];
        float sc[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          uint32_t w0 = q[t][0], w1 = q[t][1];
          asm volatile("" : "+v"(w0), "+v"(w1));
          bw[t][0] = expand_codes_x4(w0, xm);
          bw[t][1] = expand_codes_x4(w1, xm);
          sc[t] = stage_elem(ssb[sb], 64 * wave + 16 * t + l16, j);
        }
        const int buf = g & (kXpXB - 1);
#pragma unroll
        for (int i = 0; i < RT; ++i) {
          if (i < rt) {  // uniform
            const bf16x8_t a0 = *reinterpret_cast<const bf16x8_t*>(&xs[buf][i * 16 + l16][(2 * lg) * 8]);
            const bf16x8_t a1 = *reinterpret_cast<const bf16x8_t*>(&xs[buf][i * 16 + l16][(2 * lg + 1) * 8]);
            // four independent chains (one per column tile), then their epilogues
            f32x4_t c[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t)
              c[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bw[t][0], f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
            for (int t = 0; t < NT; ++t)
              c[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bw[t][1], c[t], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
              for (int r = 0; r < 4; ++r) acc[i][t][r] = __builtin_fmaf(sc[t], c[t][r], acc[i][t][r]);
            // the row tile's update completes here (otherwise every MFMA
            // result of the group is held at once)
#pragma unroll
            for (int t = 0; t < NT; ++t) asm volatile("" : "+v"(acc[i][t]));
          }
        }
      };
      // bias term of groups g4 .. g4 + 3 (g4 % 4 == 0): lane (l16, lg)
      // supplies Sx of row l16 and (b - 128 s) of column l16 for group g4 + lg
      auto bias = [&](int g4) {
        const int sb = (g4 >> 3) & 1, j = (g4 & 7) + lg;
        float bsel[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const int col = 64 * wave + 16 * t + l16;
          bsel[t] = stage_elem(bsb[sb], col, j) - 128.0f * stage_elem(ssb[sb], col, j);
        }
#pragma unroll
        for (int i = 0; i < RT; ++i) {
          if (i < rt) {
            const float asel = sxs[(g4 + lg) & 7][i * 16 + l16];
#pragma unroll
            for (int t = 0; t < NT; ++t)
              acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(asel, bsel[t], acc[i][t], 0, 0, 0);
          }
        }
      };

      __syncthreads();  // the previous pass's LDS readers are done
      publish_sb(0);
      fetch_sb(1 < C8 ? 1 : 0);
      publish_x(cx[0], 0);
      publish_x(cx[1], 1);
      fetch_x(cx[0], 2);
      fetch_x(cx[1], 3);
      // two groups per unrolled body (G is a multiple of 8): the slots are
      // fixed registers; every fetch is unconditional (past the last group
      // it re-reads the last)
      for (int g0 = 0; g0 < G; g0 += 2) {
        // x of groups g0 and g0 + 1 is in LDS; the readers of the two
        // buffers refilled in this step (groups g0 - 2, g0 - 1) are done
        __syncthreads();
#pragma unroll
        for (int d = 0; d < 2; ++d) {
          const int g = g0 + d;
          compute(cw[d], g);
          if ((g & 3) == 3) bias(g - 3);  // uniform
          if ((g & 7) == 7) {
            // the next 8 groups' scales go to the other stage (its readers,
            // 8 groups back, are done); the 8 after that are requested
            publish_sb(((g >> 3) + 1) & 1);
            const int c2 = (g >> 3) + 2;
            fetch_sb(c2 < C8 ? c2 : C8 - 1);
          }
          // this slot's x (group g + 2) goes to LDS and the slot is refilled
          // with group g + 4; the codes slot, consumed above, with g + 2
          if (g + 2 < G) publish_x(cx[d], g + 2);
          fetch_x(cx[d], g + 4 < G ? g + 4 : G - 1);
          fetch_w(cw[d], g + 2 < G ? g + 2 : G - 1);
        }
      }

      if constexpr (SW) {
        // the up results, rounded to bf16 as gather_qmm writes them, meet the
        // gate waves' in LDS over the x buffers (every wave's reads of them
        // are done at the barrier)
        static_assert(BM * BNO * 2 <= (int)sizeof(xs), "up staging fits the x buffers");
        uint16_t* ust = &xs[0][0][0];
        __syncthreads();
        if (wave >= 4) {
#pragma unroll
          for (int i = 0; i < RT; ++i) {
            if (i >= rt) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int lr = i * 16 + 4 * lg + r;
#pragma unroll
              for (int t = 0; t < NT; ++t)
                ust[lr * BNO + 64 * wcol + 16 * t + l16] = (uint16_t)(BF16::pack(acc[i][t][r], 0.0f) & 0xffffu);
            }
          }
        }
        __syncthreads();
        if (wave < 4) {
          // each gate lane replaces the up value it reads with the output
#pragma unroll
          for (int i = 0; i < RT; ++i) {
            if (i >= rt) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int lr = i * 16 + 4 * lg + r;
#pragma unroll
              for (int t = 0; t < NT; ++t) {
                uint16_t& u = ust[lr * BNO + 64 * wcol + 16 * t + l16];
                const float gv = BF16::round(acc[i][t][r]);
                const float uv = BF16::lo((uint32_t)u);
                float o;
                swiglu16<BF16, 1>(&gv, &uv, &o);
                u = (uint16_t)(BF16::pack(o, 0.0f) & 0xffffu);
              }
            }
          }
        }
        __syncthreads();
        // every wave writes the pass's rows: 16-byte pieces, 8 lanes to a
        // 128-byte line (2-byte stores from the MFMA layout wrote 1.70x the
        // output bytes to HBM)
        const int64_t nb = (int64_t)nt * BNO;
        if (yvec) {
          constexpr int PR = BNO / 8;  // pieces per row
          for (int c = tid; c < rp * PR; c += kXpT) {
            const int lr = c / PR, j = c % PR;
            const int64_t n = nb + 8 * j;
            if (n < a.N)
              *reinterpret_cast<u32x4*>(&a.y[(int64_t)list[t0 + lr] * a.ys + n]) =
                  *reinterpret_cast<const u32x4*>(&ust[lr * BNO + 8 * j]);
          }
        } else {
          for (int c = tid; c < rp * BNO; c += kXpT) {
            const int lr = c / BNO, j = c % BNO;
            const int64_t n = nb + j;
            if (n < a.N) a.y[(int64_t)list[t0 + lr] * a.ys + n] = ust[lr * BNO + j];
          }
        }
      } else if (yvec) {
        // per wave and row tile: the 16 x 64 tile through the wave's own LDS
        // slice (pitch 72) and out as 16-byte pieces, 8 lanes to a 128-byte
        // line. At the 4096-token Qwen3-Next MoE prefill the down projection
        // took 211.5 us against 222.9 with 2-byte stores, gate 189.3 / 190.1.
        constexpr int SP = 72;
        __syncthreads();  // every wave's reads of the x buffers are done
        uint16_t* wst = &xs[0][0][0] + wave * 16 * SP;
#pragma unroll
        for (int i = 0; i < RT; ++i) {
          if (i >= rt) continue;
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int t = 0; t < NT; ++t)
              wst[(4 * lg + r) * SP + 16 * t + l16] = (uint16_t)(BF16::pack(acc[i][t][r], 0.0f) & 0xffffu);
          __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
          __builtin_amdgcn_wave_barrier();
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int c = lane + 64 * h, row = c >> 3, j = c & 7;
            const int lr = i * 16 + row;
            const int64_t n = n0 + 8 * j;
            const u32x4 v = *reinterpret_cast<const u32x4*>(&wst[row * SP + 8 * j]);
            if (lr < rp && n < a.N)
              *reinterpret_cast<u32x4*>(&a.y[(int64_t)list[t0 + lr] * a.ys + n]) = v;
          }
          __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
          __builtin_amdgcn_wave_barrier();
        }
      } else {
#pragma unroll
        for (int i = 0; i < RT; ++i) {
          if (i >= rt) continue;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int lr = i * 16 + 4 * lg + r;
            if (lr >= rp) continue;
            const int64_t p = list[t0 + lr];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
              const int64_t n = n0 + 16 * t + l16;
              if (n < a.N) a.y[p * a.ys + n] = (uint16_t)(BF16::pack(acc[i][t][r], 0.0f) & 0xffffu);
            }
          }
        }
      }
    }
  }
}

bool gather_grouped_supported(int dtype, int sdt, int group_size, int bits, const void* x,
                              int64_t xs, const void* w, int64_t k, const void* experts,
                              int64_t pairs) {
  return dtype == DT_BF16 && sdt == DT_BF16 && group_size == 64 && bits == 4 && k % 64 == 0 &&
         (reinterpret_cast<uintptr_t>(x) & 15) == 0 && xs % 8 == 0 &&
         (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(experts) & 15) == 0 && pairs % 4 == 0 &&
         pairs * 4 < ((int64_t)1 << 31);
}

#ifndef HGK_GATHER_XP
#define HGK_GATHER_XP 1
#endif
#ifndef HGK_XP_RT
#define HGK_XP_RT 7
#endif

// The exact-product grouped kernel takes K in units of 8 groups and addresses
// x, the codes, scales and biases with 32-bit buffer offsets.
bool gather_xp_fits(const GatherArgs& a) {
  const int64_t lim = (int64_t)1 << 31;
  return a.K % 512 == 0 && ((a.xrows - 1) * a.xs + a.K) * 2 < lim && a.E * a.N * a.K / 2 < lim &&
         a.E * a.N * (a.K / 64) * 2 < lim;
}

void gather_xp_launch(const GatherArgs& a, hipStream_t s) {
  const int64_t ntiles = (a.N + kXpBN - 1) / kXpBN;
  // column tiles split over about 1024 blocks in all: each block lists its
  // expert's pairs once for its tiles. At 512 experts and 4 tiles (the
  // 2048-column down projection) 1 block per expert measured 224-225 us,
  // against 232 with 2 and 265 with 4 (with 96-row passes 2 had been best:
  // 244 against 261).
  int64_t gx = 1024 / (a.E + 1);
  gx = gx < 1 ? 1 : (gx > ntiles ? ntiles : gx);
  const int64_t tpg = (ntiles + gx - 1) / gx;
  gx = (ntiles + tpg - 1) / tpg;
  const dim3 grid((unsigned)gx, (unsigned)(a.E + 1));
  HGK_LAUNCH((gather_xp_kernel<HGK_XP_RT, false>), grid, dim3(kXpT), 0, s, a);
}

bool gather_swiglu_grouped_launch(const GatherArgs& a, hipStream_t s) {
  if (!HGK_GATHER_XP || !gather_xp_fits(a) || !a.w2 || !a.sc2 || !a.bi2 ||
      (reinterpret_cast<uintptr_t>(a.w2) & 15) != 0)
    return false;
  const int64_t ntiles = (a.N + kXpBN / 2 - 1) / (kXpBN / 2);
  int64_t gx = 1024 / (a.E + 1);
  gx = gx < 1 ? 1 : (gx > ntiles ? ntiles : gx);
  const int64_t tpg = (ntiles + gx - 1) / gx;
  gx = (ntiles + tpg - 1) / tpg;
  const dim3 grid((unsigned)gx, (unsigned)(a.E + 1));
  HGK_LAUNCH((gather_xp_kernel<HGK_XP_RT, true>), grid, dim3(kXpT), 0, s, a);
  return true;
}

void gather_grouped_launch(const GatherArgs& a, hipStream_t s) {
  if (HGK_GATHER_XP && gather_xp_fits(a)) {
    gather_xp_launch(a, s);
    return;
  }
  // column tiles are split over as many blocks as keep about 1024 blocks in
  // the grid; each block scans the expert ids once for all of its tiles
  // (2048, 4096 and 8192 measured slower: 12-40% more time at 512 experts,
  // the scans repeated per block)
  const int64_t ntiles = (a.N + kHlBN - 1) / kHlBN;
  int64_t gx = 1024 / (a.E + 1);
  gx = gx < 1 ? 1 : (gx > ntiles ? ntiles : gx);
  // no block without a column tile (it would scan for nothing)
  const int64_t tpg = (ntiles + gx - 1) / gx;
  gx = (ntiles + tpg - 1) / tpg;
  const dim3 grid((unsigned)gx, (unsigned)(a.E + 1));
  // 8 waves (2 per SIMD) measured 1.44x faster than 4 waves of 64 x 64 tiles
  HGK_LAUNCH((gather_hl_kernel<8>), grid, dim3(512), 0, s, a);
}


template <int MT>
void decode_launch_mt(const QgemmArgs& a, int nt, hipStream_t s) {
  const dim3 grid((unsigned)((a.N + 16 * nt - 1) / (16 * nt))), block(kDecThreads);
  switch (nt) {
    case 1: HGK_LAUNCH((qgemm_decode_kernel<MT, 1, 1>), grid, block, 0, s, a); break;
    case 2: HGK_LAUNCH((qgemm_decode_kernel<MT, 2, 1>), grid, block, 0, s, a); break;
    default: HGK_LAUNCH((qgemm_decode_kernel<MT, 3, 1>), grid, block, 0, s, a); break;
  }
}

// More than 32 rows over enough columns: each block takes one half of the
// rows and twice the columns (96), so a CU reads half of x (128 KB at 64 rows
// of 2048) against twice the codes. At M 64, N 12288, K 2048 this measured
// 13.0-13.15 against 14.3-14.4 us; every output's arithmetic is unchanged.
#ifndef HGK_DEC_MSPLIT
#define HGK_DEC_MSPLIT 1
#endif
#ifndef HGK_DEC_MS_NT
#define HGK_DEC_MS_NT 6
#endif

// The decode kernel takes K in sub-chunks of 512 and addresses x, the codes,
// scales and biases with 32-bit buffer offsets.
bool decode_fits(const QgemmArgs& a) {
  const int64_t lim = (int64_t)1 << 31;
  return a.K % 512 == 0 && ((a.M - 1) * a.xs + a.K) * 2 < lim && a.N * a.K / 2 < lim &&
         a.N * (a.K / 64) * 2 < lim;
}

void decode_launch(const QgemmArgs& a, hipStream_t s) {
  // the widest column tile (16 NT columns per block) that still gives every
  // CU a block
  // (three tiles at most: four hold more registers than a wave has at 64 rows)
  if (HGK_DEC_MSPLIT && a.M > 32) {
    constexpr int NT = HGK_DEC_MS_NT;
    const int64_t tiles = (a.N + 16 * NT - 1) / (16 * NT);
    if (2 * tiles >= kCUs) {
      const dim3 grid((unsigned)(((tiles + 7) / 8) * 16)), block(kDecThreads);
      HGK_LAUNCH((qgemm_decode_kernel<2, NT, 2>), grid, block, 0, s, a);
      return;
    }
  }
  int nt = 3;
  while (nt > 1 && (a.N + 16 * nt - 1) / (16 * nt) < kCUs) --nt;
  switch ((a.M + 15) / 16) {
    case 1: decode_launch_mt<1>(a, nt, s); break;
    case 2: decode_launch_mt<2>(a, nt, s); break;
    case 3: decode_launch_mt<3>(a, nt, s); break;
    default: decode_launch_mt<4>(a, nt, s); break;
  }
}

bool qgemm_supported(int dtype, int sdt, int group_size, int bits, const void* x, int64_t xs,
                     const void* w, int64_t k) {
  return dtype == DT_BF16 && sdt == DT_BF16 && group_size == 64 && bits == 4 && k % 64 == 0 &&
         (reinterpret_cast<uintptr_t>(x) & 15) == 0 && xs % 8 == 0 &&
         (reinterpret_cast<uintptr_t>(w) & 7) == 0 && ((k / 8) % 2) == 0;
}

void qgemm_launch(const QgemmArgs& a, hipStream_t s) {
  const unsigned gx = (unsigned)((a.N + kQgBN - 1) / kQgBN);
  if (a.M <= 64 && decode_fits(a)) {
    decode_launch(a, s);
  } else if (a.M <= 512) {
    HGK_LAUNCH(qgemm_kernel<64>, dim3(gx, (unsigned)((a.M + 63) / 64)), dim3(256), 0, s, a);
  } else {
    // 8 waves of 64 x 64 measured faster than 4 waves of 128 x 64
    HGK_LAUNCH((qgemm_hl_kernel<4, 4>), dim3(gx, (unsigned)((a.M + kHlBM - 1) / kHlBM)),
               dim3(512), 0, s, a);
  }
}

}  // namespace hgk
