/*
 * oracle.c -- CPU restatement of MLX 0.25-era CPU-device semantics for the ops
 * higgs-models calls through mlx-rs. TEST INFRASTRUCTURE ONLY (see oracle.h):
 * used by tests/, the smoke check and the benchmark's CPU-baseline leg as the
 * checker, never by the shipped library.
 *
 * Build flags matter: -ffp-contract=off (every product and sum is rounded
 * separately, as MLX's separately materialised ops are), no -ffast-math.
 *
 * Conventions: rnd(v, T) rounds an f32 value to dtype T with
 * round-to-nearest-even and returns it as f32 (identity for f32). All
 * transcendental functions are evaluated in f32.
 *
 * Unpinned points (only an import of MLX could settle them; the product
 * follows the same choice, and the bf16 1-ulp tolerance absorbs either way):
 *  U1 rms_norm: the sum of squares is accumulated in f64 and rounded once to
 *     f32 (order-independent); MLX reduces in f32 with SIMD partial sums, so
 *     the last f32 bit of the mean may differ by its summation error.
 *  U2 rope: positions are f32 ((f32(l) + offset) * scale) and the inverse
 *     frequencies f32; cos/sin are rounded to the activation dtype before the
 *     products.
 *  U3 sigmoid: MLX's CPU Sigmoid is 1/(1+exp(|x|)) selected/complemented by
 *     sign, using MLX's own polynomial exp; here the exp result is kept in f32
 *     for every activation dtype.
 *  U4 gelu_approximate: the scalar constants are f32 arrays, so a bf16 input is
 *     promoted and the op runs entirely in f32; only the final result is
 *     rounded to the requested output dtype.
 *  U5 dequantize: rnd(rnd(q*s) + b) in the scales dtype (two roundings, as the
 *     multiply and add are separate MLX ops).
 *  U6 gemma (1+w): the +1 is an f32 add at load time (gemma2.rs:802,813),
 *     which promotes the weight and hence the norm output to f32.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <stdint.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* bit-level conversions                                               */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t or_f32_to_bf16(float v) {
  uint32_t x = f2u(v);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

float or_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

uint16_t or_f32_to_f16(float v) {
  uint32_t x = f2u(v);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> inf */
  if (ax < 0x38800000u) {
    /* half subnormal (or zero): value / 2^-24 rounded to an integer, RNE */
    float t = u2f(ax) * 16777216.0f; /* exact power-of-two scaling */
    uint32_t m = (uint32_t)nearbyintf(t);
    return (uint16_t)(sign | m);
  }
  uint32_t mant = ax & 0x7fffffu;
  uint32_t e = (ax >> 23) - 127u + 15u;
  uint32_t h = (e << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

float or_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  if (e == 0) {
    float v = (float)m * (1.0f / 16777216.0f); /* exact */
    return sign ? -v : v;
  }
  if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
  return u2f(sign | ((e - 15u + 127u) << 23) | (m << 13));
}

static inline float rnd(float v, int dt) {
  switch (dt) {
    case OR_BF16: return or_bf16_to_f32(or_f32_to_bf16(v));
    case OR_F16: return or_f16_to_f32(or_f32_to_f16(v));
    default: return v;
  }
}

static inline float ld(const void* p, int dt, int64_t i) {
  switch (dt) {
    case OR_BF16: return or_bf16_to_f32(((const uint16_t*)p)[i]);
    case OR_F16: return or_f16_to_f32(((const uint16_t*)p)[i]);
    default: return ((const float*)p)[i];
  }
}

static inline void st(void* p, int dt, int64_t i, float v) {
  switch (dt) {
    case OR_BF16: ((uint16_t*)p)[i] = or_f32_to_bf16(v); break;
    case OR_F16: ((uint16_t*)p)[i] = or_f32_to_f16(v); break;
    default: ((float*)p)[i] = v; break;
  }
}

static inline int is_float_dt(int dt) { return dt == OR_F32 || dt == OR_BF16 || dt == OR_F16; }

/* MLX promote_types restricted to the float types: equal -> same; anything
 * with f32 -> f32; bf16 with f16 -> f32. */
int or_promote(int a, int b) {
  if (a == b) return a;
  return OR_F32;
}

/* ------------------------------------------------------------------ */
/* MLX CPU math                                                        */
/* ------------------------------------------------------------------ */

/* MLX's CPU exp for float types (mlx/backend/cpu/simd/math.h of the 0.2x
 * releases): x*log2(e) split into integer and fractional parts, 2^frac by the
 * degree-6 minimax polynomial of Cephes exp2f (S. L. Moshier), 2^int built
 * in the exponent field; NaN passes through, x > 88 -> inf, x < -88 -> 0. */
float or_mlx_exp(float x_init) {
  if (isnan(x_init)) return x_init;
  if (x_init > 88.0f) return INFINITY;
  if (x_init < -88.0f) return 0.0f;
  float x = x_init * 1.442695f;
  float ipart = floorf(x + 0.5f);
  float fpart = x - ipart;
  float p = 1.535336188319500e-4f;
  p = fmaf(p, fpart, 1.339887440266574e-3f);
  p = fmaf(p, fpart, 9.618437357674640e-3f);
  p = fmaf(p, fpart, 5.550332471162809e-2f);
  p = fmaf(p, fpart, 2.402264791363012e-1f);
  p = fmaf(p, fpart, 6.931472028550421e-1f);
  p = fmaf(p, fpart, 1.000000000000000f);
  uint32_t ebits = (uint32_t)((int32_t)ipart + 127) << 23;
  return u2f(ebits) * p;
}

/* MLX CPU Sigmoid: y = 1/(1+exp(|x|)); x<0 -> y, else 1-y (f32). */
float or_mlx_sigmoid(float x) {
  float y = 1.0f / (1.0f + or_mlx_exp(fabsf(x)));
  return x < 0.0f ? y : 1.0f - y;
}

/* ------------------------------------------------------------------ */
/* deterministic inputs                                                */
/* ------------------------------------------------------------------ */

/* i-th output of a splitmix64 generator seeded with `key` */
static inline uint64_t sm64_at(uint64_t key, uint64_t i) {
  uint64_t z = key + (i + 1u) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static inline double u01(uint64_t key, uint64_t i) {
  return (double)(sm64_at(key, i) >> 40) * (1.0 / 16777216.0); /* [0,1) */
}

void or_fill_normal(uint64_t key, float mean, float stdev, float* out, int64_t n) {
  const double two_pi = 6.283185307179586476925286766559;
  int64_t pairs = (n + 1) / 2;
#pragma omp parallel for schedule(static)
  for (int64_t k = 0; k < pairs; ++k) {
    double a = 1.0 - u01(key, (uint64_t)(2 * k)); /* (0,1] */
    double b = u01(key, (uint64_t)(2 * k + 1));
    double r = sqrt(-2.0 * log(a));
    out[2 * k] = (float)(mean + stdev * r * cos(two_pi * b));
    if (2 * k + 1 < n) out[2 * k + 1] = (float)(mean + stdev * r * sin(two_pi * b));
  }
}

void or_fill_uniform(uint64_t key, float lo, float hi, float* out, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i)
    out[i] = (float)((double)lo + ((double)hi - (double)lo) * u01(key, (uint64_t)i));
}

void or_fill_u32(uint64_t key, uint32_t* out, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = (uint32_t)(sm64_at(key, (uint64_t)i) >> 32);
}

void or_fill_ids(uint64_t key, uint32_t v, uint32_t* out, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i)
    out[i] = (uint32_t)(((sm64_at(key, (uint64_t)i) >> 32) * (uint64_t)v) >> 32);
}

void or_fill_offsets(uint64_t key, int32_t lo, int32_t hi, int32_t* out, int64_t n) {
  uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo + 1);
  for (int64_t i = 0; i < n; ++i)
    out[i] = (int32_t)((int64_t)lo + (int64_t)(((sm64_at(key, (uint64_t)i) >> 32) * span) >> 32));
}

void or_convert_from_f32(int dt, const float* in, void* out, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) st(out, dt, i, in[i]);
}

void or_convert_to_f32(int dt, const void* in, float* out, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = ld(in, dt, i);
}

/* ------------------------------------------------------------------ */
/* RMSNorm (fast::rms_norm CPU fallback)                               */
/* ------------------------------------------------------------------ */

/* One row: returns the f32 scale r = rsqrt(mean(x^2) + eps).
 * The sum of squares is accumulated in f64 (each square of an f32 value is
 * exact there) and rounded once to f32: an order-independent f32 sum, which
 * MLX's SIMD f32 reduction matches to its own summation error (U1). */
static inline float row_rsqrt(const void* x, int dt, int64_t base, int64_t n, float eps) {
  float inv_n = (float)(1.0 / (double)n); /* NumberOfElements(inverted) cast to f32 */
  double s = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    double v = (double)ld(x, dt, base + i);
    s = s + v * v;
  }
  float ms = (float)s * inv_n;
  return 1.0f / sqrtf(ms + eps);
}

int or_rms_norm(const void* x, int x_dt, int64_t x_rs, const void* w, int w_dt,
                int plus_one, float eps, void* y, int y_dt, int64_t y_rs,
                int64_t rows, int64_t n) {
  if (!x || !y || rows < 0 || n <= 0 || !is_float_dt(x_dt) || !is_float_dt(y_dt)) return 1;
  if (w && !is_float_dt(w_dt)) return 1;
  int w_eff = w ? (plus_one ? OR_F32 : w_dt) : x_dt;
  int t_out = or_promote(x_dt, w_eff);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    float rr = row_rsqrt(x, x_dt, r * x_rs, n, eps);
    for (int64_t i = 0; i < n; ++i) {
      float v = ld(x, x_dt, r * x_rs + i);
      float nv = rnd(v * rr, t_out);
      float o = nv;
      if (w) {
        float wv = ld(w, w_dt, i);
        if (plus_one) wv = wv + 1.0f;
        o = rnd(nv * wv, t_out);
      }
      st(y, y_dt, r * y_rs + i, o);
    }
  }
  return 0;
}

/* MLX's elementwise add on dtype dt: both operands widened to f32, one f32
 * add, one rounding to dt (the `x.add(residual)` of transformer.rs:413 and
 * 417; gemma2.rs:498, 504; qwen3_next.rs:1539, 1544). Rows of n elements with
 * separate row strides; out may be a or b itself. */
int or_add(int dt, const void* a, int64_t a_rs, const void* b, int64_t b_rs,
           void* out, int64_t o_rs, int64_t rows, int64_t n) {
  if (!a || !b || !out || rows < 0 || n < 0 || !is_float_dt(dt)) return 1;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t i = 0; i < n; ++i)
      st(out, dt, r * o_rs + i, rnd(ld(a, dt, r * a_rs + i) + ld(b, dt, r * b_rs + i), dt));
  return 0;
}

/* ------------------------------------------------------------------ */
/* RoPE                                                                */
/* ------------------------------------------------------------------ */

void or_rope_inv_freq(float base, int dims, const float* freqs, float* inv_out) {
  int half = dims / 2;
  if (freqs) {
    for (int i = 0; i < half; ++i) inv_out[i] = 1.0f / freqs[i];
    return;
  }
  /* exp(arange(0, -half, -1, f32) * f32(log(base) / half)) */
  float c = logf(base) / (float)half;
  for (int i = 0; i < half; ++i) inv_out[i] = or_mlx_exp((float)(-i) * c);
}

/* mlx-lm Llama3RoPE.__init__ evaluated in f32 (python scalars are weak and
 * take the array's f32 type). */
void or_llama3_freqs(float base, int dims, float factor, float low, float high,
                     float old_ctx, float* f) {
  int half = dims / 2;
  float low_wl = (float)((double)old_ctx / (double)low);
  float high_wl = (float)((double)old_ctx / (double)high);
  float two_pi = (float)6.283185307179586;
  float band = (float)((double)high - (double)low);
  for (int i = 0; i < half; ++i) {
    float e = (float)(2 * i) / (float)dims;
    float fr = powf(base, e);
    float wl = two_pi * fr;
    if (wl > low_wl) fr = fr * factor;
    int medium = (wl > high_wl) && (wl < low_wl);
    float sm = (old_ctx / wl - low) / band;
    float smooth = fr / ((1.0f - sm) / factor + sm);
    f[i] = medium ? smooth : fr;
  }
}

int or_norm_rope(int x_dt, const void* x, const int64_t xs[3], void* y,
                 const int64_t ys[3], int64_t B, int64_t L, int64_t H, int64_t D,
                 const void* norm_w, int w_dt, float eps, int dims,
                 const float* inv_freq, float scale, int32_t offset,
                 const int32_t* offsets) {
  return or_norm_rope_trig(x_dt, x, xs, y, ys, B, L, H, D, norm_w, w_dt, eps, dims, inv_freq,
                           scale, offset, offsets, OR_TRIG_LIBM);
}

/* cos/sin of the f32 angle th: libm's f32 cosf/sinf (MLX's CPU evaluation),
 * or the f32 rounding of the f64 cos/sin of th (the device kernels' choice).
 * The two agree except where the f32 functions miss the correctly rounded
 * value by their last bit. */
static inline void rope_trig(float th, int trig, float* c, float* s) {
  if (trig == OR_TRIG_F64) {
    *c = (float)cos((double)th);
    *s = (float)sin((double)th);
  } else {
    *c = cosf(th);
    *s = sinf(th);
  }
}

int or_norm_rope_trig(int x_dt, const void* x, const int64_t xs[3], void* y,
                      const int64_t ys[3], int64_t B, int64_t L, int64_t H, int64_t D,
                      const void* norm_w, int w_dt, float eps, int dims,
                      const float* inv_freq, float scale, int32_t offset,
                      const int32_t* offsets, int trig) {
  if (trig != OR_TRIG_LIBM && trig != OR_TRIG_F64) return 1;
  if (!x || !y || !inv_freq || B < 0 || L < 0 || H < 0 || D <= 0) return 1;
  if (dims <= 0 || dims > D || (dims & 1)) return 1;
  if (D > 4096 || dims > 1024) return 2; /* per-thread scratch rows below */
  int t = norm_w ? or_promote(x_dt, w_dt) : x_dt;
  int half = dims / 2;
  int64_t tokens = B * L;
#pragma omp parallel
  {
    float cs[512], sn[512], row[4096];
#pragma omp for schedule(static)
    for (int64_t tk = 0; tk < tokens; ++tk) {
      int64_t b = tk / L, l = tk % L;
      int32_t off = offsets ? offsets[b] : offset;
      float pos = ((float)l + (float)off) * scale;
      for (int i = 0; i < half; ++i) {
        float th = pos * inv_freq[i], c, sv;
        rope_trig(th, trig, &c, &sv);
        cs[i] = rnd(c, t);
        sn[i] = rnd(sv, t);
      }
      for (int64_t h = 0; h < H; ++h) {
        int64_t xb = b * xs[0] + l * xs[1] + h * xs[2];
        int64_t yb = b * ys[0] + l * ys[1] + h * ys[2];
        if (norm_w) {
          float rr = row_rsqrt(x, x_dt, xb, D, eps);
          for (int64_t d = 0; d < D; ++d) {
            float nv = rnd(ld(x, x_dt, xb + d) * rr, t);
            row[d] = rnd(nv * ld(norm_w, w_dt, d), t);
          }
        } else {
          for (int64_t d = 0; d < D; ++d) row[d] = ld(x, x_dt, xb + d);
        }
        for (int i = 0; i < half; ++i) {
          float a = row[i], bb = row[i + half];
          float y1 = rnd(rnd(a * cs[i], t) - rnd(bb * sn[i], t), t);
          float y2 = rnd(rnd(a * sn[i], t) + rnd(bb * cs[i], t), t);
          st(y, t, yb + i, y1);
          st(y, t, yb + i + half, y2);
        }
        for (int64_t d = dims; d < D; ++d) st(y, t, yb + d, row[d]);
      }
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ */
/* GLU activations                                                     */
/* ------------------------------------------------------------------ */

static inline float silu_mul(float g, float u, int t) {
  float sg = rnd(or_mlx_sigmoid(g), t);
  float s = rnd(g * sg, t);
  return rnd(s * u, t);
}

static inline float gelu_tanh_mul(float g, float u) {
  /* 0.5 * x * (1 + tanh(sqrt(2/pi) * (x + 0.044715 * x^3))), all f32 */
  const float k0 = 0.7978845608028654f, k1 = 0.044715f;
  float x3 = g * g * g;
  float inner = k0 * (g + k1 * x3);
  float gl = (0.5f * g) * (1.0f + tanhf(inner));
  return gl * u;
}

int or_glu(int act, int x_dt, const void* gate, int64_t g_rs, const void* up,
           int64_t u_rs, void* out, int out_dt, int64_t o_rs, int64_t rows, int64_t n) {
  if (!gate || !up || !out || rows < 0 || n < 0) return 1;
  if (act != OR_ACT_SILU && act != OR_ACT_GELU_TANH) return 2;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t i = 0; i < n; ++i) {
      float g = ld(gate, x_dt, r * g_rs + i), u = ld(up, x_dt, r * u_rs + i);
      float o = act == OR_ACT_SILU ? silu_mul(g, u, x_dt) : gelu_tanh_mul(g, u);
      st(out, out_dt, r * o_rs + i, o);
    }
  }
  return 0;
}

/* swiglu(z, norm(y)) = z * sigmoid(z) * rms_norm(y, w) */
int or_gated_rms_norm(int x_dt, const void* y, int64_t y_rs, const void* z,
                      int64_t z_rs, const void* w, int w_dt, float eps, void* out,
                      int out_dt, int64_t o_rs, int64_t rows, int64_t n) {
  if (!y || !z || !w || !out || rows < 0 || n <= 0) return 1;
  int t_n = or_promote(x_dt, w_dt);
  int t_o = or_promote(x_dt, t_n);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    float rr = row_rsqrt(y, x_dt, r * y_rs, n, eps);
    for (int64_t i = 0; i < n; ++i) {
      float nv = rnd(ld(y, x_dt, r * y_rs + i) * rr, t_n);
      nv = rnd(nv * ld(w, w_dt, i), t_n);
      float zv = ld(z, x_dt, r * z_rs + i);
      float sg = rnd(or_mlx_sigmoid(zv), x_dt);
      float a = rnd(zv * sg, x_dt);
      st(out, out_dt, r * o_rs + i, rnd(a * nv, t_o));
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ */
/* 4-bit affine QuantizedEmbedding                                     */
/* ------------------------------------------------------------------ */

int or_qembed(const void* ids, int id_dt, int64_t n_ids, const uint32_t* wq,
              const void* scales, const void* biases, int s_dt, int64_t vocab,
              int64_t hidden, int group, int bits, float out_scale, void* out) {
  if (!ids || !wq || !scales || !biases || !out || n_ids < 0 || vocab <= 0) return 1;
  if (bits != 4 || group <= 0 || hidden % group || group % 8) return 2;
  if (id_dt != OR_U32 && id_dt != OR_I32) return 1;
  int64_t wpr = hidden / 8, gpr = hidden / group;
  float sc = out_scale != 0.0f ? rnd(out_scale, s_dt) : 0.0f;
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < n_ids; ++t) {
    int64_t id;
    if (id_dt == OR_I32) {
      id = ((const int32_t*)ids)[t];
      if (id < 0) id += vocab; /* take: negative indices count from the end */
    } else {
      id = ((const uint32_t*)ids)[t];
    }
    if (id < 0 || id >= vocab) { /* out of range: defined as a zero row */
      for (int64_t k = 0; k < hidden; ++k) st(out, s_dt, t * hidden + k, 0.0f);
      continue;
    }
    for (int64_t k = 0; k < hidden; ++k) {
      uint32_t word = wq[id * wpr + k / 8];
      uint32_t q = (word >> (4 * (k % 8))) & 0xfu;
      float s = ld(scales, s_dt, id * gpr + k / group);
      float b = ld(biases, s_dt, id * gpr + k / group);
      float v = rnd(rnd((float)q * s, s_dt) + b, s_dt);
      if (out_scale != 0.0f) v = rnd(v * sc, s_dt);
      st(out, s_dt, t * hidden + k, v);
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ */
/* gather_qmm (4-bit affine, transpose = true, one row per pair)       */
/* ------------------------------------------------------------------ */

/* y[p, n] = round_dt( sum_k x[row(p), k] * (s * q + b) ), the sum taken in
 * f64 over exactly dequantized weights (s * q + b is exact in f64 for 16-bit
 * s, b and 4-bit q), i.e. the mathematical value rounded once. MLX's own
 * accumulation order and precision for quantized matmul are not restated:
 * the parity bar for this floating-point contraction is a tolerance.
 * Call sites: SwitchMlpWeights::forward_gather -> gather_qmm
 * (crates/higgs-models/src/qwen3_next.rs:844-904, 294-363). row(p) = lhs[p]
 * when lhs is given, else p / x_div; rows or experts out of range give 0. */
int or_gather_qmm(int dt, const void* x, int64_t x_rows, int64_t x_rs, int64_t x_div,
                  const int32_t* lhs, const uint32_t* w, const void* sc, const void* bi,
                  int s_dt, int64_t E, int64_t N, int64_t K, int group, const int32_t* experts,
                  int64_t pairs, void* y, int64_t y_rs) {
  if (!x || !w || !sc || !bi || !experts || !y || K % group || K % 8 || x_div <= 0) return 1;
  const int64_t gpr = K / group, wpr = K / 8;
#pragma omp parallel for schedule(static)
  for (int64_t p = 0; p < pairs; ++p) {
    int64_t e = experts[p];
    if (e < 0) e += E;
    int64_t r = lhs ? (int64_t)lhs[p] : p / x_div;
    if (lhs && r < 0) r += x_rows;
    const int ok = e >= 0 && e < E && r >= 0 && r < x_rows;
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0;
      if (ok) {
        const uint32_t* wr = w + (e * N + n) * wpr;
        for (int64_t k = 0; k < K; ++k) {
          const uint32_t q = (wr[k / 8] >> (4 * (k % 8))) & 0xfu;
          const int64_t g = (e * N + n) * gpr + k / group;
          const double wv = (double)ld(sc, s_dt, g) * (double)q + (double)ld(bi, s_dt, g);
          acc += (double)ld(x, dt, r * x_rs + k) * wv;
        }
      }
      st(y, dt, p * y_rs + n, rnd((float)acc, dt));
    }
  }
  return 0;
}

/* ------------------------------------------------------------------ */
/* GatedDeltaNet recurrence                                            */
/* ------------------------------------------------------------------ */

/* The gated-delta recurrence of the reference's Metal kernel
 * (crates/higgs-models/src/qwen3_next.rs:376-451), here in f64 per state row:
 *   g = exp(-exp(a_log) * softplus(a_t + dt_bias)), beta = sigmoid(b_t)
 *   s = s * g; kv = s.k_t; delta = (v_t - kv) * beta; s = s + k_t * delta;
 *   y_t = s.q_t
 * with q, k [B,T,Hk,Dk], v [B,T,Hv,Dv], a, b [B,T,Hv], a_log, dt_bias [Hv]
 * (dtype p_dt), state [B,Hv,Dv,Dk] read and written in dt (state_in may be
 * NULL: zeros). When qw/kw are given, q and k are first normalised as
 * or_rms_norm(x, w, eps) rows of Dk in dt (qwen3_next.rs:1172-1173). The
 * reference kernel runs in f32 with its own reduction order: the parity bar
 * against this f64 restatement is a tolerance. */
int or_gated_delta(int dt, const void* q, const void* k, const void* v, const void* a_log,
                   const void* a, const void* dt_bias, const void* b, int p_dt,
                   const void* state_in, const void* qw, const void* kw, float eps,
                   int64_t B, int64_t T, int64_t Hk, int64_t Dk, int64_t Hv, int64_t Dv,
                   void* y, void* state_out) {
  if (!q || !k || !v || !a_log || !a || !dt_bias || !b || !y || !state_out || Hv % Hk) return 1;
  const size_t es = dt == OR_F32 ? 4 : 2;
  const void* qn = q;
  const void* kn = k;
  void* qbuf = NULL;
  void* kbuf = NULL;
  if (qw && kw) {
    const int64_t rows = B * T * Hk;
    qbuf = malloc((size_t)(rows * Dk) * es);
    kbuf = malloc((size_t)(rows * Dk) * es);
    if (!qbuf || !kbuf) { free(qbuf); free(kbuf); return 1; }
    or_rms_norm(q, dt, Dk, qw, dt, 0, eps, qbuf, dt, Dk, rows, Dk);
    or_rms_norm(k, dt, Dk, kw, dt, 0, eps, kbuf, dt, Dk, rows, Dk);
    qn = qbuf;
    kn = kbuf;
  }
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t bi = 0; bi < B; ++bi) {
    for (int64_t hv = 0; hv < Hv; ++hv) {
      const int64_t hk = hv / (Hv / Hk);
      const double A = exp((double)ld(a_log, p_dt, hv));
      const double dtb = (double)ld(dt_bias, p_dt, hv);
      double* sv = (double*)malloc((size_t)(Dv * Dk) * sizeof(double));
      for (int64_t d = 0; d < Dv * Dk; ++d)
        sv[d] = state_in ? (double)ld(state_in, dt, (bi * Hv + hv) * Dv * Dk + d) : 0.0;
      for (int64_t t = 0; t < T; ++t) {
        const double x = (double)ld(a, dt, (bi * T + t) * Hv + hv) + dtb;
        const double sp = (x > 0.0 ? x : 0.0) + log1p(exp(-fabs(x)));
        const double g = exp(-A * sp);
        const double beta = 1.0 / (1.0 + exp(-(double)ld(b, dt, (bi * T + t) * Hv + hv)));
        const int64_t qk = ((bi * T + t) * Hk + hk) * Dk;
        for (int64_t dv = 0; dv < Dv; ++dv) {
          double* s = sv + dv * Dk;
          double kv = 0.0;
          for (int64_t i = 0; i < Dk; ++i) {
            s[i] *= g;
            kv += s[i] * (double)ld(kn, dt, qk + i);
          }
          const double delta = ((double)ld(v, dt, ((bi * T + t) * Hv + hv) * Dv + dv) - kv) * beta;
          double out = 0.0;
          for (int64_t i = 0; i < Dk; ++i) {
            s[i] += (double)ld(kn, dt, qk + i) * delta;
            out += s[i] * (double)ld(qn, dt, qk + i);
          }
          st(y, dt, ((bi * T + t) * Hv + hv) * Dv + dv, rnd((float)out, dt));
        }
      }
      for (int64_t d = 0; d < Dv * Dk; ++d)
        st(state_out, dt, (bi * Hv + hv) * Dv * Dk + d, rnd((float)sv[d], dt));
      free(sv);
    }
  }
  free(qbuf);
  free(kbuf);
  return 0;
}
