// hgk_common.h -- shared device helpers for the gfx950 per-layer op kernels.
//
// Element types travel as 16-bit or 32-bit storage words; every kernel loads
// and stores 16-byte chunks (8 x bf16/f16 or 4 x f32 per lane), converts to
// f32, and rounds back to the storage type exactly where MLX's CPU-device
// composition of the op materialises an intermediate.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hgk {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

enum Dtype { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2, DT_U32 = 3, DT_I32 = 4 };

__host__ __device__ inline uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ inline float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// Materialise an f32 value in a register before it is narrowed. Without it
// the backend may fold `fptrunc(a * b)` into a mixed-precision FMA
// (v_fma_mixlo_f16: a*b rounded once, straight to 16 bits), whereas the ops
// being reproduced round the product to f32 first and then to 16 bits.
__device__ inline float f32_barrier(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

// ---------------------------------------------------------------- types
struct BF16 {
  static constexpr int kCode = DT_BF16;
  static constexpr int kBytes = 2;
  __device__ static float lo(uint32_t w) { return u2f(w << 16); }
  __device__ static float hi(uint32_t w) { return u2f(w & 0xffff0000u); }
  // Two f32 -> packed pair, round-to-nearest-even (v_cvt_pk_bf16_f32).
  __device__ static uint32_t pack(float a, float b) {
    f32x2 v = {f32_barrier(a), f32_barrier(b)};
    bf16x2 h = __builtin_convertvector(v, bf16x2);
    return __builtin_bit_cast(uint32_t, h);
  }
  // a rounded to bf16, as f32: one v_cvt_pk_bf16_f32 with +0 in the low half,
  // whose result is the f32 bit pattern of the rounded value
  __device__ static float round(float a) {
    f32x2 v = {0.0f, f32_barrier(a)};
    return __builtin_bit_cast(float, __builtin_convertvector(v, bf16x2));
  }
};

struct F16 {
  static constexpr int kCode = DT_F16;
  static constexpr int kBytes = 2;
  __device__ static float lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  }
  __device__ static float hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  }
  __device__ static uint32_t pack(float a, float b) {
    f32x2 v = {f32_barrier(a), f32_barrier(b)};
    f16x2 h = __builtin_convertvector(v, f16x2);
    return __builtin_bit_cast(uint32_t, h);
  }
  __device__ static float round(float a) { return (float)(_Float16)f32_barrier(a); }
};

struct F32 {
  static constexpr int kCode = DT_F32;
  static constexpr int kBytes = 4;
  __device__ static float round(float a) { return a; }
};

// Elements of T per 16-byte chunk.
template <class T> struct Vec { static constexpr int N = 16 / T::kBytes; };

// Round two f32 values to T in place: bf16 with one conversion each (the
// rounded value lands in the high half, where it is already an f32); f16
// with one packed conversion and two widenings.
template <class T>
__device__ inline void round2(float& a, float& b) {
  if constexpr (T::kCode == DT_BF16) {
    a = T::round(a);
    b = T::round(b);
  } else if constexpr (T::kBytes == 2) {
    const uint32_t p = T::pack(a, b);
    a = T::lo(p);
    b = T::hi(p);
  }
}

// ---------------------------------------------------------------- chunk I/O
template <class T>
__device__ inline void unpack16(u32x4 r, float* v) {
  if constexpr (T::kBytes == 2) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[2 * k] = T::lo(r[k]);
      v[2 * k + 1] = T::hi(r[k]);
    }
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = u2f(r[k]);
  }
}

// Raw 16-byte load of the chunk starting at element `e` of T (kept packed in
// registers until used: half the VGPRs of unpacked f32 for 16-bit types).
template <class T>
__device__ inline u32x4 ld16(const void* base, int64_t e) {
  return *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(base) + e * T::kBytes);
}

// The same load with the non-temporal hint, for streams read exactly once in
// whole 128-byte lines per instruction: on MI355X such streams run 7-10 %
// closer to peak HBM bandwidth than with default-policy loads. Data read in
// pieces of a line by several instructions (gathers, half rows) keeps the
// default policy: a non-temporal read does not keep the line for the next.
template <class T>
__device__ inline u32x4 ld16_nt(const void* base, int64_t e) {
  return __builtin_nontemporal_load(
      reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(base) + e * T::kBytes));
}

// Element k of a packed run of T held in 32-bit words.
template <class T>
__device__ inline float elem(const uint32_t* w, int k) {
  if constexpr (T::kBytes == 2) return (k & 1) ? T::hi(w[k >> 1]) : T::lo(w[k >> 1]);
  else return u2f(w[k]);
}

template <class T>
__device__ inline float elem(const u32x4& r, int k) {
  if constexpr (T::kBytes == 2) return (k & 1) ? T::hi(r[k >> 1]) : T::lo(r[k >> 1]);
  else return u2f(r[k]);
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <class T>
__device__ inline float elem(const u32x2& r, int k) {
  if constexpr (T::kBytes == 2) return (k & 1) ? T::hi(r[k >> 1]) : T::lo(r[k >> 1]);
  else return u2f(r[k]);
}

// NB bytes of packed elements held as one vector of 32-bit words, moved with
// one load or store instruction (NB = 8 or 16).
template <int NB> struct RawVec;
template <> struct RawVec<8> { typedef u32x2 type; };
template <> struct RawVec<16> { typedef u32x4 type; };

template <int NB>
__device__ inline typename RawVec<NB>::type ld_raw(const void* base, int64_t byte_off) {
  return *reinterpret_cast<const typename RawVec<NB>::type*>(
      reinterpret_cast<const char*>(base) + byte_off);
}

template <int NB>
__device__ inline typename RawVec<NB>::type ld_raw_nt(const void* base, int64_t byte_off) {
  return __builtin_nontemporal_load(reinterpret_cast<const typename RawVec<NB>::type*>(
      reinterpret_cast<const char*>(base) + byte_off));
}

template <int NB>
__device__ inline void st_raw_nt(void* base, int64_t byte_off, typename RawVec<NB>::type v) {
  __builtin_nontemporal_store(
      v, reinterpret_cast<typename RawVec<NB>::type*>(reinterpret_cast<char*>(base) + byte_off));
}

// Load Vec<T>::N elements of T starting at element `e` (16-byte aligned).
template <class T>
__device__ inline void load_chunk(const void* base, int64_t e, float* v) {
  const u32x4* p = reinterpret_cast<const u32x4*>(
      reinterpret_cast<const char*>(base) + e * T::kBytes);
  unpack16<T>(*p, v);
}

// Load N elements of T starting at element e (N * sizeof(T) a multiple of 16).
template <class T, int N>
__device__ inline void load_elems(const void* base, int64_t e, float* v) {
  constexpr int kPer = Vec<T>::N;
  if constexpr (N * T::kBytes == 8) {
    // half chunk: 4 x 16-bit (8-byte aligned)
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 r = *reinterpret_cast<const u32x2*>(reinterpret_cast<const char*>(base) +
                                                    e * T::kBytes);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      v[2 * k] = T::lo(r[k]);
      v[2 * k + 1] = T::hi(r[k]);
    }
  } else {
    static_assert(N % kPer == 0, "whole chunks only");
#pragma unroll
    for (int c = 0; c < N / kPer; ++c) load_chunk<T>(base, e + c * kPer, v + c * kPer);
  }
}

// Store N f32 values as T at element e (values are rounded to T, RNE).
template <class T, int N, bool NT = true>
__device__ inline void store_elems(void* base, int64_t e, const float* v) {
  constexpr int kPer = Vec<T>::N;
  static_assert(N % kPer == 0, "whole chunks only");
#pragma unroll
  for (int c = 0; c < N / kPer; ++c) {
    u32x4 w;
    if constexpr (T::kBytes == 2) {
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = T::pack(v[c * kPer + 2 * k], v[c * kPer + 2 * k + 1]);
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) w[k] = f2u(v[c * kPer + k]);
    }
    u32x4* p = reinterpret_cast<u32x4*>(reinterpret_cast<char*>(base) +
                                        (e + c * kPer) * T::kBytes);
    if constexpr (NT) __builtin_nontemporal_store(w, p);
    else *p = w;
  }
}

// Load N weights of runtime dtype wdt (bf16/f16/f32) starting at element e.
template <int N>
__device__ inline void load_weights(const void* w, int wdt, int64_t e, float* v) {
  if (wdt == DT_BF16) load_elems<BF16, N>(w, e, v);
  else if (wdt == DT_F16) load_elems<F16, N>(w, e, v);
  else load_elems<F32, N>(w, e, v);
}

// Scalar load / store for the generic (unaligned / odd-size) fallbacks.
template <class T>
__device__ inline float load1(const void* base, int64_t e) {
  if constexpr (T::kBytes == 2) {
    uint16_t h = reinterpret_cast<const uint16_t*>(base)[e];
    return T::lo((uint32_t)h);
  } else {
    return reinterpret_cast<const float*>(base)[e];
  }
}

__device__ inline float load1_dt(const void* base, int dt, int64_t e) {
  if (dt == DT_BF16) return load1<BF16>(base, e);
  if (dt == DT_F16) return load1<F16>(base, e);
  return load1<F32>(base, e);
}

template <class T>
__device__ inline void store1(void* base, int64_t e, float v) {
  if constexpr (T::kBytes == 2) {
    reinterpret_cast<uint16_t*>(base)[e] = (uint16_t)(T::pack(v, 0.0f) & 0xffffu);
  } else {
    reinterpret_cast<float*>(base)[e] = v;
  }
}

// ---------------------------------------------------------------- math
// MLX's CPU exp for float types: x*log2(e) split into integer and fractional
// parts, 2^frac by the degree-6 Cephes exp2f minimax polynomial (Moshier),
// 2^int assembled in the exponent field; NaN passes through, x > 88 -> inf,
// x < -88 -> 0. Built only from IEEE mul/add/fma/floor, so host and device
// give bit-identical results (requires -ffp-contract=off).
__host__ __device__ inline float mlx_exp(float x_init) {
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
  float ic = ipart > 200.0f ? 200.0f : (ipart < -200.0f ? -200.0f : ipart);
  uint32_t eb = (uint32_t)((int32_t)ic + 127) << 23;
  float r = u2f(eb) * p;
  if (x_init > 88.0f) r = __builtin_inff();
  if (x_init < -88.0f) r = 0.0f;
  if (x_init != x_init) r = x_init;
  return r;
}

// MLX CPU Sigmoid: y = 1/(1+exp(|x|)); x < 0 -> y, else 1 - y. The division is
// IEEE (correctly rounded) on both host and device.
__host__ __device__ inline float mlx_sigmoid(float x) {
  float y = 1.0f / (1.0f + mlx_exp(fabsf(x)));
  return x < 0.0f ? y : 1.0f - y;
}

// Sum over aligned groups of W lanes (W a power of two <= 64); every lane of
// the group receives the same bit pattern.
template <int W>
__device__ inline float group_sum(float v) {
#pragma unroll
  for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, W);
  return v;
}

// Value of `v` from the partner lane selected by a DPP control (row-local).
template <int CTRL>
__device__ inline double dpp_partner(double v) {
  const uint64_t b = __builtin_bit_cast(uint64_t, v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xF, 0xF, true);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, 0xF, 0xF, true);
  return __builtin_bit_cast(double, ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

// f64 sum over aligned groups of W lanes. Within a 16-lane row the partners
// come from DPP (quad_perm xor 1, xor 2, half-row mirror, row mirror: each an
// involution, so every lane adds the same pair and ends with the same bits);
// wider groups finish with cross-row shuffles.
template <int W>
__device__ inline double group_sum(double v) {
  if constexpr (W >= 2) v += dpp_partner<0xB1>(v);   // quad_perm [1,0,3,2]
  if constexpr (W >= 4) v += dpp_partner<0x4E>(v);   // quad_perm [2,3,0,1]
  if constexpr (W >= 8) v += dpp_partner<0x141>(v);  // row_half_mirror
  if constexpr (W >= 16) v += dpp_partner<0x140>(v); // row_mirror
  if constexpr (W >= 32) v += __shfl_xor(v, 16, W);
  if constexpr (W >= 64) v += __shfl_xor(v, 32, W);
  return v;
}

// RMS scale r = 1/sqrt(f32(sum) * inv_n + eps) from an f64 sum of squares.
// Squares of f32 values are exact in f64 and the f64 sum is rounded once, so
// the result does not depend on the reduction order (MLX's mean(square(x)) is
// sum * f32(1/n) in f32; both sqrt and division are correctly rounded here).
__device__ inline float rms_scale(double ss, float inv_n, float eps) {
  const float ms = (float)ss * inv_n;
  return 1.0f / sqrtf(ms + eps);
}

// cos(th) and sin(th) of an f32 angle, evaluated in f64 and rounded to f32
// (RoPE's tables). For |th| < 2^20: th - k pi/2 with k = rint(th 2/pi) and
// pi/2 split in three parts (33 + 33 + 53 bits, so k P1 and k P2 are exact
// for |k| < 2^20), then the Taylor series of sin to r^17 and cos to r^16 on
// |r| <= pi/4 (truncation below 2^-57 relative) by Horner in f64, and the
// quadrant k mod 4: about 35 f64 operations against ~150 for the library's
// sincos, whose general reduction covers any double. Within 3 f64 ulps of the
// true values (measured: 2.8 ulps over 2e8 angles, whose f32 roundings all
// equal those of the C library's sin/cos); larger angles and non-finite ones
// take the library's sincos.
// The library's sincos for the angles the fast path does not take, out of
// line: inlined, its general argument reduction would hold registers that the
// callers' common path then cannot use.
struct SinCos {
  double s, c;
};
__device__ __attribute__((noinline)) SinCos sincos_wide(double x) {
  SinCos r;
  sincos(x, &r.s, &r.c);
  return r;
}

__device__ inline void cos_sin_f32(float th, float& c, float& s) {
  double sd, cd;
  if (fabsf(th) < 0x1p20f) {
    const double x = (double)th;
    const double k = __builtin_rint(x * 0x1.45f306dc9c883p-1);  // 2/pi
    double r = __builtin_fma(-k, 0x1.921fb54400000p+0, x);
    r = __builtin_fma(-k, 0x1.0b4611a600000p-34, r);
    r = __builtin_fma(-k, 0x1.3198a2e037073p-69, r);
    const double r2 = r * r;
    // (-1)^n / (2n+1)! and (-1)^n / (2n)!, n = 8 .. 1
    double ps = 2.8114572543455206e-15, pc = 4.779477332387385e-14;
    ps = __builtin_fma(ps, r2, -7.647163731819816e-13);
    pc = __builtin_fma(pc, r2, -1.1470745597729725e-11);
    ps = __builtin_fma(ps, r2, 1.6059043836821613e-10);
    pc = __builtin_fma(pc, r2, 2.08767569878681e-09);
    ps = __builtin_fma(ps, r2, -2.505210838544172e-08);
    pc = __builtin_fma(pc, r2, -2.755731922398589e-07);
    ps = __builtin_fma(ps, r2, 2.7557319223985893e-06);
    pc = __builtin_fma(pc, r2, 2.48015873015873e-05);
    ps = __builtin_fma(ps, r2, -0.0001984126984126984);
    pc = __builtin_fma(pc, r2, -0.001388888888888889);
    ps = __builtin_fma(ps, r2, 0.008333333333333333);
    pc = __builtin_fma(pc, r2, 0.041666666666666664);
    ps = __builtin_fma(ps, r2, -0.16666666666666666);
    pc = __builtin_fma(pc, r2, -0.5);
    const double sv = __builtin_fma(r * r2, ps, r), cv = __builtin_fma(r2, pc, 1.0);
    const int q = (int)k & 3;
    const double a = (q & 1) ? cv : sv, b = (q & 1) ? sv : cv;  // sin, cos up to sign
    sd = (q & 2) ? -a : a;
    cd = ((q + 1) & 2) ? -b : b;
  } else {
    const SinCos w = sincos_wide((double)th);
    sd = w.s;
    cd = w.c;
  }
  c = (float)cd;
  s = (float)sd;
}

}  // namespace hgk
