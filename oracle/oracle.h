/*
 * oracle.h -- CPU restatement of the arithmetic behind higgs-models' per-layer
 * ops. TEST INFRASTRUCTURE ONLY: the parity tests, the smoke check and the
 * CPU-baseline leg of the benchmark call it as the checker. Nothing in the
 * shipped library links or calls it.
 *
 * The reference (panbanda/higgs, Rust) implements none of these ops itself; each
 * is a call into mlx-rs 0.25.3 / mlx-sys 0.2.0 (git af21d79, Cargo.toml:82-83,
 * 142-144), i.e. MLX C++ of the 0.25 era, which is not vendored under the
 * reference tree. What follows restates MLX's *CPU-device* composition of each
 * op, including every intermediate rounding to the activation dtype:
 *
 *   or_rms_norm        fast::rms_norm fallback: astype(f32) -> square -> mean
 *                      (sum * f32(1/n)) -> + eps -> rsqrt -> multiply ->
 *                      astype(T_out) -> multiply(weight).  Called from
 *                      transformer.rs:407,415,525; qwen3_next.rs:1518,1540,1547;
 *                      gemma2.rs:491-503 (weights shifted by +1 at load time,
 *                      gemma2.rs:799-826, modelled by plus_one).
 *   or_norm_rope       nn::RmsNorm over head_dim (q_norm/k_norm,
 *                      transformer.rs:264-269) followed by fast::rope
 *                      (utils.rs:16-26; transformer.rs:747-802 per-request
 *                      offsets; qwen3_next.rs:754-756 partial rotary).
 *   or_add             MLX's add (the residual `x.add(r)`, transformer.rs:413,
 *                      417); with or_rms_norm it restates the fused residual
 *                      add + RMSNorm of the block boundary (transformer.rs:
 *                      413-415, 417 then 407).
 *   or_rope_inv_freq   the inverse frequencies fast::rope derives from `base`
 *                      (or 1/freqs when explicit frequencies are given,
 *                      deepseek_v2.rs:222-225).
 *   or_llama3_freqs    mlx-lm Llama3RoPE frequency table (the llama3
 *                      rope_scaling the reference parses at transformer.rs:91-92).
 *   or_glu             swiglu / nn::silu(gate)*up (qwen3_next.rs:275-277,
 *                      transformer.rs:349-353) and nn::gelu_approximate(gate)*up
 *                      (gemma2.rs:422-427).
 *   or_gated_rms_norm  swiglu(z, norm(y)) (qwen3_next.rs:1204-1205).
 *   or_qembed          ops::dequantize + take / nn::QuantizedEmbedding
 *                      (qwen3_next.rs:248-257; transformer.rs:494), with the
 *                      optional Gemma embedding scale (gemma2.rs:587-600).
 *
 * Points that only importing MLX could settle are chosen as written in
 * oracle.c and each is marked "unpinned" there.
 *
 * Dtype codes are shared with the product ABI (include/higgs_hip.h).
 */
#ifndef HIGGS_ORACLE_H
#define HIGGS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_F32 = 0, OR_BF16 = 1, OR_F16 = 2, OR_U32 = 3, OR_I32 = 4 };
enum { OR_ACT_SILU = 0, OR_ACT_GELU_TANH = 1 };

/* ---- scalar helpers (exported so tests can pin them directly) ---- */
uint16_t or_f32_to_bf16(float v);
float or_bf16_to_f32(uint16_t b);
uint16_t or_f32_to_f16(float v);
float or_f16_to_f32(uint16_t h);
float or_mlx_exp(float x);      /* MLX CPU exp (polynomial, see oracle.c) */
float or_mlx_sigmoid(float x);  /* MLX CPU Sigmoid in f32 */
int or_promote(int a, int b);   /* MLX float type promotion */

/* ---- deterministic inputs (splitmix64 -> uniform / Box-Muller) ---- */
void or_fill_normal(uint64_t key, float mean, float stdev, float* out, int64_t n);
void or_fill_uniform(uint64_t key, float lo, float hi, float* out, int64_t n);
void or_fill_u32(uint64_t key, uint32_t* out, int64_t n);
void or_fill_ids(uint64_t key, uint32_t v, uint32_t* out, int64_t n);
void or_fill_offsets(uint64_t key, int32_t lo, int32_t hi, int32_t* out, int64_t n);
/* f32 -> dtype (RNE) and dtype -> f32 */
void or_convert_from_f32(int dt, const float* in, void* out, int64_t n);
void or_convert_to_f32(int dt, const void* in, float* out, int64_t n);

/* ---- the ops ---- */
int or_rms_norm(const void* x, int x_dt, int64_t x_row_stride,
                const void* w, int w_dt, int plus_one, float eps,
                void* y, int y_dt, int64_t y_row_stride,
                int64_t rows, int64_t n);

/* MLX add on dt (f32 sum rounded once); out may alias a or b. */
int or_add(int dt, const void* a, int64_t a_rs, const void* b, int64_t b_rs,
           void* out, int64_t o_rs, int64_t rows, int64_t n);

void or_rope_inv_freq(float base, int dims, const float* freqs, float* inv_out);
void or_llama3_freqs(float base, int dims, float factor, float low_freq_factor,
                     float high_freq_factor, float original_max_pos,
                     float* freqs_out);

/* x[b,l,h,d] lives at x + b*xs[0] + l*xs[1] + h*xs[2] + d (elements); same
 * for y with ys. norm_w may be NULL (plain RoPE). offsets may be NULL
 * (then `offset` applies to every sequence). Output dtype is
 * promote(x_dt, w_dt) when norm_w is given, else x_dt. */
int or_norm_rope(int x_dt, const void* x, const int64_t xs[3],
                 void* y, const int64_t ys[3],
                 int64_t B, int64_t L, int64_t H, int64_t D,
                 const void* norm_w, int w_dt, float eps,
                 int dims, const float* inv_freq, float scale,
                 int32_t offset, const int32_t* offsets);

/* The same with a choice of cos/sin evaluation: OR_TRIG_LIBM is or_norm_rope
 * (libm's f32 cosf/sinf, as MLX's CPU rope), OR_TRIG_F64 takes the f32
 * rounding of the f64 cos/sin of the same f32 angle, the device kernels'
 * evaluation. */
enum { OR_TRIG_LIBM = 0, OR_TRIG_F64 = 1 };
int or_norm_rope_trig(int x_dt, const void* x, const int64_t xs[3],
                      void* y, const int64_t ys[3],
                      int64_t B, int64_t L, int64_t H, int64_t D,
                      const void* norm_w, int w_dt, float eps,
                      int dims, const float* inv_freq, float scale,
                      int32_t offset, const int32_t* offsets, int trig);

int or_glu(int act, int x_dt, const void* gate, int64_t g_row_stride,
           const void* up, int64_t u_row_stride,
           void* out, int out_dt, int64_t o_row_stride,
           int64_t rows, int64_t n);

int or_gated_rms_norm(int x_dt, const void* y, int64_t y_row_stride,
                      const void* z, int64_t z_row_stride,
                      const void* w, int w_dt, float eps,
                      void* out, int out_dt, int64_t o_row_stride,
                      int64_t rows, int64_t n);

int or_qembed(const void* ids, int id_dt, int64_t n_ids,
              const uint32_t* wq, const void* scales, const void* biases,
              int s_dt, int64_t vocab, int64_t hidden, int group, int bits,
              float out_scale, void* out);

/* gather_qmm, 4-bit affine, transpose = true, one x row per pair: the exact
 * (f64) contraction rounded once to dt. */
int or_gather_qmm(int dt, const void* x, int64_t x_rows, int64_t x_rs, int64_t x_div,
                  const int32_t* lhs, const uint32_t* w, const void* sc, const void* bi,
                  int s_dt, int64_t E, int64_t N, int64_t K, int group, const int32_t* experts,
                  int64_t pairs, void* y, int64_t y_rs);

/* GatedDeltaNet recurrence (qwen3_next.rs:376-451) in f64, with the optional
 * constant-weight q/k RMSNorm (1172-1173) in front. */
int or_gated_delta(int dt, const void* q, const void* k, const void* v, const void* a_log,
                   const void* a, const void* dt_bias, const void* b, int p_dt,
                   const void* state_in, const void* qw, const void* kw, float eps,
                   int64_t B, int64_t T, int64_t Hk, int64_t Dk, int64_t Hv, int64_t Dv,
                   void* y, void* state_out);

#ifdef __cplusplus
}
#endif
#endif
