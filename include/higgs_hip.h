/*
 * higgs_hip.h -- C ABI of the MI355X (gfx950) per-layer op library
 * (libhiggs_hip.so). This is the drop-in boundary for the ops that
 * panbanda/higgs' higgs-models crate calls through mlx-rs; each entry point
 * names the reference call it replaces.
 *
 * Conventions (all entry points):
 *  - Device pointers in, device pointers out; the caller owns every buffer and
 *    pre-sizes every output. Nothing here allocates device memory or retains a
 *    pointer after returning.
 *  - Sizes and strides are int64 counts of ELEMENTS. The last (innermost) axis
 *    is always unit-stride.
 *  - `stream` is a hipStream_t (NULL = the default stream). Work is enqueued
 *    on it; no entry point synchronises.
 *  - Return value: HGK_OK (0) or an error status; hgk_last_error() gives a
 *    thread-local message for the last failure on the calling thread. Invalid
 *    arguments never reach the GPU.
 *  - Floating-point results follow MLX's CPU-device composition of each op,
 *    including its intermediate roundings to the activation dtype.
 */
#ifndef HIGGS_HIP_H
#define HIGGS_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  HGK_F32 = 0,
  HGK_BF16 = 1,
  HGK_F16 = 2,
  HGK_U32 = 3,
  HGK_I32 = 4
} hgk_dtype;

typedef enum {
  HGK_OK = 0,
  HGK_ERR_ARG = 1,         /* null pointer, bad shape / stride / dtype */
  HGK_ERR_UNSUPPORTED = 2, /* valid request this build does not implement */
  HGK_ERR_HIP = 3          /* HIP launch / runtime error */
} hgk_status;

typedef enum { HGK_ACT_SILU = 0, HGK_ACT_GELU_TANH = 1 } hgk_act;

/* Empty calls: a call with no rows, tokens, ids or pairs (or, for the
 * gated-delta recurrence, no steps) is valid, enqueues nothing, and may pass
 * NULL for the data it would have read or written; the recurrence over zero
 * steps writes the input state (zeros without one) to state_out. Weights,
 * tables and other operands that do not scale with the call still have to be
 * given. */

#define HGK_ABI_VERSION 1

/* Error message of the last failed call on this thread ("" if none).
 * Mirrors the mlx_set_error_handler last-error convention at
 * crates/higgs-models/src/qwen3_next.rs:28-51. */
const char* hgk_last_error(void);

/* HGK_ABI_VERSION of the loaded library. */
int hgk_abi_version(void);

/* Blocks until the work queued on `stream` (NULL = null stream) has finished
 * and returns HGK_ERR_HIP with the runtime's message if that work failed.
 * It is the only entry point that waits on the device; every other call only
 * enqueues. Replaces the forced evaluation mlx_rs::transforms::eval at
 * crates/higgs-engine/src/simple.rs:399 (and constrained.rs:275). */
int hgk_sync(void* stream);

/*
 * RMSNorm over the last axis of x[rows, n]:
 *   y = w' * round_T(x * rsqrt(mean(x^2) + eps)),  T = promote(x, w')
 * Replaces mlx_rs::fast::rms_norm as called by nn::RmsNorm::forward
 * (crates/higgs-models/src/transformer.rs:407,415,525;
 *  qwen3_next.rs:1518,1540,1547; qwen3_moe.rs:385,389,509; gemma2.rs:491-503).
 * w may be NULL (no weight). w_plus_one != 0 applies Gemma's (1 + w) in f32,
 * exactly the weight that apply_rmsnorm_plus_one (gemma2.rs:799-826) bakes in
 * at load time; the computation type is then f32. y_dtype may differ from the
 * computation type (the result is rounded to it). Also serves the Qwen3
 * q_norm/k_norm (transformer.rs:264-269) when they are not fused with RoPE:
 * rows = tokens*heads, n = head_dim.
 */
int hgk_rms_norm(const void* x, int x_dtype, int64_t x_row_stride,
                 const void* w, int w_dtype, int w_plus_one, float eps,
                 void* y, int y_dtype, int64_t y_row_stride,
                 int64_t rows, int64_t n, void* stream);

/*
 * Residual add fused with the RMSNorm that follows it:
 *   h = round_T(x + r)              (MLX add, T = the activation dtype)
 *   y = w' * round(h * rsqrt(mean(h^2) + eps))   (as hgk_rms_norm)
 * writing both h (the new residual stream) and y. Replaces the block
 * boundary `let h = x.add(residual)?; post_attention_layernorm.forward(&h)`
 * (crates/higgs-models/src/transformer.rs:413-415; qwen3_next.rs:1539-1540)
 * and the next block's `input_layernorm.forward(x)` after `h.add(mlp_out)`
 * (transformer.rs:407, 417). x, r and h share `dtype`; w, w_plus_one, eps and
 * y_dtype mean what they mean for hgk_rms_norm. h may be NULL (y only), and
 * h may be x or r itself (an in-place residual update); y must not overlap
 * x, r or h.
 */
int hgk_add_rms_norm(int dtype, const void* x, int64_t x_row_stride,
                     const void* r, int64_t r_row_stride,
                     const void* w, int w_dtype, int w_plus_one, float eps,
                     void* h, int64_t h_row_stride,
                     void* y, int y_dtype, int64_t y_row_stride,
                     int64_t rows, int64_t n, void* stream);

/*
 * Host helper: the dims/2 inverse frequencies fast::rope uses,
 *   inv[i] = freqs ? 1/freqs[i] : exp(-i * log(base) / (dims/2)).
 * Mirrors the frequency derivation inside mlx_rs::fast::rope
 * (utils.rs:17-25; deepseek_v2.rs:222-225 for explicit freqs).
 */
int hgk_rope_inv_freq(float base, int dims, const float* freqs, float* inv_freq_out);

/*
 * Host helper: llama3 rope_scaling frequency table (mlx-lm Llama3RoPE), the
 * `rope_scaling` block that transformer.rs:91-92 parses. Pass the result as
 * `freqs` to hgk_rope / hgk_qk_norm_rope.
 */
int hgk_llama3_rope_freqs(float base, int dims, float factor, float low_freq_factor,
                          float high_freq_factor, float original_max_position,
                          float* freqs_out);

/*
 * RoPE (non-traditional / NeoX half split) over a heads tensor viewed as
 * [batch, seq_len, heads, head_dim]; element (b,l,h,d) is at
 * x + b*x_strides[0] + l*x_strides[1] + h*x_strides[2] + d, likewise y.
 * Position of (b,l) = (offsets ? offsets[b] : offset) + l, times `scale`.
 * Rotates dims [0, dims) (partial rotary when dims < head_dim); the rest is
 * copied unchanged. freqs: optional HOST array of dims/2 frequencies (else
 * `base`). offsets: optional DEVICE int32[batch] (per-sequence offsets).
 * Replaces mlx_rs::fast::rope via apply_rope (utils.rs:16-26) at
 * transformer.rs:277-287, gemma2.rs:246-256, qwen3_moe.rs:194-204,
 * qwen3_next.rs:754-756 and the per-request loop of forward_batched
 * (transformer.rs:747-802). Only traditional == 0 is implemented (the
 * setting every in-scope model uses). y may alias x when both have the same
 * strides.
 */
int hgk_rope(int dtype, const void* x, const int64_t x_strides[3],
             void* y, const int64_t y_strides[3],
             int64_t batch, int64_t seq_len, int64_t heads, int64_t head_dim,
             int dims, int traditional, float base, float scale, const float* freqs,
             int32_t offset, const int32_t* offsets, void* stream);

/*
 * Qwen3 per-head q/k RMSNorm fused with RoPE, for q and (optionally) k in one
 * launch: y = rope(rms_norm(x, norm_w, eps)) per head row; a NULL norm weight
 * skips the norm for that tensor. Layouts as in hgk_rope, so the [B,L,H,D]
 * projection output can be read and [B,H,L,D] written directly (the
 * transpose at transformer.rs:271-275 is folded in). norm weights have
 * norm_w_dtype == dtype. k may be NULL (k_heads == 0).
 * Replaces q_norm/k_norm + transpose + apply_rope at transformer.rs:264-287
 * (and 730-735 + 747-802 in forward_batched), qwen3_moe.rs:170-204 and
 * qwen3_next.rs:741-756 (strided q view, partial rotary).
 */
int hgk_qk_norm_rope(int dtype,
                     const void* q, const int64_t q_strides[3],
                     void* q_out, const int64_t q_out_strides[3],
                     int64_t q_heads, const void* q_norm_w,
                     const void* k, const int64_t k_strides[3],
                     void* k_out, const int64_t k_out_strides[3],
                     int64_t k_heads, const void* k_norm_w,
                     int norm_w_dtype, float eps,
                     int64_t batch, int64_t seq_len, int64_t head_dim,
                     int dims, float base, float scale, const float* freqs,
                     int32_t offset, const int32_t* offsets, void* stream);

/*
 * Gated linear unit over rows: out = act(gate) * up.
 *   HGK_ACT_SILU:      swiglu / nn::silu(gate) * up   (transformer.rs:349-353,
 *                      qwen3_next.rs:275-277 used at 809 and 886,
 *                      qwen3_moe.rs:338, phi3.rs:261-265)
 *   HGK_ACT_GELU_TANH: nn::gelu_approximate(gate) * up (gemma2.rs:422-427)
 * A fused gate_up projection [rows, 2n] is passed as gate = p, up = p + n,
 * both with row stride 2n.
 */
int hgk_glu(int act, int dtype, const void* gate, int64_t gate_row_stride,
            const void* up, int64_t up_row_stride,
            void* out, int out_dtype, int64_t out_row_stride,
            int64_t rows, int64_t n, void* stream);

/*
 * Qwen3-Next gated RMSNorm: out = z * sigmoid(z) * rms_norm(x, w, eps), i.e.
 * swiglu(z, norm(y)) at qwen3_next.rs:1204-1205 (norm built at 1062-1064).
 * rows = tokens*value_heads, n = head_v_dim. Row r of z starts at
 *   z + (r / z_group_rows) * z_group_stride + (r % z_group_rows) * z_row_stride
 * so z can be read in place from the in_proj_qkvz output, where each key
 * head's block holds v_per_k value-head rows of z (qwen3_next.rs:1214-1265:
 * z_group_rows = v_per_k, z_row_stride = head_v_dim, z_group_stride = the
 * per-key-head block width). z_group_rows <= 0 means one group (uniform
 * z_row_stride).
 */
int hgk_gated_rms_norm(int dtype, const void* x, int64_t x_row_stride,
                       const void* z, int64_t z_row_stride,
                       int64_t z_group_rows, int64_t z_group_stride,
                       const void* w, int w_dtype, float eps,
                       void* out, int out_dtype, int64_t out_row_stride,
                       int64_t rows, int64_t n, void* stream);

/*
 * Affine-quantized embedding gather + dequantize:
 *   out[t, k] = s * q + b,  q = nibble (k % 8) of w_q[id, k/8] (low first),
 *   s, b = scales/biases[id, k/group_size], id = ids[t];
 * then, if out_scale != 0, out *= round(out_scale) (Gemma's sqrt(hidden)
 * embedding scale, gemma2.rs:587-600). Output dtype = scales_dtype.
 * Replaces nn::QuantizedEmbedding::forward (transformer.rs:494, gemma2.rs:588)
 * and QEmbedding::forward = dequantize(...).take_axis(ids, 0)
 * (qwen3_next.rs:248-257, qwen3_moe.rs:402-416) without dequantizing the
 * table. ids are int32 (negative counts from the end) or uint32; an id outside
 * [0, vocab) yields a zero row. Implemented: bits == 4, group_size in
 * {32, 64, 128}.
 */
int hgk_quantized_embedding(const void* ids, int ids_dtype, int64_t n_ids,
                            const uint32_t* w_q, const void* scales,
                            const void* biases, int scales_dtype,
                            int64_t vocab, int64_t hidden, int group_size, int bits,
                            float out_scale, void* out, int64_t out_row_stride,
                            void* stream);

/*
 * The embedding gather fused with the first layer's input RMSNorm: writes
 * h = hgk_quantized_embedding(...) (the residual stream) and
 * y = rms_norm(h, norm_w, eps) in one pass over the gathered rows. Replaces
 * `let h = self.embed_tokens.forward(inputs)?` followed by the first block's
 * `self.input_layernorm.forward(x)?` (crates/higgs-models/src/transformer.rs:494,
 * 407; gemma2.rs:587-600 then 491 with the Gemma scale in out_scale and
 * w_plus_one = 1). The table arguments mean what they mean for
 * hgk_quantized_embedding; norm_w, w_plus_one, eps and y_dtype what they mean
 * for hgk_rms_norm (y_dtype: the scales dtype or f32). h may be NULL.
 * Invalid ids give zero rows in h and in y.
 */
int hgk_quantized_embedding_rms_norm(const void* ids, int ids_dtype, int64_t n_ids,
                                     const uint32_t* w_q, const void* scales,
                                     const void* biases, int scales_dtype,
                                     int64_t vocab, int64_t hidden, int group_size, int bits,
                                     float out_scale, void* h, int64_t h_row_stride,
                                     const void* norm_w, int norm_w_dtype, int w_plus_one,
                                     float eps, void* y, int y_dtype, int64_t y_row_stride,
                                     void* stream);

/*
 * gather_qmm for 4-bit affine weights in the MLX layout, transpose = true,
 * one activation row per (token, expert) pair -- the MoE expert projections
 * of SwitchMlpWeights::forward_gather (crates/higgs-models/src/qwen3_next.rs:
 * 844-904), which the reference runs through mlx_gather_qmm (294-363):
 *   y[p, n] = sum_k x[row(p), k] * (scales[e_p, n, k/g] * q[e_p, n, k] + biases[e_p, n, k/g])
 * x [x_rows, k] (row stride x_row_stride) in bf16/f16; w [n_experts, n, k/8]
 * u32 (8 codes per word, low nibble first); scales/biases
 * [n_experts, n, k/group_size] in x's dtype; e_p = rhs_indices[p] (int32 or
 * uint32, device); row(p) = lhs_indices[p] when lhs_indices (device int32) is
 * given, else p / x_row_div (forward_gather's broadcast of one token row over
 * its top_k experts: x_row_div = top_k for gate/up, 1 for down). y [pairs, n]
 * in x's dtype, f32 accumulation. Rows or experts out of range give zero
 * rows. With at least 16 pairs per expert on average (prefill; bf16, group
 * 64) the pairs are grouped by expert inside the kernel and run on the matrix
 * cores; otherwise one GEMV per pair.
 */
int hgk_gather_qmm(int dtype, const void* x, int64_t x_rows, int64_t x_row_stride,
                   int64_t x_row_div, const int32_t* lhs_indices, const uint32_t* w,
                   const void* scales, const void* biases, int scales_dtype, int64_t n_experts,
                   int64_t n, int64_t k, int group_size, int bits, const void* rhs_indices,
                   int rhs_dtype, int64_t pairs, void* y, int64_t y_row_stride, void* stream);

/*
 * The gate and up expert projections of SwitchMlpWeights::forward_gather and
 * the SwiGLU between them (crates/higgs-models/src/qwen3_next.rs:862-886:
 * gate_out = gather_qmm(x, gate...), up_out = gather_qmm(x, up...),
 * activated = swiglu(&gate_out, &up_out)) in one launch: for each pair p and
 * column n,
 *   g = bf16(gather_qmm(x, w_gate)[p, n]), u = bf16(gather_qmm(x, w_up)[p, n])
 *   y[p, n] = round(round(g * round(sigmoid(g))) * u)
 * bit-identical to the three calls (each projection rounded to bf16 as
 * gather_qmm writes it, then hgk_glu's SwiGLU). Operands as hgk_gather_qmm,
 * with two weight sets of the same shape [n_experts, n, k/8] and one expert
 * index per pair. Requires bf16 x and scales, k in {512, 1024, 2048, 4096}
 * and 16-byte aligned x and weights. Below 16 pairs per expert on average
 * (decode) it runs one GEMV per pair. At 16 or more (prefill) it runs the
 * expert-grouped matrix-core kernel's fused form, which further needs group
 * 64, expert ids 16-byte aligned and a pair count that is a multiple of 4.
 * Other calls return HGK_ERR_UNSUPPORTED and run as hgk_gather_qmm twice plus
 * hgk_glu.
 */
int hgk_gather_qmm_swiglu(int dtype, const void* x, int64_t x_rows, int64_t x_row_stride,
                          int64_t x_row_div, const int32_t* lhs_indices, const uint32_t* w_gate,
                          const void* scales_gate, const void* biases_gate, const uint32_t* w_up,
                          const void* scales_up, const void* biases_up, int scales_dtype,
                          int64_t n_experts, int64_t n, int64_t k, int group_size, int bits,
                          const void* rhs_indices, int rhs_dtype, int64_t pairs, void* y,
                          int64_t y_row_stride, void* stream);

/*
 * quantized_matmul(x, w, scales, biases, transpose = true, group_size, bits):
 * QLinear::forward (crates/higgs-models/src/qwen3_next.rs:174-221, via
 * quantized_forward 174-183). x [M, K] (row stride x_row_stride, unit column
 * stride) in `dtype`; w [N, K*bits/32] u32; scales/biases [N, K/group_size]
 * in scales_dtype; y [M, N] (row stride y_row_stride). bits = 4,
 * group_size 32, 64 or 128, bf16 or f16 with scales of the same dtype. With
 * bf16, group 64 and M >= 16 the matrix cores run it (exact products, f32
 * sums, one rounding); otherwise one GEMV per row.
 */
int hgk_quantized_matmul(int dtype, const void* x, int64_t m, int64_t x_row_stride,
                         const uint32_t* w, const void* scales, const void* biases,
                         int scales_dtype, int64_t n, int64_t k, int group_size, int bits,
                         void* y, int64_t y_row_stride, void* stream);

/*
 * The GatedDeltaNet recurrence of Qwen3-Next's linear-attention layers -- the
 * reference's own gated-delta kernel (crates/higgs-models/src/qwen3_next.rs:
 * 376-451, called at 1187-1201) -- with the constant-weight q/k RMSNorm that
 * precedes it (1172-1173) fused in when q_norm_w/k_norm_w are given:
 *   g = exp(-exp(a_log) * softplus(a_t + dt_bias)), beta = sigmoid(b_t)
 *   s = s * g; delta = (v_t - s . k_t) * beta; s = s + k_t * delta; y_t = s . q_t
 * q, k [B, T, Hk, Dk], v [B, T, Hv, Dv], a, b [B, T, Hv] and y [B, T, Hv, Dv]
 * contiguous in `dtype`; a_log, dt_bias [Hv] in param_dtype; state_in and
 * state_out [B, Hv, Dv, Dk] in `dtype` (state_in NULL: zeros; state_out may be
 * state_in). Value head hv reads key head hv / (Hv / Hk). The state is f32
 * inside a call and rounded to `dtype` at its end, as in the reference.
 * head_k_dim in {32, 64, 128, 256}; batch <= 65535 and v_heads <= 65535.
 * With q, k and the state 16-byte aligned a vectorised kernel runs (one
 * token per call, a few tokens, or 16-step chunks staged in LDS); otherwise a
 * per-row kernel of the same arithmetic.
 */
int hgk_gated_delta(int dtype, const void* q, const void* k, const void* v, const void* a_log,
                    const void* a, const void* dt_bias, const void* b, int param_dtype,
                    const void* state_in, const void* q_norm_w, const void* k_norm_w, float eps,
                    int64_t batch, int64_t seq_len, int64_t k_heads, int64_t head_k_dim,
                    int64_t v_heads, int64_t head_v_dim, void* y, void* state_out, void* stream);

/*
 * One decode token of the GatedDeltaNet layer from the recurrence through its
 * gated output norm (crates/higgs-models/src/qwen3_next.rs:1185-1205:
 * gated_delta_kernel_ffi, then normed = self.norm.forward(&y) and
 * gated_out = swiglu(&z, &normed)) in one launch:
 *   y   = hgk_gated_delta(...) for T = 1 (rounded to `dtype`)
 *   out = round(round(z * round(sigmoid(z))) * rms_norm(y, norm_w, norm_eps))
 * over each (b, v-head) row of Dv -- bit-identical to hgk_gated_delta then
 * hgk_gated_rms_norm. Operands as hgk_gated_delta with seq_len 1; y may be
 * NULL (not written). z's rows are addressed as in hgk_gated_rms_norm (row r
 * = b * v_heads + hv at (r / z_group_rows) * z_group_stride + (r %
 * z_group_rows) * z_row_stride, so z is read in place from in_proj_qkvz);
 * norm_w [Dv] in `dtype`; out [B, Hv, Dv] contiguous. head_v_dim a multiple
 * of 8 up to 128 (one block per value head), q, k, the state, z and norm_w
 * 16-byte aligned, z's strides whole 16-byte units, the state under 2 GiB;
 * otherwise HGK_ERR_UNSUPPORTED (run the two calls).
 */
int hgk_gated_delta_gated_norm(int dtype, const void* q, const void* k, const void* v,
                               const void* a_log, const void* a, const void* dt_bias,
                               const void* b, int param_dtype, const void* state_in,
                               const void* q_norm_w, const void* k_norm_w, float eps,
                               int64_t batch, int64_t k_heads, int64_t head_k_dim,
                               int64_t v_heads, int64_t head_v_dim, void* state_out, void* y,
                               const void* z, int64_t z_row_stride, int64_t z_group_rows,
                               int64_t z_group_stride, const void* norm_w, int norm_w_dtype,
                               float norm_eps, void* out, void* stream);

/* ------------------------------------------------------------------------
 * A decode step's per-layer op sequence in one launch.
 *
 * Replaces the chain of separate calls the layer loop makes for every
 * sequence of a continuous batch (crates/higgs-models/src/qwen3_next.rs:
 * 1508-1547, driven by crates/higgs-engine/src/batch_engine.rs:395-403):
 * input_layernorm (residual add + RMSNorm), the gated RMSNorm of a
 * linear-attention layer or the q/k RMSNorm + (partial) RoPE of a
 * full-attention layer, post_attention_layernorm (add + RMSNorm) and the
 * experts' SwiGLU, layer after layer. The ops between them (projections,
 * attention, the recurrence) are not in the list; their outputs are the ops'
 * inputs.
 *
 * One workgroup per token walks the ops in order; each op waits for the
 * previous op's stores to reach L2 before it loads. Every op is row-wise, so
 * token t reads only token t's rows. Results are the same bits as the
 * separate calls (hgk_rms_norm, hgk_add_rms_norm, hgk_gated_rms_norm,
 * hgk_qk_norm_rope with one position per token, hgk_glu).
 *
 * Operand addressing (elements): row r of token t of operand P lies at
 * P + t * P_tok + r * P_row; the innermost axis is unit-stride. Every
 * operand and weight is 16-byte aligned and every stride a multiple of 8
 * elements. Activations, weights and outputs share the list's dtype (bf16 or
 * f16).
 * ------------------------------------------------------------------------ */
typedef enum {
  HGK_OP_RMS_NORM = 0,       /* y = rms_norm(x, w, eps); w may be NULL */
  HGK_OP_ADD_RMS_NORM = 1,   /* h = x + r (written if h != NULL); y = rms_norm(h, w, eps) */
  HGK_OP_GATED_RMS_NORM = 2, /* y = silu(z) * rms_norm(x, w, eps), z = operand r, its row
                              * k at (k / z_group_rows) * z_group_stride + (k % z_group_rows)
                              * r_row from the token's base (as hgk_gated_rms_norm) */
  HGK_OP_QK_NORM_ROPE = 3,   /* q = operand x (rows = q heads), k = operand r (k_heads rows),
                              * outputs y (q) and h (k); optional norm weights w (q), w2 (k);
                              * rotation as hgk_qk_norm_rope at position offsets[t] (or offset)
                              * times scale; head_dim n a power of two in 32..512, dims a
                              * multiple of 16 */
  HGK_OP_GLU = 4             /* y = act(gate) * up, gate = operand x, up = operand r */
} hgk_op_kind;

#define HGK_OP_LIST_MAX 4096

typedef struct {
  int kind;     /* hgk_op_kind */
  int rows;     /* rows per token (the q heads for HGK_OP_QK_NORM_ROPE) */
  int n;        /* elements per row (head_dim for HGK_OP_QK_NORM_ROPE), a multiple of 8;
                 * norms: n <= 8192; GLU: rows * n <= 8192 */
  float eps;
  const void* x;
  int64_t x_tok, x_row;
  const void* r;
  int64_t r_tok, r_row;
  int64_t z_group_rows, z_group_stride; /* HGK_OP_GATED_RMS_NORM; z_group_rows <= 0: one group */
  const void* w;
  const void* w2;
  void* y;
  int64_t y_tok, y_row;
  void* h;
  int64_t h_tok, h_row;
  int act;                /* HGK_OP_GLU: hgk_act */
  int k_heads;            /* HGK_OP_QK_NORM_ROPE */
  int dims;               /* rotated dims */
  float base;             /* as hgk_rope_inv_freq: base, or freqs [dims/2] (host memory) */
  const float* freqs;
  float scale;
  const int32_t* offsets; /* device [tokens] or NULL (then `offset` for every token) */
  int32_t offset;
} hgk_op;

/* Bytes of device memory an op list of n_ops ops takes (-1 if n_ops is not in
 * 1..HGK_OP_LIST_MAX). */
int64_t hgk_op_list_bytes(int n_ops);
/* Checks the ops, computes each RoPE op's frequencies, and writes the list
 * into dev_list (caller-owned device memory of hgk_op_list_bytes(n_ops)
 * bytes, 16-byte aligned), copying on `stream`; the copy has completed when
 * the call returns. The list keeps the operand addresses, not their data. */
int hgk_op_list_upload(int dtype, const hgk_op* ops, int n_ops, void* dev_list,
                       int64_t dev_bytes, void* stream);
/* Runs the first n_ops ops of an uploaded list over `tokens` tokens in one
 * launch. dtype must be the one the list was uploaded with; a list that was
 * not written by hgk_op_list_upload for that dtype and at least n_ops ops is
 * not walked (the launch does nothing). */
int hgk_op_list_run(int dtype, const void* dev_list, int n_ops, int64_t tokens, void* stream);

/* ------------------------------------------------------------------------
 * Checkpoint files: the safetensors files MLX 4-bit checkpoints ship in
 * (u32-packed `.weight`, bf16/f16 `.scales`/`.biases`, bf16 norm weights).
 * Replaces Array::load_safetensors as used by load_quantized_safetensors_weights
 * (crates/higgs-models/src/lib.rs:600-632) and collect_safetensors_files
 * (lib.rs:682-705). Host-side only: nothing here launches a kernel.
 * ------------------------------------------------------------------------ */
typedef struct hgk_st_file hgk_st_file; /* an open, memory-mapped file */

/* Open and validate a safetensors file (header JSON, dtypes, shapes, and
 * data offsets that tile the byte buffer exactly). */
int hgk_st_open(const char* path, hgk_st_file** out);
void hgk_st_close(hgk_st_file* f);
/* Number of tensors in the file (-1 for a null file). */
int64_t hgk_st_count(const hgk_st_file* f);
/* Index of the tensor called `name`; HGK_ERR_ARG if there is none. */
int hgk_st_find(const hgk_st_file* f, const char* name, int64_t* index);
/* Tensor `index` in header order: name, the file's dtype string ("BF16",
 * "U32", ...), its hgk dtype code (-1 for a type the kernels do not take),
 * rank (<= 8), shape and byte size. The strings live as long as the file.
 * Any output pointer may be NULL. */
int hgk_st_tensor(const hgk_st_file* f, int64_t index, const char** name,
                  const char** dtype_name, int* dtype, int* ndim, int64_t shape[8],
                  int64_t* nbytes);
/* Copy tensor `index`'s bytes into host memory. */
int hgk_st_copy_to_host(const hgk_st_file* f, int64_t index, void* dst, int64_t dst_bytes);
/* Copy tensor `index`'s bytes to device memory on `stream`, through pinned
 * staging buffers; the copy has completed when the call returns. */
int hgk_st_upload(const hgk_st_file* f, int64_t index, void* dst, int64_t dst_bytes,
                  void* stream);
/* The checkpoint's files: the distinct shard files named by
 * model.safetensors.index.json (sorted), else model.safetensors, else
 * HGK_ERR_ARG with a "MissingWeight" message (lib.rs:682-705). Writes the
 * paths, each followed by a newline, NUL-terminated, into out (cap bytes);
 * the size needed is stored in *needed (out may be NULL to query it). */
int hgk_st_collect_files(const char* model_dir, char* out, int64_t cap, int64_t* needed);
/* The reference's remap_quantized_key (lib.rs:709-723): `x.weight` ->
 * `x.inner.weight`, and likewise `.scales`, `.biases`, `.bias`. Returns 0 and
 * writes the new key, or HGK_ERR_UNSUPPORTED (2) with an empty string when
 * the key has no quantized form. */
int hgk_remap_quantized_key(const char* key, char* out, int64_t cap);

/* ------------------------------------------------------------------------
 * Measurement references (no counterpart in the reference: the benchmark's
 * floors). They compute nothing; they time what a launch and a pure stream
 * of bytes cost on this part, so that an op kernel's duration can be set
 * beside them at its own grid and byte counts.
 * ------------------------------------------------------------------------ */
/* The grid of the last kernel the calling thread launched through this
 * library: workgroups (x*y*z) and threads per workgroup (0, 0 before any). */
int hgk_last_launch_grid(int64_t* blocks, int* threads_per_block);
/* An empty kernel over `blocks` workgroups of `threads_per_block` threads. */
int hgk_floor_empty(int64_t blocks, int threads_per_block, void* stream);
/* Reads read_bytes from src and writes write_bytes to dst (both multiples of
 * 16, 16-byte aligned buffers) in one pass: units_per_thread (1, 2, 4 or 8)
 * 16-byte units per thread, all loads before the stores, non-temporal
 * stores. The written bytes are a function of the read ones. */
int hgk_floor_stream(const void* src, int64_t read_bytes, void* dst, int64_t write_bytes,
                     int units_per_thread, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HIGGS_HIP_H */
