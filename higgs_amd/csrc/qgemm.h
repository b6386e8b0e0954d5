// qgemm.h -- the MFMA quantized matmul (qgemm.hip) as used by the
// quantized_matmul entry point (qmm.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hgk {

struct QgemmArgs {
  const uint16_t* x;
  int64_t xs;         // x row stride (elements, a multiple of 8)
  const uint32_t* w;  // [N, K/8]
  const uint16_t* sc; // [N, K/64]
  const uint16_t* bi;
  int64_t M, N, K;
  uint16_t* y;
  int64_t ys;         // y row stride (elements)
};

// gather_qmm over many (token, expert) pairs, grouped by expert on the matrix
// cores: y[p, :] = x[row(p), :] . W[e_p]^T, row(p) = lhs[p] or p / xdiv.
struct GatherArgs {
  const uint16_t* x;
  int64_t xrows, xs, xdiv;
  const int32_t* lhs;
  const uint32_t* w;   // [E, N, K/8]
  const uint16_t* sc;  // [E, N, K/64]
  const uint16_t* bi;
  const void* experts;
  int experts_i32;
  int64_t E, N, K, pairs;
  uint16_t* y;
  int64_t ys;
  // the up projection of the fused gate + up + SwiGLU form (null otherwise)
  const uint32_t* w2;
  const uint16_t* sc2;
  const uint16_t* bi2;
};

// Pairs per expert (on average) from which the grouped kernel runs.
constexpr int64_t kGatherMinPairsPerExpert = 16;

// bf16, group 64, 4 bits, x 16-byte aligned rows, w 16-byte aligned, K % 64,
// the expert ids 16-byte aligned and a multiple of 4 (read 4 at a time: a
// partly out-of-range 16-byte buffer load is not relied on) and under 2 GiB.
bool gather_grouped_supported(int dtype, int sdt, int group_size, int bits, const void* x,
                              int64_t xs, const void* w, int64_t k, const void* experts,
                              int64_t pairs);
void gather_grouped_launch(const GatherArgs& a, hipStream_t s);
// swiglu(gate, up) of the grouped regime in one launch (w/sc/bi: gate, w2/sc2/
// bi2: up, same shapes); false where the fused kernel does not apply.
bool gather_swiglu_grouped_launch(const GatherArgs& a, hipStream_t s);

// Rows of x at or above which the MFMA kernel runs (below: one GEMV per row).
constexpr int64_t kQgemmMinRows = 16;

// bf16 activations and scales, group 64, 4 bits, x 16-byte aligned with a
// row stride that is a multiple of 8, w 8-byte aligned.
bool qgemm_supported(int dtype, int sdt, int group_size, int bits, const void* x, int64_t xs,
                     const void* w, int64_t k);
void qgemm_launch(const QgemmArgs& a, hipStream_t s);

}  // namespace hgk
