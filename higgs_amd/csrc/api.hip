// api.hip -- library-wide C-ABI pieces: thread-local last error, ABI
// version, and the host-side RoPE frequency helpers.
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "../../include/higgs_hip.h"
#include "hgk_common.h"
#include "hgk_host.h"

namespace hgk {

namespace {
thread_local char g_last_error[512] = {0};
thread_local int64_t g_last_blocks = 0;
thread_local int g_last_threads = 0;
}

void note_launch(dim3 grid, dim3 block) {
  g_last_blocks = (int64_t)grid.x * grid.y * grid.z;
  g_last_threads = (int)(block.x * block.y * block.z);
}

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

void clear_error() { g_last_error[0] = 0; }

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(HGK_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return HGK_OK;
}

int resident_waves() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];  // 0: not yet queried
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) dev = -1;
  if (dev >= 0) {
    const int v = cached[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev < 0 ? 0 : dev) !=
          hipSuccess || cus <= 0)
    cus = 256;
  const int v = cus * 4 * 8;
  if (dev >= 0) cached[dev].store(v, std::memory_order_relaxed);
  return v;
}

int lds_per_cu() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];  // 0: not yet queried
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) dev = -1;
  if (dev >= 0) {
    const int v = cached[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
  }
  int bytes = 0;
  if (hipDeviceGetAttribute(&bytes, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor,
                            dev < 0 ? 0 : dev) != hipSuccess || bytes <= 0)
    bytes = 160 * 1024;
  if (dev >= 0) cached[dev].store(bytes, std::memory_order_relaxed);
  return bytes;
}

}  // namespace hgk

using namespace hgk;

extern "C" const char* hgk_last_error(void) { return g_last_error; }

extern "C" int hgk_abi_version(void) { return HGK_ABI_VERSION; }

extern "C" int hgk_last_launch_grid(int64_t* blocks, int* threads_per_block) {
  clear_error();
  if (!blocks || !threads_per_block) return fail(HGK_ERR_ARG, "hgk_last_launch_grid: null output");
  *blocks = g_last_blocks;
  *threads_per_block = g_last_threads;
  return HGK_OK;
}

// The one blocking call of the library: waits for the work queued on
// `stream` (NULL = the device's null stream) and reports an asynchronous
// error raised by it. Stands where the engine forces evaluation with
// mlx_rs::transforms::eval (crates/higgs-engine/src/simple.rs:399).
extern "C" int hgk_sync(void* stream) {
  clear_error();
  hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(HGK_ERR_HIP, "hgk_sync: %s", hipGetErrorString(e));
  return HGK_OK;
}

// Frequencies as fast::rope derives them: explicit freqs -> 1/freqs (f32
// reciprocal); otherwise exp(arange(0, -half, -1) * f32(log(base) / half))
// with MLX's polynomial exp (mlx_exp), evaluated in f32 on the host so the
// device receives the exact table.
extern "C" int hgk_rope_inv_freq(float base, int dims, const float* freqs, float* inv_out) {
  clear_error();
  if (!inv_out) return fail(HGK_ERR_ARG, "hgk_rope_inv_freq: null output");
  if (dims <= 0 || (dims & 1)) return fail(HGK_ERR_ARG, "hgk_rope_inv_freq: dims=%d must be even and > 0", dims);
  const int half = dims / 2;
  if (freqs) {
    for (int i = 0; i < half; ++i) inv_out[i] = 1.0f / freqs[i];
    return HGK_OK;
  }
  if (!(base > 0.0f)) return fail(HGK_ERR_ARG, "hgk_rope_inv_freq: base must be > 0");
  const float c = logf(base) / (float)half;
  for (int i = 0; i < half; ++i) inv_out[i] = mlx_exp((float)(-i) * c);
  return HGK_OK;
}

// mlx-lm Llama3RoPE frequencies, evaluated in f32 (python scalars are weak
// and take the array's f32 type):
//   f = base ** (arange(0, dims, 2) / dims);  wl = 2*pi*f
//   f = where(wl > old/low, f*factor, f)
//   sm = (old/wl - low) / (high - low)
//   f = where(old/high < wl < old/low, f / ((1 - sm)/factor + sm), f)
extern "C" int hgk_llama3_rope_freqs(float base, int dims, float factor, float low, float high,
                                     float old_ctx, float* f) {
  clear_error();
  if (!f) return fail(HGK_ERR_ARG, "hgk_llama3_rope_freqs: null output");
  if (dims <= 0 || (dims & 1)) return fail(HGK_ERR_ARG, "hgk_llama3_rope_freqs: bad dims %d", dims);
  if (!(base > 0.0f) || !(factor > 0.0f) || !(high > low) || !(low > 0.0f) || !(old_ctx > 0.0f))
    return fail(HGK_ERR_ARG, "hgk_llama3_rope_freqs: invalid scaling parameters");
  const int half = dims / 2;
  const float low_wl = (float)((double)old_ctx / (double)low);
  const float high_wl = (float)((double)old_ctx / (double)high);
  const float two_pi = (float)6.283185307179586;
  const float band = (float)((double)high - (double)low);
  for (int i = 0; i < half; ++i) {
    const float e = (float)(2 * i) / (float)dims;
    float fr = powf(base, e);
    const float wl = two_pi * fr;
    if (wl > low_wl) fr = fr * factor;
    const bool medium = (wl > high_wl) && (wl < low_wl);
    const float sm = (old_ctx / wl - low) / band;
    const float smooth = fr / ((1.0f - sm) / factor + sm);
    f[i] = medium ? smooth : fr;
  }
  return HGK_OK;
}
