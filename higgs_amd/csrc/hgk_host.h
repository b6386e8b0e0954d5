// hgk_host.h -- host-side helpers shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hgk {

// Record a thread-local error message and return `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clear the thread-local error message (called on entry by every ABI call).
void clear_error();

// After a launch: HGK_OK, or HGK_ERR_HIP with the HIP error text.
int launch_status(const char* what);

// Waves the current device keeps resident at once when each uses at most 64
// VGPRs: compute units x 4 SIMDs x 8 waves (256 x 32 = 8192 on MI355X).
// Queried once per device; used to size persistent (grid-stride) launches.
int resident_waves();
// LDS bytes per CU of the current device (160 KB on gfx950).
int lds_per_cu();

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int dtype_bytes(int dt) { return (dt == 1 || dt == 2) ? 2 : 4; }

inline bool is_float_dtype(int dt) { return dt == 0 || dt == 1 || dt == 2; }

inline const char* dtype_name(int dt) {
  switch (dt) {
    case 0: return "f32";
    case 1: return "bf16";
    case 2: return "f16";
    case 3: return "u32";
    case 4: return "i32";
    default: return "?";
  }
}

// MLX promote_types restricted to the float dtypes.
inline int promote(int a, int b) { return a == b ? a : 0; }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Remember the grid of the launch about to be made by this thread
// (hgk_last_launch_grid reports it).
void note_launch(dim3 grid, dim3 block);

}  // namespace hgk

// Every kernel launch of the library goes through this: the launch, with its
// grid noted first.
#define HGK_LAUNCH(kernel, grid, block, shmem, stream, ...)                 \
  do {                                                                      \
    ::hgk::note_launch(dim3(grid), dim3(block));                            \
    hipLaunchKernelGGL(kernel, grid, block, shmem, stream, ##__VA_ARGS__);  \
  } while (0)

namespace hgk {

}  // namespace hgk
