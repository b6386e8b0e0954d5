// floor.hip -- measurement references for the op kernels (no arithmetic).
//
// Two kernels that time what a launch costs with no work in it, and what
// moving a given number of bytes costs with no arithmetic, on this part:
//  - an empty kernel with a caller-chosen grid (the launch, dispatch and
//    drain of that many workgroups);
//  - a streaming kernel that reads `read_bytes` and writes `write_bytes` with
//    the op kernels' own access pattern: 16-byte lane accesses, each wave
//    instruction covering 1 KB contiguous, every load of a thread issued
//    before its first store, non-temporal stores, one pass (no persistent
//    loop). The written values depend on the loaded ones, so no load can be
//    dropped.
// A kernel that runs within a few percent of the streaming kernel with its
// own read:write split is at the rate this part moves those bytes.
#include "../../include/higgs_hip.h"
#include "hgk_common.h"
#include "hgk_host.h"

namespace hgk {

__global__ void floor_empty_kernel() {}

// Thread i owns 16-byte units i + k * T (k < U, T = threads in the grid) of
// the read span and of the write span; units past a span's end are skipped.
// Written unit = the xor of the thread's loaded units, xored with the unit
// index (so every store depends on every load of its thread).
template <int U>
__global__ __launch_bounds__(256) void floor_stream_kernel(const u32x4* __restrict__ src,
                                                          int64_t nr, u32x4* __restrict__ dst,
                                                          int64_t nw) {
  const int64_t T = (int64_t)gridDim.x * blockDim.x;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  u32x4 v[U];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int64_t u = i + k * T;
    v[k] = u < nr ? __builtin_nontemporal_load(src + u) : u32x4{0u, 0u, 0u, 0u};
  }
  u32x4 acc = v[0];
#pragma unroll
  for (int k = 1; k < U; ++k) acc ^= v[k];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int64_t u = i + k * T;
    if (u < nw) {
      const uint32_t t = (uint32_t)u;
      __builtin_nontemporal_store(acc ^ u32x4{t, t, t, t}, dst + u);
    }
  }
}

}  // namespace hgk

using namespace hgk;

extern "C" int hgk_floor_empty(int64_t blocks, int threads_per_block, void* stream) {
  clear_error();
  if (blocks <= 0 || blocks > ((int64_t)1 << 31) - 1 || threads_per_block <= 0 ||
      threads_per_block > 1024)
    return fail(HGK_ERR_ARG, "hgk_floor_empty: blocks=%lld threads=%d out of range",
                (long long)blocks, threads_per_block);
  HGK_LAUNCH(floor_empty_kernel, dim3((unsigned)blocks), dim3(threads_per_block), 0,
             as_stream(stream));
  return launch_status("hgk_floor_empty");
}

extern "C" int hgk_floor_stream(const void* src, int64_t read_bytes, void* dst,
                                int64_t write_bytes, int units_per_thread, void* stream) {
  clear_error();
  const char* fn = "hgk_floor_stream";
  if (read_bytes < 0 || write_bytes < 0 || read_bytes % 16 || write_bytes % 16)
    return fail(HGK_ERR_ARG, "%s: byte counts must be >= 0 and multiples of 16", fn);
  if ((read_bytes && (!src || !aligned16(src))) || (write_bytes && (!dst || !aligned16(dst))))
    return fail(HGK_ERR_ARG, "%s: null or unaligned buffer", fn);
  if (units_per_thread != 1 && units_per_thread != 2 && units_per_thread != 4 &&
      units_per_thread != 8)
    return fail(HGK_ERR_ARG, "%s: units_per_thread must be 1, 2, 4 or 8", fn);
  const int64_t nr = read_bytes / 16, nw = write_bytes / 16;
  const int64_t units = nr > nw ? nr : nw;
  if (units == 0) return HGK_OK;
  const int64_t threads = (units + units_per_thread - 1) / units_per_thread;
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > ((int64_t)1 << 31) - 1) return fail(HGK_ERR_UNSUPPORTED, "%s: too large", fn);
  const dim3 g((unsigned)blocks), b(256);
  const hipStream_t s = as_stream(stream);
  const u32x4* in = static_cast<const u32x4*>(src);
  u32x4* out = static_cast<u32x4*>(dst);
  switch (units_per_thread) {
    case 1: HGK_LAUNCH((floor_stream_kernel<1>), g, b, 0, s, in, nr, out, nw); break;
    case 2: HGK_LAUNCH((floor_stream_kernel<2>), g, b, 0, s, in, nr, out, nw); break;
    case 4: HGK_LAUNCH((floor_stream_kernel<4>), g, b, 0, s, in, nr, out, nw); break;
    default: HGK_LAUNCH((floor_stream_kernel<8>), g, b, 0, s, in, nr, out, nw); break;
  }
  return launch_status(fn);
}
