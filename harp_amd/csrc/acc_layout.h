// Accumulator layout of v_mfma_f32_32x32x16_bf16, as a host-and-device
// function: accumulator register r of lane l holds row c_row(r, l / 32) and
// column l % 32 of the 32 x 32 C tile.  Included by the kernels
// (ra_common.h) and by host code that walks their addresses.
#pragma once

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define HARP_HD __host__ __device__ __forceinline__ constexpr
#else
#define HARP_HD inline constexpr
#endif

namespace harp_ra {

HARP_HD int c_row(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

}  // namespace harp_ra
