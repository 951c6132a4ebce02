// dcr_radix.h -- wave-level scans and the histogram bin search shared by the
// top-k select kernels (select.hip) and the fused decode kernel (fused.hip).
#pragma once

#include "dcr_common.h"

namespace dcr {

// DPP controls (gfx9): row_shr:n = 0x110 + n, row_bcast:15 = 0x142,
// row_bcast:31 = 0x143.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, ROW_MASK, 0xF, false));
}

// Inclusive prefix sum within each row of 16 lanes.
__device__ __forceinline__ uint32_t row16_inclusive_scan(uint32_t v) {
    v += dpp_u32<0x111, 0xF>(v);
    v += dpp_u32<0x112, 0xF>(v);
    v += dpp_u32<0x114, 0xF>(v);
    v += dpp_u32<0x118, 0xF>(v);
    return v;
}

// Inclusive prefix sum over the 64 lanes.
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v) {
    v = row16_inclusive_scan(v);
    v += dpp_u32<0x142, 0xA>(v);
    v += dpp_u32<0x143, 0xC>(v);
    return v;
}

// One wave: given the 256 bins of a histogram (ascending key order) spread as
// c[i] = bin 255-4l-i on lane l, find the bin holding the need-th largest
// element.  Writes the bin and the count of elements in higher bins.
__device__ __forceinline__ void find_bin_regs(const uint32_t (&c)[4], uint32_t need,
                                              uint32_t* out_bin, uint32_t* out_above) {
    const int lane = lane_id();
    const uint32_t sum = c[0] + c[1] + c[2] + c[3];
    uint32_t above = wave_inclusive_scan(sum) - sum;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (above < need && above + c[i] >= need) {
            *out_bin = static_cast<uint32_t>(255 - 4 * lane - i);
            *out_above = above;
        }
        above += c[i];
    }
}

}  // namespace dcr
