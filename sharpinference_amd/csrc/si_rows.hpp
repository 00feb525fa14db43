// One value of a matrix row in its GGUF block layout, decoded as the
// reference's row dequantisation does (one rounding per operation).
#pragma once

#include "si_internal.hpp"

#include <hip/hip_fp16.h>

namespace si {

__device__ __forceinline__ float row_half(const uint8_t* p)
{
    const unsigned short h = static_cast<unsigned short>(p[0] | (p[1] << 8));
    return __half2float(__ushort_as_half(h));
}

// Column c of the row at rp (byte loads: no alignment needs).
template <int FMT>
__device__ __forceinline__ float row_value(const uint8_t* rp, int c)
{
    constexpr int BE = block_elems(FMT), BB = block_bytes(FMT);
    const uint8_t* b = rp + (c / BE) * BB;
    const int e = c % BE;
    if constexpr (FMT == FMT_F16) {
        return row_half(b);
    } else if constexpr (FMT == FMT_F32) {
        return __uint_as_float(static_cast<uint32_t>(b[0]) | (static_cast<uint32_t>(b[1]) << 8) |
                               (static_cast<uint32_t>(b[2]) << 16) | (static_cast<uint32_t>(b[3]) << 24));
    } else if constexpr (FMT == FMT_Q8_0) {
        return __fmul_rn(row_half(b), static_cast<float>(static_cast<int8_t>(b[2 + e])));
    } else if constexpr (FMT == FMT_Q4_0) {
        const int q = e < 16 ? (b[2 + e] & 15) : (b[2 + e - 16] >> 4);
        return __fmul_rn(row_half(b), static_cast<float>(q - 8));
    } else {   // Q4_K: sub-block j's 6-bit scale and min (GGML get_scale_min_k4)
        const int j = e / 32, l = e % 32;
        const uint8_t* s = b + 4;
        int sc, m;
        if (j < 4) {
            sc = s[j] & 63;
            m = s[j + 4] & 63;
        } else {
            sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
            m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        }
        const float d1 = __fmul_rn(row_half(b), static_cast<float>(sc));
        const float m1 = __fmul_rn(row_half(b + 2), static_cast<float>(m));
        const int q = (b[16 + 32 * (j >> 1) + l] >> (4 * (j & 1))) & 15;
        return __fsub_rn(__fmul_rn(d1, static_cast<float>(q)), m1);
    }
}

}  // namespace si
