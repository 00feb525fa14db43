// Cross-lane sums and maxima shared by the attention kernels.
#pragma once

#include <hip/hip_runtime.h>

namespace si {

// The value that DPP control CTRL reads for this lane.  Every control used
// by these kernels (quad_perm, row_half_mirror, row_mirror) reads a lane of
// the reading lane's own 16-lane row, so no lane is out of range and
// bound_ctrl changes no result; it lets the compiler fold the move into the
// consumer as a DPP source operand (one v_add_f32_dpp / v_max_f32_dpp
// instead of a v_mov_b32_dpp and the operation).
template <int CTRL>
__device__ __forceinline__ int dpp_row(int v)
{
    static_assert(CTRL == 0xB1 || CTRL == 0x4E || CTRL == 0x141 || CTRL == 0x140,
                  "controls whose source lane is always inside the row");
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_row(float v)
{
    return __int_as_float(dpp_row<CTRL>(__float_as_int(v)));
}

// Sum over aligned groups of N (<= 16) lanes with DPP.
template <int N>
__device__ __forceinline__ float row_sum(float v)
{
    if constexpr (N >= 2) v += dpp_row<0xB1>(v);
    if constexpr (N >= 4) v += dpp_row<0x4E>(v);
    if constexpr (N >= 8) v += dpp_row<0x141>(v);
    if constexpr (N >= 16) v += dpp_row<0x140>(v);
    return v;
}

// Maximum over aligned groups of N (<= 16) lanes with DPP.
template <int N>
__device__ __forceinline__ float row_max(float v)
{
    if constexpr (N >= 2) v = fmaxf(v, dpp_row<0xB1>(v));
    if constexpr (N >= 4) v = fmaxf(v, dpp_row<0x4E>(v));
    if constexpr (N >= 8) v = fmaxf(v, dpp_row<0x141>(v));
    if constexpr (N >= 16) v = fmaxf(v, dpp_row<0x140>(v));
    return v;
}

// Swaps between the halves (32 lanes) and the row pairs (16 lanes) of a
// wave: after both steps every lane holds the combination of the four lanes
// l, l ^ 16, l ^ 32, l ^ 48 (its column of the wave's four rows).
__device__ __forceinline__ float rows_sum(float v)
{
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ float rows_max(float v)
{
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

}  // namespace si
