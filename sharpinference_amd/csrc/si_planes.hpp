// FP32 vectors as exact int8 digit planes for v_dot4_i32_i8 products,
// shared by the matrix-vector kernels and the RWKV-7 time-mix core.
//
// Each 32-value block is scaled by a power of two 2^s chosen from the
// block's largest magnitude M (2^20 <= M * 2^s < 2^21) and rounded to
// integers X (|X| <= 2^21; the rounding is at most half a unit,
// 2^-s / 2 <= 2^-21 M per value).  X + 0x808080 has bytes b0, b1, b2 in
// [0, 255]; the signed bytes d_p = b_p - 128 are its balanced base-256
// digits, X = d0 + 256 d1 + 65536 d2 (|d2| <= 32).  Plane p packs d_p of 4
// consecutive values into one word, so a weight word of 4 signed (or
// masked 4-bit) bytes is multiplied with 4 values in one v_dot4_i32_i8,
// exactly.  A block with a non-finite value or a magnitude outside
// [2^-100, 2^100] is marked `exact`: its products take the per-weight FP32
// form instead (the planes could not keep the IEEE class of the sum).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "si_lanes.hpp"

namespace si {

constexpr uint32_t PLANE_BIG_BITS = 0x71800000u;    // 2^100
constexpr uint32_t PLANE_TINY_BITS = 0x0D800000u;   // 2^-100

// Maximum and sum over aligned groups of 8 lanes (DPP: xor-1 and xor-2
// swaps inside quads, then the mirror of each 8-lane half row).
__device__ __forceinline__ uint32_t group8_max_u32(uint32_t v)
{
    v = max(v, static_cast<uint32_t>(dpp_row<0xB1>(static_cast<int>(v))));
    v = max(v, static_cast<uint32_t>(dpp_row<0x4E>(static_cast<int>(v))));
    return max(v, static_cast<uint32_t>(dpp_row<0x141>(static_cast<int>(v))));
}
__device__ __forceinline__ int group8_sum_i32(int v)
{
    v += dpp_row<0xB1>(v);
    v += dpp_row<0x4E>(v);
    return v + dpp_row<0x141>(v);
}

// The planes of 4 consecutive values of a block whose 32 values are held
// 4 per lane by an aligned group of 8 lanes (every lane of the group calls
// this together): plane words p[0..2], the block's 2^-s, sum(X) and
// whether the block takes the per-weight form.
struct PlaneWords {
    uint32_t p[3];
    float inv;
    int sum;
    bool exact;
};

__device__ __forceinline__ PlaneWords encode_planes(float4 v)
{
    PlaneWords r;
    // largest magnitude as bits (integer order = magnitude order; NaN
    // sorts above inf), over the block's 8 lanes
    uint32_t mb = max(max(__float_as_uint(v.x) & 0x7fffffffu, __float_as_uint(v.y) & 0x7fffffffu),
                      max(__float_as_uint(v.z) & 0x7fffffffu, __float_as_uint(v.w) & 0x7fffffffu));
    mb = group8_max_u32(mb);
    r.exact = mb > PLANE_BIG_BITS || (mb != 0u && mb < PLANE_TINY_BITS);
    const uint32_t e = max(mb >> 23, 27u);                  // biased exponent of M (zero blocks: 27)
    // M < 2^(e - 126), so s = 147 - e gives M 2^s < 2^21
    const float scale = __uint_as_float((274u - e) << 23);  // 2^s
    r.inv = __uint_as_float((e - 20u) << 23);                // 2^-s
    // X + 0x808080 from the FP32 bits of X + 1.5 * 2^23 (round to nearest even)
    const uint32_t y0 = __float_as_uint(fmaf(v.x, scale, 0x1.8p23f)) - 0x4ABF7F80u;
    const uint32_t y1 = __float_as_uint(fmaf(v.y, scale, 0x1.8p23f)) - 0x4ABF7F80u;
    const uint32_t y2 = __float_as_uint(fmaf(v.z, scale, 0x1.8p23f)) - 0x4ABF7F80u;
    const uint32_t y3 = __float_as_uint(fmaf(v.w, scale, 0x1.8p23f)) - 0x4ABF7F80u;
    // byte transpose: plane p = byte p of y0..y3, then b - 128 as a signed byte
    const uint32_t t01 = __builtin_amdgcn_perm(y1, y0, 0x06020400u);   // y0.b0 y1.b0 y0.b2 y1.b2
    const uint32_t t23 = __builtin_amdgcn_perm(y3, y2, 0x06020400u);
    const uint32_t u01 = __builtin_amdgcn_perm(y1, y0, 0x0c0c0501u);   // y0.b1 y1.b1
    const uint32_t u23 = __builtin_amdgcn_perm(y3, y2, 0x0c0c0501u);
    r.p[0] = __builtin_amdgcn_perm(t23, t01, 0x05040100u) ^ 0x80808080u;
    r.p[1] = __builtin_amdgcn_perm(u23, u01, 0x05040100u) ^ 0x80808080u;
    r.p[2] = __builtin_amdgcn_perm(t23, t01, 0x07060302u) ^ 0x80808080u;
    r.sum = group8_sum_i32(static_cast<int>((y0 + y1) + (y2 + y3)) - 4 * 0x808080);
    return r;
}

__device__ __forceinline__ int dot4_planes(uint32_t q, uint32_t p, int a)
{
    return __builtin_amdgcn_sdot4(static_cast<int>(q), static_cast<int>(p), a, false);
}

// sum(q X) of one Q8_0 block (8 words of 4 signed bytes, values 4k..4k+3
// in word k) against its planes P (plane p word k at 8p + k), in FP32.
// The three-plane Horner sum would leave INT32 (32 * 128 * 2^21 = 2^33),
// so the top plane is summed on its own (|sum q d2| <= 32 * 128 * 32 =
// 2^17) and the lower two in INT32 Horner (|256 sum q d1 + sum q d0| <
// 2^28); 65536 s2 is exact in FP32 and the sum is rounded once.
__device__ __forceinline__ float q8_planes_sum(const uint32_t (&q)[8], const uint32_t* P)
{
    int s2 = 0, s01 = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        s2 = dot4_planes(q[k], P[16 + k], s2);
        s01 = dot4_planes(q[k], P[8 + k], s01);
    }
    s01 <<= 8;
#pragma unroll
    for (int k = 0; k < 8; k++)
        s01 = dot4_planes(q[k], P[k], s01);
    return fmaf(static_cast<float>(s2), 65536.0f, static_cast<float>(s01));
}

// sum(q X) of one 4-bit block (low nibbles lo[k]: values 4k..4k+3, high
// nibbles hi[k]: values 16+4k.., each masked into the low bits of its byte)
// against its planes, in INT32 (Horner in 256: |sum q X| <= 32 * 15 *
// 2^21 < 2^31).
__device__ __forceinline__ int q4_planes_sum(const uint32_t (&lo)[4], const uint32_t (&hi)[4], const uint32_t* P)
{
    int s = 0;
#pragma unroll
    for (int p = 2; p >= 0; p--) {
        if (p < 2)
            s <<= 8;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            s = dot4_planes(lo[k], P[8 * p + k], s);
            s = dot4_planes(hi[k], P[8 * p + 4 + k], s);
        }
    }
    return s;
}

}  // namespace si
