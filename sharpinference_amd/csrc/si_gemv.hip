// Matrix-vector product y = W . x for GGUF Q8_0 / Q4_0 / Q4_K weights kept
// in their native block layout and for dense F16 / F32 weights, plus the
// bit-exact decoder used to check those layouts.
//
// Semantics follow the core.mat-vec contract
// (SharpInference.Graphs/TierZeroOperationContracts.cs:113-115,152,161):
// W is [rows, cols] row-major (GGUF ne0 = cols contiguous), x is FP32 [cols],
// y is FP32 [rows], FP32 arithmetic and accumulation.  The reference's CPU
// form dequantises a row into FP32 and takes an FP32 dot
// (SharpInference.Backends.Cpu/CpuHalfMatrixOperators.cs:24-41); this kernel
// computes the same sum factored per block, d * sum(q * x), in FP32.
//
// Fast path layout (one "unit" = 64 columns of one row):
//   Q8_0  two 34-byte blocks, 68 bytes = 17 dwords, dword aligned
//   Q4_0  two 18-byte blocks, 36 bytes =  9 dwords, dword aligned
//   Q4_K  one 32-byte quant chunk of a 144-byte super-block plus the
//         super-block's 16-byte header (d, dmin, 12 scale bytes)
//   F16   128 bytes = 32 dwords;  F32  256 bytes = 64 dwords
// A wave holds 64 / LK row slots of LK lanes; lane k of a slot takes units
// k, k + LK, ... of RL consecutive rows, so every unit's x values are read
// from LDS once and reused for RL rows.  All weight loads of a lane are
// issued before x is staged into LDS, so HBM latency overlaps the staging.
#include "si_internal.hpp"
#include "si_lanes.hpp"
#include "si_planes.hpp"

#include <hip/hip_fp16.h>

#include <algorithm>

namespace si {
namespace {

constexpr int WG = 256;          // threads per workgroup (4 waves)
constexpr int XS_UNIT = 68;      // LDS floats per unit: 64 values + 4 pad (bank spread)

struct __attribute__((aligned(4))) u32x4 {
    uint32_t x, y, z, w;
};

__device__ __forceinline__ u32x4 ld4(const uint8_t* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ uint32_t ld1(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }

__device__ __forceinline__ float half_lo(uint32_t v)
{
    return __half2float(__ushort_as_half(static_cast<unsigned short>(v & 0xffffu)));
}
__device__ __forceinline__ float half_hi(uint32_t v)
{
    return __half2float(__ushort_as_half(static_cast<unsigned short>(v >> 16)));
}

// Sum of v over the wave, in every lane: DPP inside each 16-lane row, then
// swaps between the halves and between row pairs.
__device__ __forceinline__ float wave_sum(float v);

// 4 signed bytes of q times 4 floats, accumulated.
__device__ __forceinline__ float dot4_i8(uint32_t q, const float4& x, float a)
{
    a = fmaf(static_cast<float>(static_cast<int8_t>(q)), x.x, a);
    a = fmaf(static_cast<float>(static_cast<int8_t>(q >> 8)), x.y, a);
    a = fmaf(static_cast<float>(static_cast<int8_t>(q >> 16)), x.z, a);
    a = fmaf(static_cast<float>(static_cast<int8_t>(q >> 24)), x.w, a);
    return a;
}

// Hides the known-zero bits of a masked value from the optimiser, so the
// byte conversions below select one v_cvt_f32_ubyteN each instead of a
// bit-field extract plus a conversion.
__device__ __forceinline__ uint32_t opaque(uint32_t v)
{
    asm("" : "+v"(v));
    return v;
}

// Sum of v over aligned groups of N lanes (N = 2, 4, 8, 16), left in every
// lane of the group, with DPP lane moves (no LDS traffic):
// xor-1 and xor-2 swaps inside quads, then the mirror of each 8- and
// 16-lane row, which pairs every lane with one in the other half.
template <int N>
__device__ __forceinline__ float group_sum(float v)
{
    if constexpr (N >= 2)
        v += dpp_row<0xB1>(v);   // quad_perm 1,0,3,2
    if constexpr (N >= 4)
        v += dpp_row<0x4E>(v);   // quad_perm 2,3,0,1
    if constexpr (N >= 8)
        v += dpp_row<0x141>(v);  // row_half_mirror
    if constexpr (N >= 16)
        v += dpp_row<0x140>(v);  // row_mirror
    static_assert(N <= 16, "groups wider than a DPP row use shuffles");
    return v;
}

// ---- x as integer digit planes ----------------------------------------------
// The staged x of the 4-bit formats (and of Q8_0 at some shapes) is held as
// int8 digit planes (encode_planes: a power-of-two scale per 32-column
// block, x rounded to a 21-bit grid, at most 2^-21 M per value for a block
// of largest magnitude M).  The FP32 reference multiplies the FP32 x itself
// (CpuHalfMatrixOperators.cs:29-41); the products' error stays within the
// mat-vec tolerance but is not the reference's FP32 rounding.  Per block
// and row the planes' products combine in INT32 and the block enters the
// FP32 row sum once: d * 2^-s * sum((q - offset) * X).
//
// LDS per 64-column unit (PLANE_UNIT words): block h's planes at 24h +
// 8p + w (word w = values 4w..4w+3 of the block), then inv_0, inv_1
// (2^-s, or NaN when the block takes the per-weight FP32 form with x read
// from global memory), then aux_0, aux_1 (Q4_0: 8 sum(X) as INT32; Q4_K:
// sum(X) 2^-s as FP32; unused by Q8_0).  52 words: 16 lanes reading
// consecutive units with 16-byte reads touch distinct banks.
constexpr int PLANE_UNIT = 52;

__device__ __forceinline__ float wave_sum(float v)
{
    v = group_sum<16>(v);
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// 4 unsigned bytes (each < 256) of q times 4 floats, accumulated.
__device__ __forceinline__ float dot4_u8(uint32_t q, const float4& x, float a)
{
    a = fmaf(static_cast<float>(q & 0xffu), x.x, a);
    a = fmaf(static_cast<float>((q >> 8) & 0xffu), x.y, a);
    a = fmaf(static_cast<float>((q >> 16) & 0xffu), x.z, a);
    a = fmaf(static_cast<float>(q >> 24), x.w, a);
    return a;
}

template <int FMT>
struct QUnit;

// Two Q8_0 blocks {fp16 d; int8 q[32]} back to back.
template <>
struct QUnit<FMT_Q8_0> {
    static constexpr int UNIT_BYTES = 68;
    uint32_t v[17];
    __device__ __forceinline__ void prepare() {}

    __device__ __forceinline__ void load(const uint8_t* row, int u)
    {
        const uint8_t* p = row + u * UNIT_BYTES;
        const u32x4 a = ld4(p), b = ld4(p + 16), c = ld4(p + 32), d = ld4(p + 48);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        v[8] = c.x; v[9] = c.y; v[10] = c.z; v[11] = c.w;
        v[12] = d.x; v[13] = d.y; v[14] = d.z; v[15] = d.w;
        v[16] = ld1(p + 64);
    }

    // Contribution of block h (columns 32h..32h+31 of the unit).
    __device__ __forceinline__ float half(int h, const float4* x, float /*sx*/) const
    {
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k += 2) {
            const uint32_t q0 = h == 0 ? __builtin_amdgcn_alignbit(v[k + 1], v[k], 16) : v[9 + k];
            const uint32_t q1 = h == 0 ? __builtin_amdgcn_alignbit(v[k + 2], v[k + 1], 16) : v[10 + k];
            a0 = dot4_i8(q0, x[k], a0);
            a1 = dot4_i8(q1, x[k + 1], a1);
        }
        const float d = h == 0 ? half_lo(v[0]) : half_hi(v[8]);
        return d * (a0 + a1);
    }

    // Block h against x's digit planes P; inv = 2^-s.  sum(q X) scaled by
    // 2^-s (exact) and by the block scale, as the per-weight form
    // d * sum(q x) does.
    __device__ __forceinline__ float planes(int h, const uint32_t* P, float inv, float /*aux*/, float acc) const
    {
        uint32_t q[8];
#pragma unroll
        for (int k = 0; k < 8; k++)
            q[k] = h == 0 ? __builtin_amdgcn_alignbit(v[k + 1], v[k], 16) : v[9 + k];
        const float d = h == 0 ? half_lo(v[0]) : half_hi(v[8]);
        return fmaf(d, q8_planes_sum(q, P) * inv, acc);
    }

    // Non-finite or huge x: the per-weight FP32 form above.
    __device__ float half_exact(int h, const float4* x) const { return half(h, x, 0.0f); }
};

// Two Q4_0 blocks {fp16 d; u8 q[16]}: element j < 16 is the low nibble of
// q[j], element j + 16 the high nibble, value d * (nibble - 8).
// Fast form: the low nibbles are masked in place (q & 0x0f..) and the high
// ones too (q & 0xf0.., i.e. 16 * nibble), each byte converted by one
// v_cvt_f32_ubyteN; the factor 16 and the offset 8 are applied once per
// block: d * (a_lo + a_hi / 16 - 8 * sum(x)).
template <>
struct QUnit<FMT_Q4_0> {
    static constexpr int UNIT_BYTES = 36;
    uint32_t v[9];
    __device__ __forceinline__ void prepare() {}

    __device__ __forceinline__ void load(const uint8_t* row, int u)
    {
        const uint8_t* p = row + u * UNIT_BYTES;
        const u32x4 a = ld4(p), b = ld4(p + 16);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        v[8] = ld1(p + 32);
    }

    __device__ __forceinline__ uint32_t qword(int h, int k) const
    {
        return h == 0 ? __builtin_amdgcn_alignbit(v[k + 1], v[k], 16) : v[5 + k];
    }
    __device__ __forceinline__ float scale(int h) const { return h == 0 ? half_lo(v[0]) : half_hi(v[4]); }

    __device__ __forceinline__ float half(int h, const float4* x, float sx) const
    {
        float a_lo = 0.0f, a_hi = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t q = qword(h, k);
            a_lo = dot4_u8(opaque(q & 0x0f0f0f0fu), x[k], a_lo);
            a_hi = dot4_u8(opaque(q & 0xf0f0f0f0u), x[4 + k], a_hi);
        }
        return scale(h) * fmaf(-8.0f, sx, fmaf(a_hi, 0.0625f, a_lo));
    }

    // Block h against x's digit planes P (24 words, plane p word w at
    // 8p + w); inv = 2^-s, sum8 = 8 sum(X).  Low nibbles are values 4k..4k+3
    // (plane word k), high nibbles values 16+4k.. (word 4+k).
    __device__ __forceinline__ float planes(int h, const uint32_t* P, float inv, int sum8, float acc) const
    {
        constexpr uint32_t M = 0x0f0f0f0fu;
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            if (h == 0) {
                lo[k] = __builtin_amdgcn_alignbit(v[k + 1], v[k], 16) & M;
                hi[k] = __builtin_amdgcn_alignbit(v[k + 1], v[k], 20) & M;
            } else {
                lo[k] = v[5 + k] & M;
                hi[k] = (v[5 + k] >> 4) & M;
            }
        }
        return fmaf(scale(h) * inv, static_cast<float>(q4_planes_sum(lo, hi, P) - sum8), acc);
    }

    // Classification-exact form for non-finite or huge x: (nibble ^ 8) is
    // (nibble - 8) as a signed 4-bit number; moved to the top of a byte it
    // reads as the signed byte 16 * (nibble - 8), so every product carries
    // the sign and class of the dequantised weight (no sum(x) term).
    __device__ float half_exact(int h, const float4* x) const
    {
        float a = 0.0f;
        for (int k = 0; k < 4; k++) {
            const uint32_t t = qword(h, k) ^ 0x88888888u;
            a = dot4_i8((t << 4) & 0xf0f0f0f0u, x[k], a);
            a = dot4_i8(t & 0xf0f0f0f0u, x[4 + k], a);
        }
        return (scale(h) * 0.0625f) * a;
    }
};

// Q4_K super-block {fp16 d; fp16 dmin; u8 scales[12]; u8 q[128]}; unit u is
// chunk c = u % 4 (64 elements: low nibbles of q[32c..32c+31] are sub-block
// 2c, high nibbles sub-block 2c+1), value (d*sc)*q - (dmin*m).
template <>
struct QUnit<FMT_Q4_K> {
    static constexpr int UNIT_BYTES = 36;   // amortised: 144 bytes per 4 units
    uint32_t hd[4];
    uint32_t qs[8];
    int chunk;

    __device__ __forceinline__ void load(const uint8_t* row, int u)
    {
        chunk = u & 3;
        const uint8_t* p = row + (u >> 2) * 144;
        const u32x4 h = ld4(p), a = ld4(p + 16 + 32 * chunk), b = ld4(p + 32 + 32 * chunk);
        hd[0] = h.x; hd[1] = h.y; hd[2] = h.z; hd[3] = h.w;
        qs[0] = a.x; qs[1] = a.y; qs[2] = a.z; qs[3] = a.w;
        qs[4] = b.x; qs[5] = b.y; qs[6] = b.z; qs[7] = b.w;
    }

    // d * sc and dmin * m of the unit's sub-blocks 2c (low nibbles) and
    // 2c + 1 (high nibbles), c = chunk (GGML get_scale_min_k4).  Their scale
    // bytes are the pair jj, jj + 1 with jj = 2 (c % 2) of each scale word,
    // so both are extracted at once (byte lanes of a 16-bit field), with
    // selects so lanes of different chunks do not diverge:
    //   j < 4:  sc = scales[j] & 63, m = scales[j + 4] & 63
    //   j >= 4: sc = (scales[j + 4] & 15) | (scales[j - 4] >> 6) << 4,
    //           m = (scales[j + 4] >> 4) | (scales[j] >> 6) << 4
    float dsc[2], dmn[2];
    __device__ __forceinline__ void prepare()
    {
        const int sh = 16 * (chunk & 1);
        const uint32_t s0 = hd[1] >> sh, s1 = hd[2] >> sh, s2 = hd[3] >> sh;
        const bool low = chunk < 2;
        const uint32_t sc = low ? (s0 & 0x3f3fu) : ((s2 & 0x0f0fu) | ((s0 >> 2) & 0x3030u));
        const uint32_t m = low ? (s1 & 0x3f3fu) : (((s2 >> 4) & 0x0f0fu) | ((s1 >> 2) & 0x3030u));
        const float d = half_lo(hd[0]), dm = half_hi(hd[0]);
        dsc[0] = d * static_cast<float>(sc & 0xffu);
        dsc[1] = d * static_cast<float>((sc >> 8) & 0xffu);
        dmn[0] = dm * static_cast<float>(m & 0xffu);
        dmn[1] = dm * static_cast<float>((m >> 8) & 0xffu);
    }

    // The high nibbles are masked in place (16 * q per byte); 1/16 goes
    // into the sub-block scale, which stays exact (a power of two).
    __device__ __forceinline__ float half(int h, const float4* x, float sx) const
    {
        const uint32_t mask = h == 0 ? 0x0f0f0f0fu : 0xf0f0f0f0u;
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k += 2) {
            a0 = dot4_u8(opaque(qs[k] & mask), x[k], a0);
            a1 = dot4_u8(opaque(qs[k + 1] & mask), x[k + 1], a1);
        }
        const float d1 = dsc[h] * (h == 0 ? 1.0f : 0.0625f);
        return fmaf(d1, a0 + a1, -(dmn[h] * sx));
    }

    // Sub-block 2c + h against x's digit planes P (nibble word k holds
    // values 4k..4k+3, plane word k); inv = 2^-s, sxq = sum(X) 2^-s.
    __device__ __forceinline__ float planes(int h, const uint32_t* P, float inv, float sxq, float acc) const
    {
        constexpr uint32_t M = 0x0f0f0f0fu;
        uint32_t q[8];
#pragma unroll
        for (int k = 0; k < 8; k++)
            q[k] = (h == 0 ? qs[k] : qs[k] >> 4) & M;
        int s = 0;
#pragma unroll
        for (int p = 2; p >= 0; p--) {
            if (p < 2)
                s <<= 8;
#pragma unroll
            for (int k = 0; k < 8; k++)
                s = dot4_planes(q[k], P[8 * p + k], s);
        }
        return fmaf(dsc[h] * inv, static_cast<float>(s), fmaf(-dmn[h], sxq, acc));
    }

    // Same contribution with every weight decoded as the oracle does,
    // w = (d*sc)*q - (dmin*m) rounded per operation, then w*x accumulated.
    // Used when x holds non-finite or huge values, where the factored form
    // above could change the IEEE class of the result (inf - inf).
    __device__ float half_exact(int h, const float4* x) const
    {
        const float d1 = dsc[h], m1 = dmn[h];
        float a = 0.0f;
        for (int k = 0; k < 8; k++) {
            const uint32_t q = h == 0 ? (qs[k] & 0x0f0f0f0fu) : ((qs[k] >> 4) & 0x0f0f0f0fu);
            const float xs[4] = {x[k].x, x[k].y, x[k].z, x[k].w};
            for (int i = 0; i < 4; i++) {
                const float w = __fsub_rn(__fmul_rn(d1, static_cast<float>((q >> (8 * i)) & 0xffu)), m1);
                a = fmaf(w, xs[i], a);
            }
        }
        return a;
    }
};

// 64 F16 weights (128 bytes, 32 words): each weight converted exactly to
// FP32 and multiplied into the sum in one fused op (v_fma_mix_f32), the
// reference's ConvertToSingle + Dot (CpuHalfMatrixOperators.cs:29-41).
template <>
struct QUnit<FMT_F16> {
    static constexpr int UNIT_BYTES = 128;
    uint32_t v[32];
    __device__ __forceinline__ void prepare() {}

    __device__ __forceinline__ void load(const uint8_t* row, int u)
    {
        const uint8_t* p = row + u * UNIT_BYTES;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const u32x4 a = ld4(p + 16 * i);
            v[4 * i] = a.x; v[4 * i + 1] = a.y; v[4 * i + 2] = a.z; v[4 * i + 3] = a.w;
        }
    }

    __device__ __forceinline__ float half(int h, const float4* x, float /*sx*/) const
    {
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t w0 = v[16 * h + 2 * k], w1 = v[16 * h + 2 * k + 1];
            a0 = fmaf(half_lo(w0), x[k].x, a0);
            a1 = fmaf(half_hi(w0), x[k].y, a1);
            a0 = fmaf(half_lo(w1), x[k].z, a0);
            a1 = fmaf(half_hi(w1), x[k].w, a1);
        }
        return a0 + a1;
    }
};

// 64 F32 weights (256 bytes), one FMA each (CpuPrimitiveOperatorBackend.cs:222-227).
template <>
struct QUnit<FMT_F32> {
    static constexpr int UNIT_BYTES = 256;
    uint32_t v[64];
    __device__ __forceinline__ void prepare() {}

    __device__ __forceinline__ void load(const uint8_t* row, int u)
    {
        const uint8_t* p = row + u * UNIT_BYTES;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const u32x4 a = ld4(p + 16 * i);
            v[4 * i] = a.x; v[4 * i + 1] = a.y; v[4 * i + 2] = a.z; v[4 * i + 3] = a.w;
        }
    }

    __device__ __forceinline__ float half(int h, const float4* x, float /*sx*/) const
    {
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t* w = v + 32 * h + 4 * k;
            a0 = fmaf(__uint_as_float(w[0]), x[k].x, a0);
            a1 = fmaf(__uint_as_float(w[1]), x[k].y, a1);
            a0 = fmaf(__uint_as_float(w[2]), x[k].z, a0);
            a1 = fmaf(__uint_as_float(w[3]), x[k].w, a1);
        }
        return a0 + a1;
    }
};

// Tiled kernel.  A workgroup of NW waves covers a group of rows; its waves
// split the row's units into KS consecutive K slices (wave w takes slice
// w % KS of row group w / KS).  Inside a wave, RS = 64 / LK row slots of LK
// lanes; lane k of a slot takes units k, k + LK, ... (UPL of them) of its
// slice for RL consecutive rows.  Partial sums are reduced across the LK
// lanes with shuffles and across the KS slices through LDS in a fixed
// order, so results do not depend on timing.
// ---- launch descriptors -----------------------------------------------------

// Device copy of one GemvOp.  A launch carries up to MAX_SEGS of them by
// value.  The tiled kernel runs a 1D grid of exactly the ops' workgroups
// (op i from workgroup first[i]; a workgroup finds its op with a uniform
// scan of the kernel arguments); the short-row and any-shape kernels run a
// 2D grid, grid row i being op i (as wide as the largest op needs), whose
// workgroups past their op's rows leave before any load or barrier.
struct Seg {
    const uint8_t* w;
    const float* x;
    float* y;
    const float* residual;
    const float* nw;        // norm weight
    const float* nb;        // norm bias
    const float* mix;
    const float* prev;
    float* norm_out;
    const float* copy_src;
    float* copy_dst;
    int rows;               // output rows
    int in;                 // XformKind
    int out;                // OutKind
    int copy_n;
    int blocks;             // blocks per row (generic kernel)
    float eps;
};
constexpr int MAX_SEGS = 8;
// A launch of one op carries a one-entry table, so its kernel reads its
// descriptor at fixed kernel-argument offsets (no dependent lookup).
template <int NS>
struct Segs {
    Seg s[NS];
    int count;
    // tiled kernel, NS > 1: a 1D grid, op i owning workgroups first[i] ..
    // first[i + 1] - 1 (the short-row and any-shape kernels run one grid
    // row per op instead)
    int first[NS];
};

// Output function of one row (OUT_SWIGLU_ROWS is handled by the callers,
// which hold both halves); res is the row's residual, loaded at the start
// of the kernel when the op has one.
__device__ __forceinline__ float finish(const Seg& sg, float v, float res, bool has_res)
{
    switch (sg.out) {
    case OUT_RELU_SQUARE: {
        const float h = v > 0.0f ? v : (v != v ? v : 0.0f);   // max(v, 0) with NaN kept
        return h * h;
    }
    case OUT_TANH: return tanhf(v);
    case OUT_SIGMOID: return 1.0f / (1.0f + expf(-v));
    default: return has_res ? v + res : v;
    }
}

__device__ __forceinline__ float silu_mul(float g, float u)
{
    return g / (1.0f + expf(-g)) * u;
}

// The op's first workgroup copies copy_n floats (a state store that must
// happen after every reader of the destination has run).  The first
// SIDE_HELD * threads values are loaded at the start of the kernel, ahead
// of the weights, and stored at its end; the rest (if any) at the end.
constexpr int SIDE_HELD = 8;

// The whole copy in one pass (kernels whose weight stream is short).
__device__ __forceinline__ void side_copy(const Seg& sg, int b, int threads)
{
    if (sg.copy_n > 0 && b == 0)
        for (int i = threadIdx.x; i < sg.copy_n; i += threads)
            sg.copy_dst[i] = sg.copy_src[i];
}

__device__ __forceinline__ float4 f4_sub(float4 a, float m) { return make_float4(a.x - m, a.y - m, a.z - m, a.w - m); }

// FULL = false compiles the plain product (no input transform, plain
// output with an optional residual, no side copy): the hot decode GEMV keeps
// the registers and the instruction stream it had before the fused forms.
//
// A one-op launch (NS = 1) also receives the weight base, x, the residual,
// the norm weight, the row count, the output kind, the input transform and
// the side-copy length as leading scalar arguments.  Those are preloaded into SGPRs at wave
// launch, so the weight and x loads are issued without first waiting for
// the descriptor's kernel-argument fetch, which then completes under the
// weight stream.  A lane's loads complete in issue order, so everything
// the kernel needs before its products (x, the transform's vectors) and
// the residual of the rows a thread stores (which may alias y) are loaded
// before the weights: loaded after them, they would wait for the whole
// weight stream and the x staging and products could not overlap it.
//
// NV is the number of transform vectors the fused form loads per x value: 1
// (SwiGLU's up half or the RMSNorm weight; none needed loads x again) or 4
// (LayerNorm weight and bias, token-mix and previous-token vectors).
template <int FMT, int LK, int UPL, int RL, int KS, int NW, int NS, bool FULL, int NV = 1, int XM = 0>
__global__ __launch_bounds__(64 * NW) void gemv_fast_kernel(const uint8_t* __restrict__ w0,
                                                           const float* __restrict__ x0, const float* res0,
                                                           const float* __restrict__ nw0, int rows0, int out0,
                                                           int in0, int copy0, Segs<NS> segs)
{
    static_assert(NW % KS == 0, "waves must cover whole row groups");
    constexpr int THREADS = 64 * NW;
    constexpr int RS = 64 / LK;                   // row slots per wave
    constexpr int ROWS_PER_GROUP = RS * RL;
    constexpr int GROUPS = NW / KS;
    constexpr int ROWS_PER_WG = ROWS_PER_GROUP * GROUPS;
    constexpr int HALF = ROWS_PER_WG / 2;         // OUT_SWIGLU_ROWS: gate rows, then up rows
    static_assert(HALF % RL == 0, "a lane's rows stay in one half");
    constexpr int UPS = LK * UPL;                 // units per slice
    constexpr int UPR = UPS * KS;                 // units per row
    constexpr int K = UPR * 64;
    constexpr int64_t ROW_BYTES = static_cast<int64_t>(UPR) * QUnit<FMT>::UNIT_BYTES;
    static_assert(K % 32 == 0 && THREADS % 8 == 0, "x staging keeps 8-thread groups whole");

    constexpr bool PLANES = XM == 1;
    static_assert(!PLANES || FMT == FMT_Q4_0 || FMT == FMT_Q4_K || FMT == FMT_Q8_0, "digit planes serve the block formats");
    __shared__ float4 xs4[PLANES ? 1 : UPR * XS_UNIT / 4];
    __shared__ float bs[PLANES ? 1 : UPR * 2];
    __shared__ uint4 xp4[PLANES ? UPR * PLANE_UNIT / 4 : 1];
    __shared__ float part[ROWS_PER_WG * KS];
    __shared__ float red[NW], red2[NW];

    // the op of this workgroup (a uniform scan of the table's first
    // workgroups) and the workgroup's index within it
    int op = 0;
    if constexpr (NS > 1) {
#pragma unroll
        for (int k = 1; k < NS; k++)
            op = k < segs.count && static_cast<int>(blockIdx.x) >= segs.first[k] ? k : op;
    }
    const Seg& sg = segs.s[op];
    const int b = static_cast<int>(blockIdx.x) - (NS == 1 ? 0 : segs.first[op]);
    const int rows = NS == 1 ? rows0 : sg.rows;
    const uint8_t* wbase = NS == 1 ? w0 : sg.w;
    const bool swiglu = FULL && (NS == 1 ? out0 : sg.out) == OUT_SWIGLU_ROWS;
    const int in_kind = FULL ? (NS == 1 ? in0 : sg.in) : static_cast<int>(XF_PLAIN);
    const int rb = b * (swiglu ? HALF : ROWS_PER_WG);   // first output row of this workgroup

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: index math stays scalar
    const int slice = wave % KS;
    const int group = wave / KS;
    const int lk = lane % LK;
    const int lr = lane / LK;
    const int local_row0 = group * ROWS_PER_GROUP + lr * RL;
    const int unit0 = slice * UPS + lk;

    // 1. x first: it is small and mostly an L2 hit, and a lane's loads
    //    complete in issue order, so loading it ahead of the weights lets
    //    it be staged into LDS while the weights are still in flight
    //    x is staged in XPT rounds of THREADS float4 values; only the last
    //    round can be partial, and an aligned group of 8 threads (32
    //    columns) is either wholly inside x or wholly past its end
    constexpr int XPT = (K / 4 + THREADS - 1) / THREADS;
    //    (loads are unconditional, their index clamped into x, so that no
    //    value has to be merged before the weight loads are issued; the
    //    threads past the end zero their values when staging)
    auto xin = [](int j) { return (K / 4) % THREADS == 0 || j < XPT - 1 || threadIdx.x + j * THREADS < K / 4; };
    auto xidx = [](int j) { return min(static_cast<int>(threadIdx.x) + j * THREADS, K / 4 - 1); };
    const float4* x4 = reinterpret_cast<const float4*>(NS == 1 ? x0 : sg.x);
    float4 xr[XPT];
#pragma unroll
    for (int j = 0; j < XPT; j++)
        xr[j] = x4[xidx(j)];

    // the input transform's vectors (step 3): SwiGLU's up half, the norm
    // weight, LayerNorm's bias, mix and previous-token vectors
    //    (pointers chosen per launch; a vector the transform does not use
    //    reads x again)
    float4 ta[XPT], tb[XPT], tc[XPT], td[XPT];
    if constexpr (FULL) {
        const bool ln = in_kind == XF_LAYERNORM || in_kind == XF_LAYERNORM_MIX;
        const bool mix = in_kind == XF_LAYERNORM_MIX;
        const float* nw = NS == 1 ? nw0 : sg.nw;
        const float4* pa = reinterpret_cast<const float4*>(
            in_kind == XF_SWIGLU ? (NS == 1 ? x0 : sg.x) + K : (in_kind == XF_RMSNORM || ln) ? nw : (NS == 1 ? x0 : sg.x));
#pragma unroll
        for (int j = 0; j < XPT; j++)
            ta[j] = pa[xidx(j)];
        if constexpr (NV == 4) {
            const float4* pb = ln ? reinterpret_cast<const float4*>(sg.nb) : x4;
            const float4* pc = mix ? reinterpret_cast<const float4*>(sg.mix) : x4;
            const float4* pd = mix ? reinterpret_cast<const float4*>(sg.prev) : x4;
#pragma unroll
            for (int j = 0; j < XPT; j++) {
                tb[j] = pb[xidx(j)];
                tc[j] = pc[xidx(j)];
                td[j] = pd[xidx(j)];
            }
        }
    }

    // the side copy's values (stored after the products)
    float cpv[SIDE_HELD];
    const bool copying = FULL && b == 0 && (NS == 1 ? copy0 : sg.copy_n) > 0;
    if (copying) {
#pragma unroll
        for (int k = 0; k < SIDE_HELD; k++)
            cpv[k] = sg.copy_src[min(static_cast<int>(threadIdx.x) + k * THREADS, sg.copy_n - 1)];
    }

    // residual of the rows this thread stores (step 5 below)
    const float* resid = NS == 1 ? res0 : sg.residual;
    const bool has_res = resid != nullptr && !swiglu;
    constexpr bool LANE_STORES = KS == 1;     // else thread t stores row rb + t
    float rres[RL];
#pragma unroll
    for (int t = 0; t < RL; t++)
        rres[t] = 0.0f;
    if (has_res) {
        if (LANE_STORES) {
            if (lk == 0) {
#pragma unroll
                for (int t = 0; t < RL; t++) {
                    const int r = rb + local_row0 + t;
                    if (r < rows)
                        rres[t] = resid[r];
                }
            }
        } else if (threadIdx.x < ROWS_PER_WG && rb + static_cast<int>(threadIdx.x) < rows) {
            rres[0] = resid[rb + threadIdx.x];
        }
    }

    // 2. issue every weight load of this lane (rows past the end are
    //    clamped into the matrix; their results are dropped)
    QUnit<FMT> w[UPL][RL];
#pragma unroll
    for (int t = 0; t < RL; t++) {
        const int l = local_row0 + t;
        int r;
        if (swiglu) {
            const int o = min(rb + l % HALF, rows - 1);
            r = l < HALF ? o : o + rows;
        } else {
            r = min(rb + l, rows - 1);
        }
        const uint8_t* rp = wbase + static_cast<int64_t>(r) * ROW_BYTES;
#pragma unroll
        for (int i = 0; i < UPL; i++)
            w[i][t].load(rp, unit0 + i * LK);
    }
    // 3. stage x into LDS (padded per unit), with its transform
#pragma unroll
    for (int j = 0; j < XPT; j++)
        if (!xin(j))
            xr[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float ln_mean = 0.0f, ln_inv = 0.0f;   // LayerNorm statistics (the per-weight form recomputes x)
    if (in_kind == XF_SWIGLU) {
        // x = [gate | up]; reference order: gate / (1 + exp(-gate)) * up
#pragma unroll
        for (int j = 0; j < XPT; j++) {
            const float4 u = ta[j];
            xr[j].x = silu_mul(xr[j].x, u.x);
            xr[j].y = silu_mul(xr[j].y, u.y);
            xr[j].z = silu_mul(xr[j].z, u.z);
            xr[j].w = silu_mul(xr[j].w, u.w);
        }
    } else if (in_kind == XF_RMSNORM) {
        // scale = 1 / sqrt(sum(x^2) / K + eps) is common to every x_i * weight_i,
        // so x * weight is staged now and the scale multiplies each row's
        // sum at the end: sum_k W_k (x_k * scale * g_k) = scale * sum_k W_k (x_k * g_k),
        // equal up to FP32 rounding.  The per-wave sums of x^2 go through
        // LDS at the staging barrier below.
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < XPT; j++) {
            ss += (xr[j].x * xr[j].x + xr[j].y * xr[j].y) + (xr[j].z * xr[j].z + xr[j].w * xr[j].w);
            const float4 g = ta[j];
            xr[j].x = xr[j].x * g.x;
            xr[j].y = xr[j].y * g.y;
            xr[j].z = xr[j].z * g.z;
            xr[j].w = xr[j].w * g.w;
        }
        ss = wave_sum(ss);
        if ((threadIdx.x & 63) == 0)
            red[wave] = ss;
    } else if (NV == 4 && (in_kind == XF_LAYERNORM || in_kind == XF_LAYERNORM_MIX)) {
        // mean = sum(x) / K; c = x - mean; var = sum(c^2) / K;
        // ln = (c * (1 / sqrt(var + eps))) * weight + bias.
        // Each wave takes the two-pass mean and sum of squared deviations of
        // its own values (in registers, DPP / lane-swap sums); the waves'
        // (count, mean, M2) merge after one barrier (Chan et al.'s pairwise
        // update: M2 = sum M2_w + n_w (mean_w - mean)^2).
        auto wave_count = [](int w) {   // values of wave w (the last round may be partial)
            int n = 0;
#pragma unroll
            for (int j = 0; j < XPT; j++)
                n += 4 * max(0, min(64, K / 4 - (j * THREADS + 64 * w)));
            return n;
        };
        float s1 = 0.0f;
#pragma unroll
        for (int j = 0; j < XPT; j++)
            s1 += (xr[j].x + xr[j].y) + (xr[j].z + xr[j].w);
        const int nown = wave_count(wave);
        const float mw = nown > 0 ? wave_sum(s1) / static_cast<float>(nown) : 0.0f;
        float s2 = 0.0f;
#pragma unroll
        for (int j = 0; j < XPT; j++) {
            if (!xin(j))
                continue;
            const float4 c = f4_sub(xr[j], mw);
            s2 += (c.x * c.x + c.y * c.y) + (c.z * c.z + c.w * c.w);
        }
        s2 = wave_sum(s2);
        if ((threadIdx.x & 63) == 0) {
            red[wave] = mw;
            red2[wave] = s2;
        }
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++)
            tot += static_cast<float>(wave_count(w)) * red[w];
        const float mean = tot / static_cast<float>(K);
        float m2 = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float dm = red[w] - mean;
            m2 += red2[w] + static_cast<float>(wave_count(w)) * dm * dm;
        }
        const float var = m2 / static_cast<float>(K);
        const float inv = 1.0f / sqrtf(var + sg.eps);
        ln_mean = mean;
        ln_inv = inv;
#pragma unroll
        for (int j = 0; j < XPT; j++)
            if (xin(j))
                xr[j] = f4_sub(xr[j], mean);
        const bool store = sg.norm_out != nullptr && b == 0;
        const bool mixing = in_kind == XF_LAYERNORM_MIX;
#pragma unroll
        for (int j = 0; j < XPT; j++) {
            if (!xin(j))
                continue;
            const int i = threadIdx.x + j * THREADS;
            const float4 g = ta[j], bb = tb[j];
            float4 v;
            v.x = xr[j].x * inv * g.x + bb.x;
            v.y = xr[j].y * inv * g.y + bb.y;
            v.z = xr[j].z * inv * g.z + bb.z;
            v.w = xr[j].w * inv * g.w + bb.w;
            if (store)
                reinterpret_cast<float4*>(sg.norm_out)[i] = v;
            if (mixing) {
                const float4 m = tc[j], p = td[j];
                v.x = v.x + (p.x - v.x) * m.x;
                v.y = v.y + (p.y - v.y) * m.y;
                v.z = v.z + (p.z - v.z) * m.z;
                v.w = v.w + (p.w - v.w) * m.w;
            }
            xr[j] = v;
        }
    }
    if constexpr (PLANES) {
        // digit planes of each 32-column block (8 threads of 4 values)
        uint32_t* xp = reinterpret_cast<uint32_t*>(xp4);
#pragma unroll
        for (int j = 0; j < XPT; j++) {
            const int i = threadIdx.x + j * THREADS;
            const PlaneWords pl = encode_planes(xr[j]);   // the block's 8 threads together
            if (xin(j)) {
                const int col = 4 * i;
                const int h = (col >> 5) & 1;
                uint32_t* ub = xp + (col >> 6) * PLANE_UNIT;
                uint32_t* pw = ub + 24 * h + ((col >> 2) & 7);
                pw[0] = pl.p[0];
                pw[8] = pl.p[1];
                pw[16] = pl.p[2];
                if ((i & 7) == 0) {
                    ub[48 + h] = pl.exact ? 0x7fc00000u : __float_as_uint(pl.inv);
                    ub[50 + h] = FMT == FMT_Q4_0 ? static_cast<uint32_t>(8 * pl.sum)
                                                 : __float_as_uint(static_cast<float>(pl.sum) * pl.inv);
                }
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < XPT; j++) {
            const int col = 4 * (threadIdx.x + j * THREADS);
            if (xin(j))
                xs4[(col >> 6) * (XS_UNIT / 4) + ((col & 63) >> 2)] = xr[j];
        }
    }
    // The factored Q4 forms need sum(x) per 32 columns.  A block holding a
    // non-finite or huge (|x| > 2^100) value stores NaN instead (NaN fails
    // every comparison, so it counts as wide too): its products then take
    // the per-weight form, which keeps each product's IEEE class.
    constexpr bool SUMS = (FMT == FMT_Q4_0 || FMT == FMT_Q4_K) && !PLANES;
    if constexpr (SUMS) {
#pragma unroll
        for (int j = 0; j < XPT; j++) {
            const int i = threadIdx.x + j * THREADS;
            const bool wide = !(fabsf(xr[j].x) <= 0x1p100f && fabsf(xr[j].y) <= 0x1p100f &&
                                fabsf(xr[j].z) <= 0x1p100f && fabsf(xr[j].w) <= 0x1p100f);
            const float v = wide ? __builtin_nanf("") : (xr[j].x + xr[j].y) + (xr[j].z + xr[j].w);
            const float sum = group_sum<8>(v);
            if ((i & 7) == 0 && xin(j))
                bs[i >> 3] = sum;
        }
    }
    __syncthreads();

    // 4. per-unit dot products, x read once per unit and reused for RL rows
    // the RMSNorm scale, applied to each row's sum by the threads that
    // store rows (and computed only there)
    auto out_scale = [&]() {
        if (!FULL || in_kind != XF_RMSNORM)
            return 1.0f;
        float total = 0.0f;
#pragma unroll
        for (int i = 0; i < NW; i++)
            total += red[i];
        return 1.0f / sqrtf(total / static_cast<float>(K) + sg.eps);
    };
    // the staged values of float4 q recomputed from global memory (the
    // per-weight form of a block whose digit planes are not valid)
    auto xval4 = [&](int q) -> float4 {
        float4 v = x4[q];
        if constexpr (FULL) {
            const float* nw = NS == 1 ? nw0 : sg.nw;
            if (in_kind == XF_SWIGLU) {
                const float4 up = x4[K / 4 + q];
                v = make_float4(silu_mul(v.x, up.x), silu_mul(v.y, up.y), silu_mul(v.z, up.z), silu_mul(v.w, up.w));
            } else if (in_kind == XF_RMSNORM) {
                const float4 g = reinterpret_cast<const float4*>(nw)[q];
                v = make_float4(v.x * g.x, v.y * g.y, v.z * g.z, v.w * g.w);
            } else if (NV == 4 && (in_kind == XF_LAYERNORM || in_kind == XF_LAYERNORM_MIX)) {
                const float4 g = reinterpret_cast<const float4*>(nw)[q];
                const float4 bb = reinterpret_cast<const float4*>(sg.nb)[q];
                v = f4_sub(v, ln_mean);
                v = make_float4(v.x * ln_inv * g.x + bb.x, v.y * ln_inv * g.y + bb.y, v.z * ln_inv * g.z + bb.z,
                                v.w * ln_inv * g.w + bb.w);
                if (in_kind == XF_LAYERNORM_MIX) {
                    const float4 m = reinterpret_cast<const float4*>(sg.mix)[q];
                    const float4 pv = reinterpret_cast<const float4*>(sg.prev)[q];
                    v = make_float4(v.x + (pv.x - v.x) * m.x, v.y + (pv.y - v.y) * m.y, v.z + (pv.z - v.z) * m.z,
                                    v.w + (pv.w - v.w) * m.w);
                }
            }
        }
        return v;
    };
    float acc[RL];
#pragma unroll
    for (int t = 0; t < RL; t++)
        acc[t] = 0.0f;
#pragma unroll
    for (int i = 0; i < UPL; i++) {
        const int u = unit0 + i * LK;
#pragma unroll
        for (int t = 0; t < RL; t++)
            w[i][t].prepare();
        if constexpr (PLANES) {
            const uint4* ub = xp4 + u * (PLANE_UNIT / 4);
            const uint4 info = ub[12];   // inv_0, inv_1, aux_0, aux_1
#pragma unroll
            for (int h = 0; h < 2; h++) {
                uint32_t P[24];
#pragma unroll
                for (int k = 0; k < 6; k++) {
                    const uint4 q = ub[6 * h + k];
                    P[4 * k] = q.x; P[4 * k + 1] = q.y; P[4 * k + 2] = q.z; P[4 * k + 3] = q.w;
                }
                const float inv = __uint_as_float(h == 0 ? info.x : info.y);
                const uint32_t aux = h == 0 ? info.z : info.w;
                if (__builtin_expect(inv == inv, 1)) {
#pragma unroll
                    for (int t = 0; t < RL; t++) {
                        if constexpr (FMT == FMT_Q4_0)
                            acc[t] = w[i][t].planes(h, P, inv, static_cast<int>(aux), acc[t]);
                        else
                            acc[t] = w[i][t].planes(h, P, inv, __uint_as_float(aux), acc[t]);
                    }
                } else {
                    float4 xv[8];
                    for (int k = 0; k < 8; k++)
                        xv[k] = xval4(u * 16 + h * 8 + k);
                    for (int t = 0; t < RL; t++)
                        acc[t] += w[i][t].half_exact(h, xv);
                }
            }
            continue;
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
            float4 xv[8];
            const float4* src = xs4 + u * (XS_UNIT / 4) + h * 8;
#pragma unroll
            for (int k = 0; k < 8; k++)
                xv[k] = src[k];
            if constexpr (SUMS) {
                const float sx = bs[2 * u + h];
                if (__builtin_expect(sx == sx, 1)) {
#pragma unroll
                    for (int t = 0; t < RL; t++)
                        acc[t] += w[i][t].half(h, xv, sx);
                } else {
                    for (int t = 0; t < RL; t++)
                        acc[t] += w[i][t].half_exact(h, xv);
                }
            } else {
#pragma unroll
                for (int t = 0; t < RL; t++)
                    acc[t] += w[i][t].half(h, xv, 0.0f);
            }
        }
    }

    // 5. reduce across the LK lanes of a row slot, then across K slices
#pragma unroll
    for (int t = 0; t < RL; t++) {
        if constexpr (LK <= 16) {
            acc[t] = group_sum<LK>(acc[t]);
        } else {
#pragma unroll
            for (int off = LK / 2; off > 0; off >>= 1)
                acc[t] += __shfl_xor(acc[t], off);
        }
    }
    if (KS == 1 && !swiglu) {
        if (lk == 0) {
            const float sc = out_scale();
#pragma unroll
            for (int t = 0; t < RL; t++) {
                const int r = rb + local_row0 + t;
                if (r < rows)
                    sg.y[r] = FULL ? finish(sg, acc[t] * sc, rres[t], has_res) : (has_res ? acc[t] + rres[t] : acc[t]);
            }
        }
    } else {
        if (lk == 0) {
#pragma unroll
            for (int t = 0; t < RL; t++)
                part[(local_row0 + t) * KS + slice] = acc[t];
        }
        __syncthreads();
        const int t = threadIdx.x;
        if (t < (swiglu ? HALF : ROWS_PER_WG)) {
            const float sc = out_scale();
            float v = part[t * KS];
#pragma unroll
            for (int s2 = 1; s2 < KS; s2++)
                v += part[t * KS + s2];
            v *= sc;
            const int r = rb + t;
            if (swiglu) {
                float u = part[(t + HALF) * KS];
#pragma unroll
                for (int s2 = 1; s2 < KS; s2++)
                    u += part[(t + HALF) * KS + s2];
                u *= sc;
                if (r < rows)
                    sg.y[r] = silu_mul(v, u);
            } else if (r < rows) {
                sg.y[r] = FULL ? finish(sg, v, rres[0], has_res) : (has_res ? v + rres[0] : v);
            }
        }
    }
    if (copying) {
#pragma unroll
        for (int k = 0; k < SIDE_HELD; k++) {
            const int i = threadIdx.x + k * THREADS;
            if (i < sg.copy_n)
                sg.copy_dst[i] = cpv[k];
        }
        for (int i = threadIdx.x + SIDE_HELD * THREADS; i < sg.copy_n; i += THREADS)
            sg.copy_dst[i] = sg.copy_src[i];
    }
}

// ---- generic path: any whole number of blocks per row ------------------

__device__ __forceinline__ float ld_half(const uint8_t* p)
{
    const unsigned short h = static_cast<unsigned short>(p[0] | (p[1] << 8));
    return __half2float(__ushort_as_half(h));
}

template <int FMT>
__device__ float block_dot(const uint8_t* b, const float* x);

template <>
__device__ float block_dot<FMT_Q8_0>(const uint8_t* b, const float* x)
{
    float a = 0.0f;
    for (int i = 0; i < 32; i++)
        a = fmaf(static_cast<float>(static_cast<int8_t>(b[2 + i])), x[i], a);
    return ld_half(b) * a;
}

template <>
__device__ float block_dot<FMT_Q4_0>(const uint8_t* b, const float* x)
{
    float a = 0.0f;
    for (int i = 0; i < 16; i++) {
        a = fmaf(static_cast<float>((b[2 + i] & 15) - 8), x[i], a);
        a = fmaf(static_cast<float>((b[2 + i] >> 4) - 8), x[i + 16], a);
    }
    return ld_half(b) * a;
}

template <>
__device__ float block_dot<FMT_Q4_K>(const uint8_t* b, const float* x)
{
    const float d = ld_half(b), dmin = ld_half(b + 2);
    const uint8_t* s = b + 4;
    const uint8_t* q = b + 16;
    float a = 0.0f;
    for (int j = 0; j < 8; j++) {
        int sc, m;
        if (j < 4) {
            sc = s[j] & 63;
            m = s[j + 4] & 63;
        } else {
            sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
            m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        }
        const float d1 = __fmul_rn(d, static_cast<float>(sc));
        const float m1 = __fmul_rn(dmin, static_cast<float>(m));
        const uint8_t* qc = q + 32 * (j >> 1);
        const int shift = 4 * (j & 1);
        for (int l = 0; l < 32; l++) {
            const float w = __fsub_rn(__fmul_rn(d1, static_cast<float>((qc[l] >> shift) & 15)), m1);
            a = fmaf(w, x[32 * j + l], a);
        }
    }
    return a;
}

// One F16 / F32 weight from its bytes (byte loads: no alignment needs).
template <int FMT>
__device__ __forceinline__ float elem(const uint8_t* p)
{
    if constexpr (FMT == FMT_F16)
        return ld_half(p);
    return __uint_as_float(static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8) |
                           (static_cast<uint32_t>(p[2]) << 16) | (static_cast<uint32_t>(p[3]) << 24));
}

template <>
__device__ float block_dot<FMT_F16>(const uint8_t* b, const float* x)
{
    return elem<FMT_F16>(b) * x[0];
}

template <>
__device__ float block_dot<FMT_F32>(const uint8_t* b, const float* x)
{
    return elem<FMT_F32>(b) * x[0];
}

template <int FMT>
__device__ __forceinline__ float row_dot(const uint8_t* rp, const float* x, int blocks, int lane)
{
    float acc = 0.0f;
    if constexpr (block_elems(FMT) == 1) {   // F16 / F32: one fused multiply-add per weight
        for (int k = lane; k < blocks; k += 64)
            acc = fmaf(elem<FMT>(rp + static_cast<int64_t>(k) * block_bytes(FMT)), x[k], acc);
    } else {
        for (int k = lane; k < blocks; k += 64)
            acc += block_dot<FMT>(rp + static_cast<int64_t>(k) * block_bytes(FMT),
                                  x + static_cast<int64_t>(k) * block_elems(FMT));
    }
    for (int off = 32; off > 0; off >>= 1)
        acc += __shfl_xor(acc, off);
    return acc;
}

// One wave per output row, lanes stride over blocks, byte loads (no
// alignment needs); x is taken as is (no input transform).
template <int FMT, int NS>
__global__ __launch_bounds__(WG) void gemv_generic_kernel(Segs<NS> segs)
{
    const Seg& sg = segs.s[NS == 1 ? 0 : blockIdx.y];   // the op of this grid row
    const int b = static_cast<int>(blockIdx.x);
    side_copy(sg, b, WG);
    const int row = b * (WG / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= sg.rows)
        return;   // whole wave leaves together; no barrier follows
    const int64_t rbytes = static_cast<int64_t>(sg.blocks) * block_bytes(FMT);
    const float acc = row_dot<FMT>(sg.w + row * rbytes, sg.x, sg.blocks, lane);
    if (sg.out == OUT_SWIGLU_ROWS) {
        const float u = row_dot<FMT>(sg.w + (static_cast<int64_t>(row) + sg.rows) * rbytes, sg.x, sg.blocks, lane);
        if (lane == 0)
            sg.y[row] = silu_mul(acc, u);
    } else if (lane == 0) {
        sg.y[row] = finish(sg, acc, sg.residual ? sg.residual[row] : 0.0f, sg.residual != nullptr);
    }
}

// Short rows (at most SHORT_MAX_BLOCKS blocks and SHORT_MAX_COLS columns,
// e.g. the K = 64..256 LoRA outputs of RWKV-7): one lane per block, a wave
// holds 64 / blocks rows, x is staged once per workgroup, and the blocks of
// a row are summed in order by the row's first lane.
constexpr int SHORT_MAX_BLOCKS = 32;
constexpr int SHORT_MAX_COLS = 2048;

template <int FMT, int NS>
__global__ __launch_bounds__(WG) void gemv_short_kernel(Segs<NS> segs)
{
    __shared__ float xs[SHORT_MAX_COLS];
    __shared__ float part[2][WG];
    const Seg& sg = segs.s[NS == 1 ? 0 : blockIdx.y];   // the op of this grid row
    const int b = static_cast<int>(blockIdx.x);
    const int nb = sg.blocks;
    const int rpw = 64 / nb;                       // row slots per wave
    if (NS > 1 && b * (WG / 64) * rpw >= sg.rows)
        return;                                    // past this op's rows: the whole workgroup
    side_copy(sg, b, WG);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int slot = lane / nb, blk = lane - slot * nb;
    const int row = (b * (WG / 64) + wave) * rpw + slot;
    const int K = nb * block_elems(FMT);
    for (int i = threadIdx.x; i < K; i += WG)
        xs[i] = sg.x[i];
    __syncthreads();
    const bool swiglu = sg.out == OUT_SWIGLU_ROWS;
    const bool active = slot < rpw && row < sg.rows;
    float acc = 0.0f, accu = 0.0f;
    if (active) {
        const int64_t rb = static_cast<int64_t>(nb) * block_bytes(FMT);
        const int64_t off = static_cast<int64_t>(blk) * block_bytes(FMT);
        acc = block_dot<FMT>(sg.w + row * rb + off, xs + blk * block_elems(FMT));
        if (swiglu)
            accu = block_dot<FMT>(sg.w + (static_cast<int64_t>(row) + sg.rows) * rb + off, xs + blk * block_elems(FMT));
    }
    part[0][threadIdx.x] = acc;
    part[1][threadIdx.x] = accu;
    __syncthreads();
    if (active && blk == 0) {
        float v = 0.0f, u = 0.0f;
        for (int k = 0; k < nb; k++) {
            v += part[0][threadIdx.x + k];
            u += part[1][threadIdx.x + k];
        }
        sg.y[row] = swiglu ? silu_mul(v, u) : finish(sg, v, sg.residual ? sg.residual[row] : 0.0f, sg.residual != nullptr);
    }
}

// ---- block decoder (bit-exact dequantisation) ----------------------------

template <int FMT>
__global__ __launch_bounds__(WG) void dequant_kernel(const uint8_t* __restrict__ W, float* __restrict__ out,
                                                       int64_t nblocks)
{
    const int64_t blk = static_cast<int64_t>(blockIdx.x) * WG + threadIdx.x;
    if (blk >= nblocks)
        return;
    const uint8_t* b = W + blk * block_bytes(FMT);
    float* o = out + blk * block_elems(FMT);
    if constexpr (FMT == FMT_F16 || FMT == FMT_F32) {
        o[0] = elem<FMT>(b);
    } else if constexpr (FMT == FMT_Q8_0) {
        const float d = ld_half(b);
        for (int i = 0; i < 32; i++)
            o[i] = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(b[2 + i])));
    } else if constexpr (FMT == FMT_Q4_0) {
        const float d = ld_half(b);
        for (int i = 0; i < 16; i++) {
            o[i] = __fmul_rn(d, static_cast<float>((b[2 + i] & 15) - 8));
            o[i + 16] = __fmul_rn(d, static_cast<float>((b[2 + i] >> 4) - 8));
        }
    } else {
        const float d = ld_half(b), dmin = ld_half(b + 2);
        const uint8_t* s = b + 4;
        const uint8_t* q = b + 16;
        for (int j = 0; j < 8; j++) {
            int sc, m;
            if (j < 4) {
                sc = s[j] & 63;
                m = s[j + 4] & 63;
            } else {
                sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
                m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
            }
            const float d1 = __fmul_rn(d, static_cast<float>(sc));
            const float m1 = __fmul_rn(dmin, static_cast<float>(m));
            const uint8_t* qc = q + 32 * (j >> 1);
            const int shift = 4 * (j & 1);
            for (int l = 0; l < 32; l++)
                o[32 * j + l] = __fsub_rn(__fmul_rn(d1, static_cast<float>((qc[l] >> shift) & 15)), m1);
        }
    }
}

__global__ void fill_u32_kernel(uint32_t* __restrict__ dst, uint32_t value, uint64_t count)
{
    const uint64_t i = static_cast<uint64_t>(blockIdx.x) * WG + threadIdx.x;
    if (i < count)
        dst[i] = value;
}

// Partial sums (mod 2^32) of the 32-bit words of src: workgroup b of the
// grid (at most CHECKSUM_PARTS) writes parts[b]; the first workgroup also
// zeroes parts[grid..CHECKSUM_PARTS).  A plain streaming read, no atomics:
// each pass issues every 16-byte load of a thread (LOADS of them, a
// workgroup's 4 KB apart) before the first is used, so a pass costs one
// memory round trip; LOADS is the smallest of 2, 4, 8, 16 that covers the
// buffer in one pass of CHECKSUM_PARTS workgroups.
constexpr int CHECKSUM_PARTS = 1024;

template <int CHECKSUM_LOADS>
__global__ __launch_bounds__(WG) void checksum_kernel(const uint32_t* __restrict__ src, uint64_t words,
                                                     uint32_t* __restrict__ parts)
{
    __shared__ uint32_t red[WG / 64];
    const uint4* v = reinterpret_cast<const uint4*>(src);
    const uint64_t n16 = words / 4;
    const uint64_t span = static_cast<uint64_t>(WG) * CHECKSUM_LOADS;
    uint32_t sum = 0;
    for (uint64_t base = static_cast<uint64_t>(blockIdx.x) * span + threadIdx.x; base < n16;
         base += static_cast<uint64_t>(gridDim.x) * span) {
        uint4 a[CHECKSUM_LOADS];
#pragma unroll
        for (int k = 0; k < CHECKSUM_LOADS; k++) {
            const uint64_t i = base + static_cast<uint64_t>(k) * WG;
            a[k] = i < n16 ? v[i] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int k = 0; k < CHECKSUM_LOADS; k++)
            sum += (a[k].x + a[k].y) + (a[k].z + a[k].w);
    }
    if (blockIdx.x == 0 && threadIdx.x < words % 4)
        sum += src[n16 * 4 + threadIdx.x];
    for (int off = 32; off > 0; off >>= 1)
        sum += __shfl_xor(sum, off);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = sum;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = 0;
        for (int w = 0; w < WG / 64; w++)
            t += red[w];
        parts[blockIdx.x] = t;
    }
    if (blockIdx.x == 0)
        for (int j = static_cast<int>(gridDim.x) + threadIdx.x; j < CHECKSUM_PARTS; j += WG)
            parts[j] = 0;
}

// ---- dispatch --------------------------------------------------------------

Seg to_seg(const GemvOp& op)
{
    Seg g{};
    g.w = static_cast<const uint8_t*>(op.w);
    g.x = op.x;
    g.y = op.y;
    g.residual = op.residual;
    g.nw = op.norm_weight;
    g.nb = op.norm_bias;
    g.mix = op.mix;
    g.prev = op.prev;
    g.norm_out = op.norm_out;
    g.copy_src = op.copy_src;
    g.copy_dst = op.copy_dst;
    g.copy_n = static_cast<int>(op.copy_n);
    g.rows = static_cast<int>(op.rows);
    g.in = op.in;
    g.out = op.out;
    g.blocks = static_cast<int>(op.cols / block_elems(op.fmt));
    g.eps = op.eps;
    return g;
}

bool is_plain(const GemvOp& op)
{
    return op.in == XF_PLAIN && op.out == OUT_PLAIN && op.copy_n == 0;
}

// Builds the descriptor table of n ops and returns the 2D launch grid: op
// i takes ceil(rows / per_wg(op)) workgroups; a table of several ops runs
// one grid row per op, as wide as the largest op needs.
template <int NS, typename PerWg>
dim3 fill_segs(Segs<NS>& t, const GemvOp* ops, int n, PerWg per_wg)
{
    t = Segs<NS>{};
    t.count = n;
    unsigned width = 1;
    for (int i = 0; i < n; i++) {
        t.s[i] = to_seg(ops[i]);
        const int per = per_wg(ops[i]);
        width = std::max(width, static_cast<unsigned>((ops[i].rows + per - 1) / per));
    }
    return dim3(width, static_cast<unsigned>(n));
}

template <int FMT, int LK, int UPL, int RL, int KS, int NW, int XM = 0>
hipError_t launch_tiled(const GemvOp* ops, int n, hipStream_t s)
{
    constexpr int R = (64 / LK) * RL * (NW / KS);
    // an OUT_SWIGLU_ROWS op puts half as many output rows in a workgroup
    // (its gate and up rows share the tile)
    auto per = [](const GemvOp& op) { return op.out == OUT_SWIGLU_ROWS ? R / 2 : R; };
    const uint8_t* w0 = static_cast<const uint8_t*>(ops[0].w);
    const int rows0 = static_cast<int>(ops[0].rows);
    // a LayerNorm input transform loads four vectors per x value
    bool ln = false;
    for (int i = 0; i < n; i++)
        ln |= ops[i].in == XF_LAYERNORM || ops[i].in == XF_LAYERNORM_MIX;
    const GemvOp& o = ops[0];
    if (n == 1) {
        Segs<1> t;
        const dim3 grid = fill_segs(t, ops, n, per);
        if (is_plain(o))
            hipLaunchKernelGGL((gemv_fast_kernel<FMT, LK, UPL, RL, KS, NW, 1, false, 1, XM>), grid, dim3(64 * NW), 0,
                               s, w0, o.x, o.residual, o.norm_weight, rows0, o.out, o.in, static_cast<int>(o.copy_n), t);
        else if (ln)
            hipLaunchKernelGGL((gemv_fast_kernel<FMT, LK, UPL, RL, KS, NW, 1, true, 4, XM>), grid, dim3(64 * NW), 0,
                               s, w0, o.x, o.residual, o.norm_weight, rows0, o.out, o.in, static_cast<int>(o.copy_n), t);
        else
            hipLaunchKernelGGL((gemv_fast_kernel<FMT, LK, UPL, RL, KS, NW, 1, true, 1, XM>), grid, dim3(64 * NW), 0,
                               s, w0, o.x, o.residual, o.norm_weight, rows0, o.out, o.in, static_cast<int>(o.copy_n), t);
    } else {
        Segs<MAX_SEGS> t;
        fill_segs(t, ops, n, per);
        unsigned total = 0;   // 1D grid: op i's workgroups follow op i - 1's
        for (int i = 0; i < n; i++) {
            t.first[i] = static_cast<int>(total);
            total += static_cast<unsigned>((ops[i].rows + per(ops[i]) - 1) / per(ops[i]));
        }
        const dim3 grid(total);
        if (ln)
            hipLaunchKernelGGL((gemv_fast_kernel<FMT, LK, UPL, RL, KS, NW, MAX_SEGS, true, 4, XM>), grid, dim3(64 * NW),
                               0, s, w0, o.x, o.residual, o.norm_weight, rows0, o.out, o.in, static_cast<int>(o.copy_n), t);
        else
            hipLaunchKernelGGL((gemv_fast_kernel<FMT, LK, UPL, RL, KS, NW, MAX_SEGS, true, 1, XM>), grid, dim3(64 * NW),
                               0, s, w0, o.x, o.residual, o.norm_weight, rows0, o.out, o.in, static_cast<int>(o.copy_n), t);
    }
    return hipGetLastError();
}

// Shape table of the tiled kernel, from measurements on MI355X (rotating
// weight copies larger than the Infinity Cache).  Matrices with few rows
// are latency bound: the K slices spread each row over KS waves so every
// lane handles one 64-column unit and the grid covers all CUs.  Tall
// matrices are throughput bound: one wave per row group (KS = 1) with
// several units and rows per lane amortises the x staging and the
// reductions over more weights.  `rows64` counts the weight rows of every
// op of the launch.
template <int FMT>
hipError_t launch_fast(const GemvOp* ops, int n, int64_t rows64, int64_t cols, hipStream_t s)
{
    const bool mid = rows64 >= 12288, tall = rows64 >= 49152;
    switch (cols) {
    case 1024: return mid ? launch_tiled<FMT, 16, 1, 2, 1, 4>(ops, n, s) : launch_tiled<FMT, 16, 1, 1, 1, 4>(ops, n, s);
    case 2048:
        if constexpr (FMT == FMT_Q8_0) {
            // x as digit planes (v_dot4_i32_i8 on the signed weight bytes),
            // 32 rows per workgroup from 4096 rows: the RWKV-7 shapes with
            // weights streamed from HBM, against FP32 staging with the tiles
            // of the other formats: time-mix batch of 6656 rows 7.42 -> 6.07
            // us, FFN key 8192 rows 6.32 -> 5.90, 65536-row head 27.2 ->
            // 26.3, output 2048 rows 2.66 -> 2.62
            return rows64 >= 4096 ? launch_tiled<FMT, 16, 1, 2, 2, 8, 1>(ops, n, s)
                                  : launch_tiled<FMT, 16, 1, 1, 2, 4, 1>(ops, n, s);
        }
        return mid              ? launch_tiled<FMT, 16, 2, 2, 1, 4>(ops, n, s)
               : rows64 >= 8192 ? launch_tiled<FMT, 16, 2, 1, 1, 4>(ops, n, s)
               : rows64 >= 4096 ? launch_tiled<FMT, 16, 1, 1, 2, 8>(ops, n, s)
                                : launch_tiled<FMT, 16, 1, 1, 2, 4>(ops, n, s);
    case 3072:
        if constexpr (FMT == FMT_Q8_0)   // the 200064-row head: 104.0 -> 101.5 us with planes, 4 rows per lane group
            if (tall)
                return launch_tiled<FMT, 16, 3, 1, 1, 4, 1>(ops, n, s);
        if (tall)
            return launch_tiled<FMT, 16, 3, 2, 1, 4>(ops, n, s);
        if constexpr (FMT == FMT_Q8_0)
            return mid ? launch_tiled<FMT, 16, 3, 1, 1, 4>(ops, n, s) : launch_tiled<FMT, 16, 1, 1, 3, 3>(ops, n, s);
        else if (mid)   // Q4_K: the Phi-4-mini gate / up rows (RMSNorm and SwiGLU fused), weights from HBM:
                        // 8 waves 8.26 -> 7.85 us (Q4_0 plain: 4 waves 6.95, 8 waves 7.03)
            return FMT == FMT_Q4_K ? launch_tiled<FMT, 16, 3, 1, 1, 8, 1>(ops, n, s)
                                   : launch_tiled<FMT, 16, 3, 1, 1, 4, 1>(ops, n, s);
        else   // Q4 formats: wide workgroups (one per CU at 3072 and 5120 rows)
            // stage x once per CU instead of once per 4 rows, as digit planes
            // for the integer dot products
            return rows64 >= 5120   ? launch_tiled<FMT, 16, 1, 1, 3, 15, 1>(ops, n, s)
                   : rows64 >= 3072 ? launch_tiled<FMT, 16, 1, 1, 3, 12, 1>(ops, n, s)
                                    : launch_tiled<FMT, 16, 1, 1, 3, 3>(ops, n, s);
    case 4096: return mid ? launch_tiled<FMT, 16, 2, 2, 2, 4>(ops, n, s) : launch_tiled<FMT, 16, 1, 1, 4, 4>(ops, n, s);
    case 6144: return mid ? launch_tiled<FMT, 16, 3, 2, 2, 4>(ops, n, s) : launch_tiled<FMT, 16, 1, 1, 6, 6>(ops, n, s);
    case 8192:
        if (mid)
            return launch_tiled<FMT, 16, 4, 2, 2, 4>(ops, n, s);
        // 4 rows per workgroup: deriving digit planes of 8192 values would
        // cost more than the integer products save (weights from HBM, 3072
        // rows: Q4_K 5.53 us against 5.64 with planes and 12 rows per
        // workgroup; Q4_0 5.52 against 5.61; RWKV-7's Q8_0 2048 rows 5.46
        // against 5.50)
        return launch_tiled<FMT, 16, 1, 1, 8, 8>(ops, n, s);
    default: return hipErrorNotSupported;
    }
}

// Shape table of the F16 / F32 weights (2 and 4 bytes per weight: the
// streams are 2-4x a Q8_0 row's, so fewer units per lane keep the registers
// of a wave's loads in bounds: F16 units are 32 words, F32 units 64).
template <int FMT>
hipError_t launch_fast_dense(const GemvOp* ops, int n, int64_t rows64, int64_t cols, hipStream_t s)
{
    const bool mid = rows64 >= 12288;
    if constexpr (FMT == FMT_F32) {
        switch (cols) {
        case 1024: return launch_tiled<FMT, 16, 1, 1, 1, 4>(ops, n, s);
        case 2048: return launch_tiled<FMT, 16, 1, 1, 2, 4>(ops, n, s);
        case 3072: return launch_tiled<FMT, 16, 1, 1, 3, 3>(ops, n, s);
        case 4096: return launch_tiled<FMT, 16, 1, 1, 4, 4>(ops, n, s);
        case 6144: return launch_tiled<FMT, 16, 1, 1, 6, 6>(ops, n, s);
        case 8192: return launch_tiled<FMT, 16, 1, 1, 8, 8>(ops, n, s);
        default: return hipErrorNotSupported;
        }
    } else {
        switch (cols) {
        case 1024: return launch_tiled<FMT, 16, 1, 1, 1, 4>(ops, n, s);
        case 2048: return mid ? launch_tiled<FMT, 16, 2, 1, 1, 4>(ops, n, s) : launch_tiled<FMT, 16, 1, 1, 2, 4>(ops, n, s);
        // one unit per lane, the row's 48 units split over 3 waves; 12, 16
        // or 20 rows per workgroup (one workgroup per CU at 3072 and 5120
        // rows).  The Phi-4 F16 shapes against 4 rows per workgroup or 3
        // units per lane: qkv 8.68 -> 7.86, o 6.06 -> 5.58, gate/up with
        // SwiGLU rows 20.1 -> 18.8, tied head 211 -> 197 us
        case 3072: return mid              ? launch_tiled<FMT, 16, 1, 1, 3, 12>(ops, n, s)
                          : rows64 >= 5120 ? launch_tiled<FMT, 16, 1, 1, 3, 15>(ops, n, s)
                                           : launch_tiled<FMT, 16, 1, 1, 3, 9>(ops, n, s);
        case 4096: return mid ? launch_tiled<FMT, 16, 2, 1, 2, 4>(ops, n, s) : launch_tiled<FMT, 16, 1, 1, 4, 4>(ops, n, s);
        case 6144: return mid ? launch_tiled<FMT, 16, 3, 1, 2, 4>(ops, n, s) : launch_tiled<FMT, 16, 1, 1, 6, 6>(ops, n, s);
        case 8192: return mid ? launch_tiled<FMT, 16, 2, 1, 4, 4>(ops, n, s) : launch_tiled<FMT, 16, 1, 1, 8, 8>(ops, n, s);
        default: return hipErrorNotSupported;
        }
    }
}

template <int FMT>
hipError_t launch_generic(const GemvOp* ops, int n, hipStream_t s)
{
    auto per = [](const GemvOp&) { return WG / 64; };   // one output row per wave
    if (n == 1) {
        Segs<1> t;
        const dim3 grid = fill_segs(t, ops, n, per);
        hipLaunchKernelGGL((gemv_generic_kernel<FMT, 1>), grid, dim3(WG), 0, s, t);
    } else {
        Segs<MAX_SEGS> t;
        const dim3 grid = fill_segs(t, ops, n, per);
        hipLaunchKernelGGL((gemv_generic_kernel<FMT, MAX_SEGS>), grid, dim3(WG), 0, s, t);
    }
    return hipGetLastError();
}

template <int FMT>
hipError_t launch_short(const GemvOp* ops, int n, hipStream_t s)
{
    auto per = [](const GemvOp& op) { return (WG / 64) * (64 / static_cast<int>(op.cols / block_elems(FMT))); };
    if (n == 1) {
        Segs<1> t;
        const dim3 grid = fill_segs(t, ops, n, per);
        hipLaunchKernelGGL((gemv_short_kernel<FMT, 1>), grid, dim3(WG), 0, s, t);
    } else {
        Segs<MAX_SEGS> t;
        const dim3 grid = fill_segs(t, ops, n, per);
        hipLaunchKernelGGL((gemv_short_kernel<FMT, MAX_SEGS>), grid, dim3(WG), 0, s, t);
    }
    return hipGetLastError();
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The tiled kernel takes the op: column count in its table, whole-dword
// weight rows and 16-byte aligned float operands.
bool tiled_ok(const GemvOp& op)
{
    return gemv_tiled_cols(op.cols) && (reinterpret_cast<uintptr_t>(op.w) & 3u) == 0 && aligned16(op.x) &&
           aligned16(op.norm_weight) && aligned16(op.norm_bias) && aligned16(op.mix) && aligned16(op.prev) &&
           aligned16(op.norm_out);
}

int kind_of(const GemvOp& op)
{
    if (op.any_shape)
        return PATH_GENERIC;
    if (tiled_ok(op))
        return PATH_FAST;
    const int64_t nb = op.cols / block_elems(op.fmt);
    return nb <= SHORT_MAX_BLOCKS && op.cols <= SHORT_MAX_COLS ? PATH_SHORT : PATH_GENERIC;
}

hipError_t launch_group(const GemvOp* ops, int n, int kind, hipStream_t s)
{
    const int fmt = ops[0].fmt;
    if (kind == PATH_GENERIC || kind == PATH_SHORT) {
        const bool sh = kind == PATH_SHORT;
        switch (fmt) {
        case FMT_Q8_0: return sh ? launch_short<FMT_Q8_0>(ops, n, s) : launch_generic<FMT_Q8_0>(ops, n, s);
        case FMT_Q4_0: return sh ? launch_short<FMT_Q4_0>(ops, n, s) : launch_generic<FMT_Q4_0>(ops, n, s);
        case FMT_Q4_K: return sh ? launch_short<FMT_Q4_K>(ops, n, s) : launch_generic<FMT_Q4_K>(ops, n, s);
        case FMT_F16: return sh ? launch_short<FMT_F16>(ops, n, s) : launch_generic<FMT_F16>(ops, n, s);
        case FMT_F32: return sh ? launch_short<FMT_F32>(ops, n, s) : launch_generic<FMT_F32>(ops, n, s);
        default: return hipErrorInvalidValue;
        }
    }
    int64_t wrows = 0;
    for (int i = 0; i < n; i++)
        wrows += ops[i].out == OUT_SWIGLU_ROWS ? 2 * ops[i].rows : ops[i].rows;
    switch (fmt) {
    case FMT_Q8_0: return launch_fast<FMT_Q8_0>(ops, n, wrows, ops[0].cols, s);
    case FMT_Q4_0: return launch_fast<FMT_Q4_0>(ops, n, wrows, ops[0].cols, s);
    case FMT_Q4_K: return launch_fast<FMT_Q4_K>(ops, n, wrows, ops[0].cols, s);
    case FMT_F16: return launch_fast_dense<FMT_F16>(ops, n, wrows, ops[0].cols, s);
    case FMT_F32: return launch_fast_dense<FMT_F32>(ops, n, wrows, ops[0].cols, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_gemv_ops(const GemvOp* ops, int count, hipStream_t stream, int* paths)
{
    int i = 0;
    while (i < count) {
        const int kind = kind_of(ops[i]);
        if (kind != PATH_FAST && ops[i].in != XF_PLAIN)
            return hipErrorNotSupported;
        int n = 1;
        while (i + n < count && n < MAX_SEGS && ops[i + n].fmt == ops[i].fmt && kind_of(ops[i + n]) == kind &&
               (kind != PATH_FAST || ops[i + n].cols == ops[i].cols))
            n++;
        const hipError_t e = launch_group(ops + i, n, kind, stream);
        if (e != hipSuccess)
            return e;
        if (paths)
            for (int k = 0; k < n; k++)
                paths[i + k] = kind;
        i += n;
    }
    return hipSuccess;
}

hipError_t launch_gemv(int fmt, const void* w, const float* x, float* y, int64_t rows, int64_t cols,
                       const float* residual, hipStream_t stream, int* path)
{
    GemvOp op;
    op.fmt = fmt;
    op.w = w;
    op.x = x;
    op.y = y;
    op.rows = rows;
    op.cols = cols;
    op.residual = residual;
    return launch_gemv_ops(&op, 1, stream, path);
}

bool gemv_tiled_cols(int64_t cols)
{
    return cols == 1024 || cols == 2048 || cols == 3072 || cols == 4096 || cols == 6144 || cols == 8192;
}

hipError_t launch_dequant(int fmt, const void* wv, float* out, int64_t rows, int64_t cols, hipStream_t s)
{
    const uint8_t* w = static_cast<const uint8_t*>(wv);
    const int be = block_elems(fmt);
    if (be == 0)
        return hipErrorInvalidValue;
    const int64_t nblocks = rows * (cols / be);
    const dim3 grid(static_cast<unsigned>((nblocks + WG - 1) / WG));
    switch (fmt) {
    case FMT_Q8_0: hipLaunchKernelGGL((dequant_kernel<FMT_Q8_0>), grid, dim3(WG), 0, s, w, out, nblocks); break;
    case FMT_Q4_0: hipLaunchKernelGGL((dequant_kernel<FMT_Q4_0>), grid, dim3(WG), 0, s, w, out, nblocks); break;
    case FMT_Q4_K: hipLaunchKernelGGL((dequant_kernel<FMT_Q4_K>), grid, dim3(WG), 0, s, w, out, nblocks); break;
    case FMT_F16: hipLaunchKernelGGL((dequant_kernel<FMT_F16>), grid, dim3(WG), 0, s, w, out, nblocks); break;
    case FMT_F32: hipLaunchKernelGGL((dequant_kernel<FMT_F32>), grid, dim3(WG), 0, s, w, out, nblocks); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_checksum(const void* src, uint64_t bytes, uint32_t* parts, hipStream_t s)
{
    const uint64_t n16 = bytes / 16;
    const uint64_t cover = static_cast<uint64_t>(CHECKSUM_PARTS) * WG;   // 16-byte loads per load slot
    const int loads = n16 <= 2 * cover ? 2 : n16 <= 4 * cover ? 4 : n16 <= 8 * cover ? 8 : 16;
    const uint64_t chunks = (n16 + static_cast<uint64_t>(loads) * WG - 1) / (static_cast<uint64_t>(loads) * WG);
    const dim3 grid(static_cast<unsigned>(std::max<uint64_t>(1, std::min<uint64_t>(chunks, CHECKSUM_PARTS))));
    const uint32_t* w = static_cast<const uint32_t*>(src);
    switch (loads) {
    case 2: hipLaunchKernelGGL(checksum_kernel<2>, grid, dim3(WG), 0, s, w, bytes / 4, parts); break;
    case 4: hipLaunchKernelGGL(checksum_kernel<4>, grid, dim3(WG), 0, s, w, bytes / 4, parts); break;
    case 8: hipLaunchKernelGGL(checksum_kernel<8>, grid, dim3(WG), 0, s, w, bytes / 4, parts); break;
    default: hipLaunchKernelGGL(checksum_kernel<16>, grid, dim3(WG), 0, s, w, bytes / 4, parts); break;
    }
    return hipGetLastError();
}

hipError_t launch_fill_u32(void* dst, uint32_t value, uint64_t count, hipStream_t s)
{
    if (count == 0)
        return hipSuccess;
    const dim3 grid(static_cast<unsigned>((count + WG - 1) / WG));
    hipLaunchKernelGGL(fill_u32_kernel, grid, dim3(WG), 0, s, static_cast<uint32_t*>(dst), value, count);
    return hipGetLastError();
}

}  // namespace si
