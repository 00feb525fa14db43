// Batched prefill product Y[m, n] = sum_k X[m, k] * W[n, k] on MFMA.
//
// W is a GGUF block-quantized matrix [N, K] (Q4_0, Q8_0 or Q4_K), X holds M
// token rows of bf16 activations [M, K], Y is FP32 [M, N] (one output row per
// token), FP32 accumulation.  Reference semantics: the transpose_right branch
// of CpuInstructionNumerics.MatrixMultiply
// (SharpInference.Instructions.Cpu/CpuInstructionNumerics.cs:66-77), i.e. one
// core.mat-vec per token row, and the batched prefill matvec of the D3D12
// transformer program (GpuBatchTransformerInstructions.cs:224-279), whose B=16
// token batch re-reads W per token.  Here every W element is decoded once per
// workgroup tile of 128 or 256 tokens:
//
//   * a workgroup (4 waves) owns 32*NT rows of W and 4*MW token rows of X;
//   * per step of two 32-column blocks, the 256 threads decode the blocks of
//     each W row exactly as the CPU decoder does (FP32, one rounding per
//     operation), round them to bf16 and write a double-buffered LDS tile;
//     the raw bytes are loaded a step ahead;
//   * each wave multiplies its MW token rows by the tile with
//     v_mfma_f32_32x32x16_bf16 (MW/32 x NT accumulator tiles of 32 x 32
//     FP32), its X fragments loaded a step ahead straight from global memory
//     (X is small and stays in L2 / the Infinity Cache);
//   * the tile is the largest whose grid still covers the 256 CUs.
//
// MFMA fragment layout (32x32x16 bf16): lane l holds A[l % 32][8*(l/32)+e]
// and B[8*(l/32)+e][l % 32] for e = 0..7; accumulator register r of lane l
// is C[8*(r/4) + 4*(l/32) + r%4][l % 32].
#include "si_internal.hpp"

#include <hip/hip_fp16.h>

namespace si {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int PF_THREADS = 256;
constexpr int WS_STRIDE = 40;       // bf16 per LDS tile row: 32 values + 8 pad

// Raw bytes of one group of 4 values, loaded a step ahead of their decode.
struct Raw4 {
    uint32_t a, b, c;
};

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p)
{
    return *reinterpret_cast<const unsigned short*>(p);
}

template <int FMT>
__device__ __forceinline__ Raw4 load_raw(const uint8_t* row, int blk, int p);

// Q8_0 {fp16 d; int8 q[32]}: d, q[4p..4p+1], q[4p+2..4p+3] (2-byte aligned)
template <>
__device__ __forceinline__ Raw4 load_raw<FMT_Q8_0>(const uint8_t* row, int blk, int p)
{
    const uint8_t* b = row + blk * 34;
    return Raw4{ld_u16(b), ld_u16(b + 2 + 4 * p), ld_u16(b + 4 + 4 * p)};
}

// Q4_0 {fp16 d; u8 qs[16]}: d and the 4 bytes holding elements 4p..4p+3
template <>
__device__ __forceinline__ Raw4 load_raw<FMT_Q4_0>(const uint8_t* row, int blk, int p)
{
    const uint8_t* b = row + blk * 18;
    const uint8_t* q = b + 2 + 4 * (p & 3);
    return Raw4{ld_u16(b), ld_u16(q), ld_u16(q + 2)};
}

// Q4_K: d | dmin << 16, the 3 scale bytes of sub-block j, 4 quant bytes
// (16-byte aligned super-blocks, so the quant word is dword aligned)
template <>
__device__ __forceinline__ Raw4 load_raw<FMT_Q4_K>(const uint8_t* row, int blk, int p)
{
    const uint8_t* b = row + (blk >> 3) * 144;
    const int j = blk & 7;
    const uint8_t* s = b + 4;
    const uint32_t sb = j < 4 ? (s[j] | (s[j + 4] << 8)) : (s[j + 4] | (s[j - 4] << 8) | (s[j] << 16));
    return Raw4{ld_u16(b) | (ld_u16(b + 2) << 16), sb,
                *reinterpret_cast<const uint32_t*>(b + 16 + 32 * (j >> 1) + 4 * p)};
}

__device__ __forceinline__ float half_bits(uint32_t h)
{
    return __half2float(__ushort_as_half(static_cast<unsigned short>(h & 0xffffu)));
}

// The 4 values in FP32, bit-identical to the block decoder (one rounding
// per operation).
template <int FMT>
__device__ __forceinline__ void decode_raw(const Raw4& r, int blk, int p, float out[4]);

template <>
__device__ __forceinline__ void decode_raw<FMT_Q8_0>(const Raw4& r, int, int, float out[4])
{
    const float d = half_bits(r.a);
    const uint32_t q = r.b | (r.c << 16);
#pragma unroll
    for (int i = 0; i < 4; i++)
        out[i] = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(q >> (8 * i))));
}

template <>
__device__ __forceinline__ void decode_raw<FMT_Q4_0>(const Raw4& r, int, int p, float out[4])
{
    const float d = half_bits(r.a);
    const uint32_t q = r.b | (r.c << 16);
    const int shift = p < 4 ? 0 : 4;
#pragma unroll
    for (int i = 0; i < 4; i++)
        out[i] = __fmul_rn(d, static_cast<float>(static_cast<int>((q >> (8 * i + shift)) & 15) - 8));
}

template <>
__device__ __forceinline__ void decode_raw<FMT_Q4_K>(const Raw4& r, int blk, int, float out[4])
{
    const int j = blk & 7;
    const float d = half_bits(r.a), dmin = half_bits(r.a >> 16);
    int sc, m;
    if (j < 4) {
        sc = r.b & 63;
        m = (r.b >> 8) & 63;
    } else {   // bytes s[j+4], s[j-4], s[j]
        sc = (r.b & 15) | (((r.b >> 8) >> 6 & 3) << 4);
        m = ((r.b >> 4) & 15) | (((r.b >> 16) >> 6 & 3) << 4);
    }
    const float d1 = __fmul_rn(d, static_cast<float>(sc));
    const float m1 = __fmul_rn(dmin, static_cast<float>(m));
    const int shift = 4 * (j & 1);
#pragma unroll
    for (int i = 0; i < 4; i++)
        out[i] = __fsub_rn(__fmul_rn(d1, static_cast<float>((r.c >> (8 * i + shift)) & 15)), m1);
}

// MW token rows per wave (32 or 64: MW / 32 accumulator tiles along M),
// 32 * NT rows of W per workgroup, two 32-column blocks per step.  The raw
// W bytes of step s + 1 and the X fragments of step s + 1 are requested
// before the matrix-core work of step s, and decoded into the other LDS
// buffer after it, so memory latency hides behind the MFMAs; one barrier
// per step.
template <int FMT, int MW, int NT>
__global__ __launch_bounds__(PF_THREADS) void prefill_mfma_kernel(const uint8_t* __restrict__ W,
                                                                   const __bf16* __restrict__ X,
                                                                   float* __restrict__ Y, int M, int N, int K,
                                                                   int64_t row_bytes)
{
    constexpr int MT = MW / 32;                           // accumulator tiles along M per wave
    constexpr int NROWS = 32 * NT;                        // W rows per workgroup
    constexpr int BPS = 2;                                // 32-column blocks per step
    constexpr int GROUPS = NROWS * 8 * BPS / PF_THREADS;  // 4-value groups per thread per step
    static_assert(GROUPS * PF_THREADS == NROWS * 8 * BPS, "whole groups per thread");
    __shared__ __attribute__((aligned(16))) __bf16 ws[2][BPS][NROWS * WS_STRIDE];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = blockIdx.x * NROWS;
    const int m0 = blockIdx.y * (4 * MW) + wave * MW;
    const int g = lane >> 5;          // K group of the fragment (0, 1)
    const int li = lane & 31;
    const int nblk = K / 32;
    const int nsteps = (nblk + BPS - 1) / BPS;

    // token rows of this lane's A fragments (clamped for loads)
    const __bf16* xrow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
        xrow[mt] = X + static_cast<int64_t>(min(m0 + 32 * mt + li, M - 1)) * K + 8 * g;

    // this thread's decode groups: (block of the step, W row, part)
    int gb[GROUPS], gp[GROUPS];
    const uint8_t* grow[GROUPS];
#pragma unroll
    for (int e = 0; e < GROUPS; e++) {
        const int item = threadIdx.x + e * PF_THREADS;
        gb[e] = item / (NROWS * 8);
        const int rem = item % (NROWS * 8);
        gp[e] = rem & 7;
        grow[e] = W + static_cast<int64_t>(min(n0 + (rem >> 3), N - 1)) * row_bytes;
    }

    f32x16 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
            acc[mt][nt] = f32x16{};

    Raw4 raw[GROUPS];
    auto load_step = [&](int step) {
#pragma unroll
        for (int e = 0; e < GROUPS; e++) {
            const int blk = min(BPS * step + gb[e], nblk - 1);
            raw[e] = load_raw<FMT>(grow[e], blk, gp[e]);
        }
    };
    auto store_step = [&](int step, int buf) {
#pragma unroll
        for (int e = 0; e < GROUPS; e++) {
            const int blk = min(BPS * step + gb[e], nblk - 1);
            float v[4];
            decode_raw<FMT>(raw[e], blk, gp[e], v);
            bf16x4 h;
            h[0] = static_cast<__bf16>(v[0]);
            h[1] = static_cast<__bf16>(v[1]);
            h[2] = static_cast<__bf16>(v[2]);
            h[3] = static_cast<__bf16>(v[3]);
            const int r = (threadIdx.x + e * PF_THREADS) % (NROWS * 8) >> 3;
            *reinterpret_cast<bf16x4*>(&ws[buf][gb[e]][r * WS_STRIDE + 4 * gp[e]]) = h;
        }
    };
    bf16x8 a[BPS][MT][2], an[BPS][MT][2];
    auto load_a = [&](int step, bf16x8 (&dst)[BPS][MT][2]) {
#pragma unroll
        for (int bo = 0; bo < BPS; bo++) {
            const int blk = min(BPS * step + bo, nblk - 1);
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int h = 0; h < 2; h++)
                    dst[bo][mt][h] = *reinterpret_cast<const bf16x8*>(xrow[mt] + blk * 32 + 16 * h);
        }
    };

    load_step(0);
    load_a(0, a);
    store_step(0, 0);
    __syncthreads();
    for (int step = 0; step < nsteps; step++) {
        const int buf = step & 1;
        const bool more = step + 1 < nsteps;
        if (more) {
            load_step(step + 1);
            load_a(step + 1, an);
        }
#pragma unroll
        for (int bo = 0; bo < BPS; bo++) {
            if (BPS * step + bo < nblk) {
#pragma unroll
                for (int h = 0; h < 2; h++) {
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) {
                        const bf16x8 b =
                            *reinterpret_cast<const bf16x8*>(&ws[buf][bo][(32 * nt + li) * WS_STRIDE + 16 * h + 8 * g]);
#pragma unroll
                        for (int mt = 0; mt < MT; mt++)
                            acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[bo][mt][h], b, acc[mt][nt], 0, 0, 0);
                    }
                }
            }
        }
        if (more) {
            store_step(step + 1, buf ^ 1);
#pragma unroll
            for (int bo = 0; bo < BPS; bo++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int h = 0; h < 2; h++)
                        a[bo][mt][h] = an[bo][mt][h];
        }
        __syncthreads();
    }

#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int n = n0 + 32 * nt + li;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = m0 + 32 * mt + 8 * (r >> 2) + 4 * g + (r & 3);
                if (m < M && n < N)
                    Y[static_cast<int64_t>(m) * N + n] = acc[mt][nt][r];
            }
        }
    }
}

template <int FMT, int MW, int NT>
hipError_t launch_prefill_shape(const void* w, const void* x, float* y, int64_t m, int64_t n, int64_t k, hipStream_t s)
{
    const int64_t rb = row_bytes(FMT, k);
    const dim3 grid(static_cast<unsigned>((n + 32 * NT - 1) / (32 * NT)), static_cast<unsigned>((m + 4 * MW - 1) / (4 * MW)));
    hipLaunchKernelGGL((prefill_mfma_kernel<FMT, MW, NT>), grid, dim3(PF_THREADS), 0, s, static_cast<const uint8_t*>(w),
                       static_cast<const __bf16*>(x), y, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k), rb);
    return hipGetLastError();
}

// The largest tile whose grid still covers the 256 CUs: 256 tokens x 64
// rows, else 128 x 64, else 128 x 32.
template <int FMT>
hipError_t launch_prefill_fmt(const void* w, const void* x, float* y, int64_t m, int64_t n, int64_t k, hipStream_t s)
{
    auto wgs = [&](int mt, int nt) { return ((n + nt - 1) / nt) * ((m + mt - 1) / mt); };
    if (wgs(256, 64) >= 256)
        return launch_prefill_shape<FMT, 64, 2>(w, x, y, m, n, k, s);
    if (wgs(128, 64) >= 256)
        return launch_prefill_shape<FMT, 32, 2>(w, x, y, m, n, k, s);
    return launch_prefill_shape<FMT, 32, 1>(w, x, y, m, n, k, s);
}

}  // namespace

hipError_t launch_prefill(int fmt, const void* w, const void* x_bf16, float* y, int64_t m, int64_t rows, int64_t cols,
                          hipStream_t stream)
{
    switch (fmt) {
    case FMT_Q8_0: return launch_prefill_fmt<FMT_Q8_0>(w, x_bf16, y, m, rows, cols, stream);
    case FMT_Q4_0: return launch_prefill_fmt<FMT_Q4_0>(w, x_bf16, y, m, rows, cols, stream);
    case FMT_Q4_K: return launch_prefill_fmt<FMT_Q4_K>(w, x_bf16, y, m, rows, cols, stream);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace si
