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
// 256 tokens:
//
//   * a workgroup (4 waves) owns 32*NT rows of W and 256 token rows of X;
//   * per 32-column block step, the 256 threads decode the block of each W
//     row exactly as the CPU decoder does (FP32, one rounding per operation),
//     round it to bf16 and write it to a double-buffered LDS tile;
//   * each wave multiplies its 64 token rows by the tile with
//     v_mfma_f32_32x32x16_bf16 (2 x NT accumulator tiles of 32 x 32 FP32),
//     its X fragments loaded straight from global memory (X is small and
//     stays in L2 / the Infinity Cache).
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
constexpr int PF_MT = 256;          // token rows per workgroup
constexpr int WS_STRIDE = 40;       // bf16 per LDS tile row: 32 values + 8 pad

__device__ __forceinline__ float ld_half_u(const uint8_t* p)
{
    const unsigned short h = static_cast<unsigned short>(p[0] | (p[1] << 8));
    return __half2float(__ushort_as_half(h));
}

// The 4 decoded values (elements 4p..4p+3 of block `blk` of row `row`) in
// FP32, bit-identical to the block decoder.
template <int FMT>
__device__ __forceinline__ void decode4(const uint8_t* row, int blk, int p, float out[4]);

template <>
__device__ __forceinline__ void decode4<FMT_Q8_0>(const uint8_t* row, int blk, int p, float out[4])
{
    const uint8_t* b = row + blk * 34;
    const float d = ld_half_u(b);
#pragma unroll
    for (int i = 0; i < 4; i++)
        out[i] = __fmul_rn(d, static_cast<float>(static_cast<int8_t>(b[2 + 4 * p + i])));
}

template <>
__device__ __forceinline__ void decode4<FMT_Q4_0>(const uint8_t* row, int blk, int p, float out[4])
{
    const uint8_t* b = row + blk * 18;
    const float d = ld_half_u(b);
    const int shift = p < 4 ? 0 : 4;
    const uint8_t* q = b + 2 + 4 * (p & 3);
#pragma unroll
    for (int i = 0; i < 4; i++)
        out[i] = __fmul_rn(d, static_cast<float>(((q[i] >> shift) & 15) - 8));
}

template <>
__device__ __forceinline__ void decode4<FMT_Q4_K>(const uint8_t* row, int blk, int p, float out[4])
{
    // block = 32-element sub-block j of super-block blk / 8
    const uint8_t* b = row + (blk >> 3) * 144;
    const int j = blk & 7;
    const float d = ld_half_u(b), dmin = ld_half_u(b + 2);
    const uint8_t* s = b + 4;
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
    const uint8_t* q = b + 16 + 32 * (j >> 1) + 4 * p;
    const int shift = 4 * (j & 1);
#pragma unroll
    for (int i = 0; i < 4; i++)
        out[i] = __fsub_rn(__fmul_rn(d1, static_cast<float>((q[i] >> shift) & 15)), m1);
}

template <int FMT, int NT>
__global__ __launch_bounds__(PF_THREADS) void prefill_mfma_kernel(const uint8_t* __restrict__ W,
                                                                   const __bf16* __restrict__ X,
                                                                   float* __restrict__ Y, int M, int N, int K,
                                                                   int64_t row_bytes)
{
    constexpr int NROWS = 32 * NT;                        // W rows per workgroup
    constexpr int ELEMS = NROWS * 32 / PF_THREADS;        // decoded values per thread per step
    static_assert(ELEMS % 4 == 0, "threads decode groups of 4 values");
    __shared__ __attribute__((aligned(16))) __bf16 ws[2][NROWS * WS_STRIDE];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = blockIdx.x * NROWS;
    const int m0 = blockIdx.y * PF_MT + wave * 64;
    const int g = lane >> 5;          // K group of the fragment (0, 1)
    const int li = lane & 31;
    const int nblk = K / 32;

    // token rows of this lane's A fragments (clamped for loads)
    const __bf16* xrow[2];
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
        xrow[mt] = X + static_cast<int64_t>(min(m0 + 32 * mt + li, M - 1)) * K + 8 * g;

    f32x16 acc[2][NT];
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
            acc[mt][nt] = f32x16{};

    auto decode_step = [&](int blk, int buf) {
#pragma unroll
        for (int e = 0; e < ELEMS / 4; e++) {
            const int item = threadIdx.x + e * PF_THREADS;    // (row, part) pairs
            const int r = item >> 3, p = item & 7;
            const uint8_t* rp = W + static_cast<int64_t>(min(n0 + r, N - 1)) * row_bytes;
            float v[4];
            decode4<FMT>(rp, blk, p, v);
            bf16x4 h;
            h[0] = static_cast<__bf16>(v[0]);
            h[1] = static_cast<__bf16>(v[1]);
            h[2] = static_cast<__bf16>(v[2]);
            h[3] = static_cast<__bf16>(v[3]);
            *reinterpret_cast<bf16x4*>(&ws[buf][r * WS_STRIDE + 4 * p]) = h;
        }
    };

    decode_step(0, 0);
    __syncthreads();
    for (int blk = 0; blk < nblk; blk++) {
        const int buf = blk & 1;
        // A fragments of this block (two K halves of 16)
        bf16x8 a[2][2];
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int h = 0; h < 2; h++)
                a[mt][h] = *reinterpret_cast<const bf16x8*>(xrow[mt] + blk * 32 + 16 * h);
        // decode the next block into the other buffer while this one is used
        if (blk + 1 < nblk)
            decode_step(blk + 1, buf ^ 1);
#pragma unroll
        for (int h = 0; h < 2; h++) {
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                const bf16x8 b = *reinterpret_cast<const bf16x8*>(&ws[buf][(32 * nt + li) * WS_STRIDE + 16 * h + 8 * g]);
#pragma unroll
                for (int mt = 0; mt < 2; mt++)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[mt][h], b, acc[mt][nt], 0, 0, 0);
            }
        }
        __syncthreads();
    }

#pragma unroll
    for (int mt = 0; mt < 2; mt++) {
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

template <int FMT>
hipError_t launch_prefill_fmt(const void* w, const void* x, float* y, int64_t m, int64_t n, int64_t k, hipStream_t s)
{
    constexpr int NT = 2;
    const int64_t rb = row_bytes(FMT, k);
    const dim3 grid(static_cast<unsigned>((n + 32 * NT - 1) / (32 * NT)), static_cast<unsigned>((m + PF_MT - 1) / PF_MT));
    hipLaunchKernelGGL((prefill_mfma_kernel<FMT, NT>), grid, dim3(PF_THREADS), 0, s, static_cast<const uint8_t*>(w),
                       static_cast<const __bf16*>(x), y, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k), rb);
    return hipGetLastError();
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
