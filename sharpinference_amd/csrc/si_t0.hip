// T0 primitive and portable tensor operators, one launch each: the
// operators an unfused logical graph (the portable RWKV-7 forward-token
// graph, PortableRwkv7GraphProvider.cs:13-295) dispatches between its
// mat-vecs.  Semantics follow the T0 contracts
// (TierZeroOperationContracts.cs, PortableTensorOperationContracts.cs:54-63)
// and the reference's GPU forms (GpuTierZeroInstruction.cs:376-466):
// elementwise FP32 arithmetic on dense tensors, maximum with NaN
// propagation and +0 above -0, tanh(0) = 0 exactly, sigmoid as
// 1 / (1 + exp(-x)), reductions in FP32.
//
// These are small vectors (a few KB to 512 KB): each launch is bound by its
// launch latency, so the kernels are plain grid-stride loops with 16-byte
// accesses where the operands allow, and one wave per reduced row.
#include "si_t0.hpp"
#include "si_lanes.hpp"

#include <hip/hip_fp16.h>

namespace si {
namespace {

constexpr int T0_THREADS = 256;

// IEEE 754-2019 maximum: NaN if either operand is NaN, +0 above -0
// (GpuInstructionHelpers.cs:7-8, TensorPrimitives.Max).
__device__ __forceinline__ float maximum32(float a, float b)
{
    if (a != a || b != b)
        return __uint_as_float(0x7fc00000u);
    if (a == 0.0f && b == 0.0f)
        return __uint_as_float(__float_as_uint(a) & __float_as_uint(b) & 0x80000000u);
    return a > b ? a : b;
}

template <int OP>
__device__ __forceinline__ float apply(float a, float b)
{
    if constexpr (OP == T0_COPY) return a;
    if constexpr (OP == T0_ADD) return a + b;
    if constexpr (OP == T0_SUBTRACT) return a - b;
    if constexpr (OP == T0_MULTIPLY) return a * b;
    if constexpr (OP == T0_DIVIDE) return a / b;
    if constexpr (OP == T0_MAXIMUM) return maximum32(a, b);
    if constexpr (OP == T0_EXP) return expf(a);
    if constexpr (OP == T0_TANH) return a == 0.0f ? a : tanhf(a);
    if constexpr (OP == T0_SIGMOID) return 1.0f / (1.0f + expf(-a));
    if constexpr (OP == T0_RSQRT) return 1.0f / sqrtf(a);
    if constexpr (OP == T0_SQUARE) return a * a;
    if constexpr (OP == T0_RELU) return maximum32(a, 0.0f);
    return 0.0f;
}

template <int OP, bool VEC>
__global__ __launch_bounds__(T0_THREADS) void elementwise_kernel(const float* __restrict__ l,
                                                                 const float* __restrict__ r, float* __restrict__ o,
                                                                 int64_t n)
{
    const int64_t stride = static_cast<int64_t>(gridDim.x) * T0_THREADS;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * T0_THREADS + threadIdx.x;
    if constexpr (VEC) {
        const int64_t n4 = n / 4;
        for (int64_t i = t; i < n4; i += stride) {
            const float4 a = reinterpret_cast<const float4*>(l)[i];
            float4 b = a;
            if (r)
                b = reinterpret_cast<const float4*>(r)[i];
            reinterpret_cast<float4*>(o)[i] =
                make_float4(apply<OP>(a.x, b.x), apply<OP>(a.y, b.y), apply<OP>(a.z, b.z), apply<OP>(a.w, b.w));
        }
    } else {
        for (int64_t i = t; i < n; i += stride)
            o[i] = apply<OP>(l[i], r ? r[i] : 0.0f);
    }
}

__global__ __launch_bounds__(T0_THREADS) void cast_f16_kernel(const __half* __restrict__ in, float* __restrict__ o,
                                                              int64_t n)
{
    const int64_t stride = static_cast<int64_t>(gridDim.x) * T0_THREADS;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * T0_THREADS + threadIdx.x; i < n; i += stride)
        o[i] = __half2float(in[i]);
}

__global__ __launch_bounds__(T0_THREADS) void fill_kernel(float* __restrict__ o, float v, int64_t n)
{
    const int64_t stride = static_cast<int64_t>(gridDim.x) * T0_THREADS;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * T0_THREADS + threadIdx.x; i < n; i += stride)
        o[i] = v;
}

// Sum over the 64 lanes of a wave, the result in every lane: DPP moves
// inside quads and 16-lane rows, then swaps between row pairs and halves.
__device__ __forceinline__ float wave_sum(float v)
{
    v += dpp_row<0xB1>(v);   // quad_perm 1,0,3,2
    v += dpp_row<0x4E>(v);   // quad_perm 2,3,0,1
    v += dpp_row<0x141>(v);  // row_half_mirror
    v += dpp_row<0x140>(v);  // row_mirror
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// out[r] = sum_c in[r][c] (divided by cols when MEAN): one wave per row,
// lane-strided partial sums in a fixed order, then the wave tree.
template <bool MEAN>
__global__ __launch_bounds__(T0_THREADS) void reduce_last_kernel(const float* __restrict__ in, float* __restrict__ o,
                                                                 int64_t rows, int64_t cols)
{
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (T0_THREADS / 64) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows)   // wave-uniform: the whole wave leaves
        return;
    const float* p = in + row * cols;
    float s = 0.0f;
    for (int64_t c = lane; c < cols; c += 64)
        s += p[c];
    s = wave_sum(s);
    if (lane == 0)
        o[row] = MEAN ? s / static_cast<float>(cols) : s;
}

// out[i] = in[base + sum_a coord_a(i) * stride_a] over the output's
// row-major coordinates (rank <= 4): broadcast (stride 0 on repeated axes)
// and slice (the input's strides, base = start * stride of the axis).
__global__ __launch_bounds__(T0_THREADS) void gather_kernel(const float* __restrict__ in, float* __restrict__ o,
                                                            GatherShape g)
{
    const int64_t stride = static_cast<int64_t>(gridDim.x) * T0_THREADS;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * T0_THREADS + threadIdx.x; i < g.count; i += stride) {
        int64_t flat = i, s = g.base;
        for (int a = g.rank - 1; a >= 0; a--) {
            const int64_t c = flat % g.dims[a];
            flat /= g.dims[a];
            s += c * g.strides[a];
        }
        o[i] = in[s];
    }
}

// out[h][i][j] = left[h][i] * right[h][j].
__global__ __launch_bounds__(T0_THREADS) void head_outer_kernel(const float* __restrict__ l,
                                                                const float* __restrict__ r, float* __restrict__ o,
                                                                int64_t heads, int64_t rows, int64_t cols)
{
    const int64_t n = heads * rows * cols;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * T0_THREADS;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * T0_THREADS + threadIdx.x; i < n; i += stride) {
        const int64_t h = i / (rows * cols), k = i - h * rows * cols;
        const int64_t row = k / cols, col = k - row * cols;
        o[i] = l[h * rows + row] * r[h * cols + col];
    }
}

unsigned blocks_for(int64_t n)
{
    const int64_t b = (n + T0_THREADS - 1) / T0_THREADS;
    return static_cast<unsigned>(b < 1 ? 1 : b > 4096 ? 4096 : b);
}

template <int OP>
hipError_t launch_op(const float* l, const float* r, float* o, int64_t n, hipStream_t s)
{
    const bool vec = n % 4 == 0 && ((reinterpret_cast<uintptr_t>(l) | reinterpret_cast<uintptr_t>(r) |
                                     reinterpret_cast<uintptr_t>(o)) & 15u) == 0;
    if (vec)
        hipLaunchKernelGGL((elementwise_kernel<OP, true>), dim3(blocks_for(n / 4)), dim3(T0_THREADS), 0, s, l, r, o, n);
    else
        hipLaunchKernelGGL((elementwise_kernel<OP, false>), dim3(blocks_for(n)), dim3(T0_THREADS), 0, s, l, r, o, n);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_t0_elementwise(int op, const float* l, const float* r, float* o, int64_t n, hipStream_t s)
{
    switch (op) {
    case T0_COPY: return launch_op<T0_COPY>(l, nullptr, o, n, s);
    case T0_ADD: return launch_op<T0_ADD>(l, r, o, n, s);
    case T0_SUBTRACT: return launch_op<T0_SUBTRACT>(l, r, o, n, s);
    case T0_MULTIPLY: return launch_op<T0_MULTIPLY>(l, r, o, n, s);
    case T0_DIVIDE: return launch_op<T0_DIVIDE>(l, r, o, n, s);
    case T0_MAXIMUM: return launch_op<T0_MAXIMUM>(l, r, o, n, s);
    case T0_EXP: return launch_op<T0_EXP>(l, nullptr, o, n, s);
    case T0_TANH: return launch_op<T0_TANH>(l, nullptr, o, n, s);
    case T0_SIGMOID: return launch_op<T0_SIGMOID>(l, nullptr, o, n, s);
    case T0_RSQRT: return launch_op<T0_RSQRT>(l, nullptr, o, n, s);
    case T0_SQUARE: return launch_op<T0_SQUARE>(l, nullptr, o, n, s);
    case T0_RELU: return launch_op<T0_RELU>(l, nullptr, o, n, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_t0_cast_f16(const void* in, float* o, int64_t n, hipStream_t s)
{
    hipLaunchKernelGGL(cast_f16_kernel, dim3(blocks_for(n)), dim3(T0_THREADS), 0, s, static_cast<const __half*>(in),
                       o, n);
    return hipGetLastError();
}

hipError_t launch_t0_fill(float* o, float v, int64_t n, hipStream_t s)
{
    hipLaunchKernelGGL(fill_kernel, dim3(blocks_for(n)), dim3(T0_THREADS), 0, s, o, v, n);
    return hipGetLastError();
}

hipError_t launch_t0_reduce_last(bool mean, const float* in, float* o, int64_t rows, int64_t cols, hipStream_t s)
{
    const dim3 grid(static_cast<unsigned>((rows + T0_THREADS / 64 - 1) / (T0_THREADS / 64)));
    if (mean)
        hipLaunchKernelGGL((reduce_last_kernel<true>), grid, dim3(T0_THREADS), 0, s, in, o, rows, cols);
    else
        hipLaunchKernelGGL((reduce_last_kernel<false>), grid, dim3(T0_THREADS), 0, s, in, o, rows, cols);
    return hipGetLastError();
}

hipError_t launch_t0_gather(const float* in, float* o, const GatherShape& g, hipStream_t s)
{
    hipLaunchKernelGGL(gather_kernel, dim3(blocks_for(g.count)), dim3(T0_THREADS), 0, s, in, o, g);
    return hipGetLastError();
}

hipError_t launch_t0_head_outer(const float* l, const float* r, float* o, int64_t heads, int64_t rows, int64_t cols,
                                hipStream_t s)
{
    hipLaunchKernelGGL(head_outer_kernel, dim3(blocks_for(heads * rows * cols)), dim3(T0_THREADS), 0, s, l, r, o,
                       heads, rows, cols);
    return hipGetLastError();
}

}  // namespace si
