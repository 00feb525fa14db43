// The transformer operators of the reference's D3D12 decode program as
// separate launches, with the reference's semantics and buffer layouts
// (SharpInference.Instructions.D3D12/GpuTransformerInstructionCollection.cs):
//
//   rms-norm            :323-368   out = x * (1 / sqrt(sum(x^2) / n + eps)) * w
//   residual-rms-norm   :370-417   updated = hidden + residual; out = rms-norm(updated)
//   swiglu              :419-443   out_i = g_i / (1 + exp(-g_i)) * u_i over [g | u]
//   rope-kv-write       :445-543   rotate q and k of one token at *position, write
//                                  q to `query` and k, v to cache row *position
//   grouped-query-attention :46-143  softmax(q . K^T / sqrt(head)) . V over rows
//                                  0..min(max(*position, 0), context - 1), split
//                                  into 64-row chunks merged by a second launch
//
// KV caches are [context][kv_heads][head_size] (a token's row holds every KV
// head), FP32 as in the reference or fp16 (rounded to nearest even on
// write).  The fused decode step (si_decode.hip) keeps its own layout; these
// launches are the op-by-op form a VM program dispatches.
#include "si_internal.hpp"
#include "si_transformer.hpp"

#include <hip/hip_fp16.h>

namespace si {
namespace {

constexpr int NORM_THREADS = 1024;

__device__ __forceinline__ float wave_sum_f(float v)
{
    for (int off = 32; off > 0; off >>= 1)
        v += __shfl_xor(v, off);
    return v;
}

__device__ __forceinline__ float wave_max_f(float v)
{
    for (int off = 32; off > 0; off >>= 1)
        v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// Sum over the workgroup (every thread gets it); `red` holds one float per wave.
template <int THREADS>
__device__ __forceinline__ float block_sum(float v, float* red)
{
    v = wave_sum_f(v);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < THREADS / 64; w++)
        t += red[w];
    __syncthreads();
    return t;
}

template <int THREADS>
__device__ __forceinline__ float block_max(float v, float* red)
{
    v = wave_max_f(v);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = red[0];
#pragma unroll
    for (int w = 1; w < THREADS / 64; w++)
        t = fmaxf(t, red[w]);
    __syncthreads();
    return t;
}

// One workgroup: the sum of squares of (hidden [+ residual]) over n values,
// then out_j = v_j * scale * w_j (the reference's operation order).
template <bool RESIDUAL>
__global__ __launch_bounds__(NORM_THREADS) void rms_norm_kernel(const float* __restrict__ hidden,
                                                                const float* __restrict__ residual,
                                                                const float* __restrict__ weight,
                                                                float* __restrict__ updated, float* __restrict__ out,
                                                                int n, float eps)
{
    __shared__ float red[NORM_THREADS / 64];
    float ss = 0.0f;
    for (int j = threadIdx.x; j < n; j += NORM_THREADS) {
        float v = hidden[j];
        if (RESIDUAL) {
            v = v + residual[j];
            updated[j] = v;
        }
        ss = fmaf(v, v, ss);
    }
    const float total = block_sum<NORM_THREADS>(ss, red);
    const float scale = 1.0f / sqrtf(total / static_cast<float>(n) + eps);
    for (int j = threadIdx.x; j < n; j += NORM_THREADS) {
        // each thread re-reads only values it wrote itself above
        const float v = RESIDUAL ? updated[j] : hidden[j];
        out[j] = v * scale * weight[j];
    }
}

__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ gate_up, float* __restrict__ out,
                                                     int64_t n)
{
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < n) {
        const float g = gate_up[i];
        out[i] = g / (1.0f + expf(-g)) * gate_up[n + i];
    }
}

template <typename T>
__device__ __forceinline__ void store_cache(T* cache, int64_t i, float v);
template <>
__device__ __forceinline__ void store_cache<float>(float* cache, int64_t i, float v) { cache[i] = v; }
template <>
__device__ __forceinline__ void store_cache<__half>(__half* cache, int64_t i, float v) { cache[i] = __float2half_rn(v); }

// One thread per value of qkv = [q (query_size) | k (kv_size) | v (kv_size)].
template <typename T>
__global__ __launch_bounds__(256) void rope_kv_write_kernel(RopeKvWriteArgs a, T* __restrict__ kc, T* __restrict__ vc)
{
    const int total = a.query_size + 2 * a.kv_size;
    const int i = static_cast<int>(blockIdx.x) * 256 + threadIdx.x;
    const int token = *a.position;
    if (token < 0 || token >= a.context || i >= total)
        return;
    const int half = a.rotary_size / 2;
    auto rotate = [&](int local, float value) {
        const int d = local % a.head_size;
        if (d >= a.rotary_size)
            return value;
        const int ri = d < half ? d : d - half;
        const int pair = d < half ? i + half : i - half;
        const float angle = static_cast<float>(token) * a.frequencies[ri];
        const float c = cosf(angle) * a.rope_scale, s = sinf(angle) * a.rope_scale;
        const float other = a.qkv[pair];
        return d < half ? value * c - other * s : value * c + other * s;
    };
    const float value = a.qkv[i];
    if (i < a.query_size) {
        a.query[i] = rotate(i, value);
    } else if (i < a.query_size + a.kv_size) {
        const int local = i - a.query_size;
        store_cache<T>(kc, static_cast<int64_t>(token) * a.kv_size + local, rotate(local, value));
    } else {
        const int local = i - a.query_size - a.kv_size;
        store_cache<T>(vc, static_cast<int64_t>(token) * a.kv_size + local, value);
    }
}

// 8 consecutive cache values of one row as floats (one 16-byte fp16 load or
// two 16-byte FP32 loads).
__device__ __forceinline__ void load8(const float* p, float* f)
{
    const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}
__device__ __forceinline__ void load8(const __half* p, float* f)
{
    const uint4 r = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        f[2 * k] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[k] & 0xffffu)));
        f[2 * k + 1] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[k] >> 16)));
    }
}
__device__ __forceinline__ float load1(const float* p) { return *p; }
__device__ __forceinline__ float load1(const __half* p) { return __half2float(*p); }

constexpr int GQA_THREADS = 256;
constexpr int GQA_CHUNK = 64;      // cache rows per partial workgroup

// One workgroup per (query head, 64-row chunk): scores of the chunk's rows
// (head_size / 8 lanes per row, 8 channels each: coalesced row reads,
// shuffle sums), the chunk's softmax maximum m and sum l, and its
// unnormalised weighted sum of value rows o; partial (m, l, o[head]) goes
// to the workspace.  Rows past the active range count as absent (weight 0);
// a chunk wholly past it is never read by the merge.
template <typename T, int HEAD>
__global__ __launch_bounds__(GQA_THREADS) void gqa_partial_kernel(GqaArgs a, const T* __restrict__ kc,
                                                                  const T* __restrict__ vc)
{
    __shared__ float scores[GQA_CHUNK];
    __shared__ float red[GQA_THREADS / 64];
    __shared__ float vpart[GQA_THREADS];
    constexpr int LPT = HEAD / 8;                  // lanes per cache row
    constexpr int ROWS = GQA_THREADS / LPT;        // rows per pass
    constexpr int PASSES = GQA_CHUNK / ROWS;
    const int head = blockIdx.x, chunk = blockIdx.y;
    const int kvh = head / (a.query_heads / a.kv_heads);
    const int active = min(max(*a.position, 0), a.context - 1);
    const int t0 = chunk * GQA_CHUNK;
    if (t0 > active)
        return;                                    // whole workgroup: nothing to merge from this chunk
    const int64_t row_stride = static_cast<int64_t>(a.kv_heads) * HEAD;
    const float scale = 1.0f / sqrtf(static_cast<float>(HEAD));
    const int part = threadIdx.x % LPT, sub = threadIdx.x / LPT;
    float q[8];
    load8(a.query + static_cast<int64_t>(head) * HEAD + 8 * part, q);
    float k[PASSES][8];
#pragma unroll
    for (int i = 0; i < PASSES; i++) {
        const int t = min(t0 + i * ROWS + sub, active);
        load8(kc + static_cast<int64_t>(t) * row_stride + static_cast<int64_t>(kvh) * HEAD + 8 * part, k[i]);
    }
#pragma unroll
    for (int i = 0; i < PASSES; i++) {
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; c++)
            s = fmaf(q[c], k[i][c], s);
#pragma unroll
        for (int off = LPT / 2; off > 0; off >>= 1)
            s += __shfl_xor(s, off);
        const int r = i * ROWS + sub;
        if (part == 0)
            scores[r] = t0 + r <= active ? s * scale : -INFINITY;
    }
    __syncthreads();
    float m = -INFINITY;
    if (threadIdx.x < GQA_CHUNK)
        m = scores[threadIdx.x];
    m = block_max<GQA_THREADS>(m, red);            // finite: row t0 is active
    float p = 0.0f;
    if (threadIdx.x < GQA_CHUNK) {
        p = expf(scores[threadIdx.x] - m);         // exp(-inf) = 0 for absent rows
        scores[threadIdx.x] = p;
    }
    const float l = block_sum<GQA_THREADS>(p, red);   // its barriers also publish the weights
    const int rows = min(GQA_CHUNK, active - t0 + 1);
    float* dst = a.workspace + (static_cast<int64_t>(head) * a.chunks + chunk) * (HEAD + 2);
    for (int d0 = 0; d0 < HEAD; d0 += GQA_THREADS / 2) {
        const int d = d0 + threadIdx.x % (GQA_THREADS / 2), h2 = threadIdx.x / (GQA_THREADS / 2);
        float acc = 0.0f;
        if (d < HEAD) {
            const T* vrow = vc + static_cast<int64_t>(t0) * row_stride + static_cast<int64_t>(kvh) * HEAD + d;
            for (int r = h2; r < rows; r += 2)
                acc = fmaf(scores[r], load1(vrow + static_cast<int64_t>(r) * row_stride), acc);
        }
        vpart[threadIdx.x] = acc;
        __syncthreads();
        if (h2 == 0 && d < HEAD)
            dst[2 + d] = acc + vpart[threadIdx.x + GQA_THREADS / 2];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        dst[0] = m;
        dst[1] = l;
    }
}

// One workgroup per query head: out = sum_c o_c e^(m_c - M) / sum_c l_c e^(m_c - M)
// over the active chunks, M = max_c m_c.
template <int HEAD>
__global__ __launch_bounds__(HEAD) void gqa_merge_kernel(GqaArgs a)
{
    const int head = blockIdx.x, d = threadIdx.x;
    const int active = min(max(*a.position, 0), a.context - 1);
    const int n = active / GQA_CHUNK + 1;
    const float* src = a.workspace + static_cast<int64_t>(head) * a.chunks * (HEAD + 2);
    float M = -INFINITY;
    for (int c = 0; c < n; c++)
        M = fmaxf(M, src[static_cast<int64_t>(c) * (HEAD + 2)]);
    float L = 0.0f, O = 0.0f;
    for (int c = 0; c < n; c++) {
        const float* pc = src + static_cast<int64_t>(c) * (HEAD + 2);
        const float e = expf(pc[0] - M);
        L = fmaf(pc[1], e, L);
        O = fmaf(pc[2 + d], e, O);
    }
    a.output[static_cast<int64_t>(head) * HEAD + d] = O / L;
}

}  // namespace

hipError_t launch_rms_norm(const float* x, const float* w, float* out, int n, float eps, hipStream_t s)
{
    hipLaunchKernelGGL((rms_norm_kernel<false>), dim3(1), dim3(NORM_THREADS), 0, s, x, nullptr, w, nullptr, out, n, eps);
    return hipGetLastError();
}

hipError_t launch_residual_rms_norm(const float* hidden, const float* residual, const float* w, float* updated,
                                    float* out, int n, float eps, hipStream_t s)
{
    hipLaunchKernelGGL((rms_norm_kernel<true>), dim3(1), dim3(NORM_THREADS), 0, s, hidden, residual, w, updated, out, n,
                       eps);
    return hipGetLastError();
}

hipError_t launch_swiglu(const float* gate_up, float* out, int64_t n, hipStream_t s)
{
    hipLaunchKernelGGL(swiglu_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, gate_up, out, n);
    return hipGetLastError();
}

hipError_t launch_rope_kv_write(const RopeKvWriteArgs& a, hipStream_t s)
{
    const int total = a.query_size + 2 * a.kv_size;
    const dim3 grid(static_cast<unsigned>((total + 255) / 256));
    if (a.cache_fp16)
        hipLaunchKernelGGL((rope_kv_write_kernel<__half>), grid, dim3(256), 0, s, a, static_cast<__half*>(a.key_cache),
                           static_cast<__half*>(a.value_cache));
    else
        hipLaunchKernelGGL((rope_kv_write_kernel<float>), grid, dim3(256), 0, s, a, static_cast<float*>(a.key_cache),
                           static_cast<float*>(a.value_cache));
    return hipGetLastError();
}

int64_t gqa_workspace_floats(int query_heads, int head_size, int context)
{
    return static_cast<int64_t>(query_heads) * ((context + GQA_CHUNK - 1) / GQA_CHUNK) * (head_size + 2);
}

hipError_t launch_gqa(const GqaArgs& a, hipStream_t s)
{
    const dim3 grid(static_cast<unsigned>(a.query_heads), static_cast<unsigned>(a.chunks));
    const dim3 heads(static_cast<unsigned>(a.query_heads));
#define SI_GQA(T, H)                                                                                              \
    do {                                                                                                          \
        hipLaunchKernelGGL((gqa_partial_kernel<T, H>), grid, dim3(GQA_THREADS), 0, s, a,                         \
                           static_cast<const T*>(a.key_cache), static_cast<const T*>(a.value_cache));            \
        const hipError_t e = hipGetLastError();                                                                   \
        if (e != hipSuccess)                                                                                      \
            return e;                                                                                             \
        hipLaunchKernelGGL((gqa_merge_kernel<H>), heads, dim3(H), 0, s, a);                                       \
    } while (0)
    switch (a.head_size) {
    case 64: if (a.cache_fp16) SI_GQA(__half, 64); else SI_GQA(float, 64); break;
    case 128: if (a.cache_fp16) SI_GQA(__half, 128); else SI_GQA(float, 128); break;
    case 256: if (a.cache_fp16) SI_GQA(__half, 256); else SI_GQA(float, 256); break;
    default: return hipErrorInvalidValue;
    }
#undef SI_GQA
    return hipGetLastError();
}

}  // namespace si
