// The batched (prefill) transformer operators of the reference's D3D12
// prefill program as separate launches, with the reference's semantics and
// layouts (SharpInference.Instructions.D3D12/GpuBatchTransformerInstructions.cs).
// control = device int32[2] {start, valid}; batch row r is the token at
// position start + r and only rows r < valid are read or written.
//
//   batch-gather-rows        :646-679  out[r] = table[start + r] (rows inside the table)
//   batch-rms-norm           :101-156  per row: x * (1 / sqrt(sum(x^2) / H + eps)) * w
//   batch-residual-rms-norm  :158-222  updated = hidden + residual; out = rms-norm(updated)
//   batch-shared-matvec      :224-279  y[r] = W x[r], FP32 products and sums
//   batch-swiglu             :281-316  out[r][i] = g / (1 + exp(-g)) * u over [g | u]
//   batch-rope-kv-write      :318-413  rotate q and k of row r at position start + r,
//                                      q to `query`, k / v to that cache row
//   batch-gqa-scores         :415-470  q . k / sqrt(head) for cache rows <= start + r,
//                                      -FLT_MAX elsewhere, every context column
//   batch-causal-softmax     :472-542  softmax over columns <= start + r, 0 elsewhere
//   batch-gqa-values         :544-598  sum over columns <= start + r of p * v
//   batch-select-last        :600-625  out = in[valid - 1]
//   (scores, softmax and values fused into two launches for programs whose
//   scores and probabilities are not read afterwards: no reference operator)
//
// Caches are [context][kv_heads][head] (FP32 as in the reference, or fp16).
// The attention launches are built for 128-value heads.
#include "si_batch.hpp"
#include "si_internal.hpp"
#include "si_lanes.hpp"

#include <hip/hip_fp16.h>

#include <cfloat>

namespace si {
namespace {

constexpr int NORM_THREADS = 1024;
constexpr int THREADS = 256;

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float half_bits(uint32_t h)
{
    return __half2float(__ushort_as_half(static_cast<unsigned short>(h & 0xffffu)));
}

template <int THREADS_>
__device__ __forceinline__ float block_sum(float v, float* red)
{
    for (int off = 32; off > 0; off >>= 1)
        v += __shfl_xor(v, off);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < THREADS_ / 64; w++)
        t += red[w];
    __syncthreads();
    return t;
}

template <int THREADS_>
__device__ __forceinline__ float block_max(float v, float* red)
{
    for (int off = 32; off > 0; off >>= 1)
        v = fmaxf(v, __shfl_xor(v, off));
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = red[0];
#pragma unroll
    for (int w = 1; w < THREADS_ / 64; w++)
        t = fmaxf(t, red[w]);
    __syncthreads();
    return t;
}

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
        f[2 * k] = half_bits(w[k]);
        f[2 * k + 1] = half_bits(w[k] >> 16);
    }
}
__device__ __forceinline__ float2 load2(const float* p) { return *reinterpret_cast<const float2*>(p); }
__device__ __forceinline__ float2 load2(const __half* p)
{
    const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
    return make_float2(half_bits(w), half_bits(w >> 16));
}

template <typename T>
__device__ __forceinline__ void store_cache(T* cache, int64_t i, float v);
template <>
__device__ __forceinline__ void store_cache<float>(float* cache, int64_t i, float v) { cache[i] = v; }
template <>
__device__ __forceinline__ void store_cache<__half>(__half* cache, int64_t i, float v) { cache[i] = __float2half_rn(v); }

// ---- row-wise operators ----------------------------------------------------------------

__global__ __launch_bounds__(THREADS) void batch_gather_rows_kernel(const float* __restrict__ table,
                                                                    int64_t table_rows, int width,
                                                                    const int32_t* __restrict__ control,
                                                                    float* __restrict__ out, int64_t total)
{
    const int64_t e = static_cast<int64_t>(blockIdx.x) * THREADS + threadIdx.x;
    if (e >= total)
        return;
    const int row = static_cast<int>(e / width);
    const int64_t src = static_cast<int64_t>(control[0]) + row;
    if (row < control[1] && src >= 0 && src < table_rows)
        out[e] = table[src * width + (e - static_cast<int64_t>(row) * width)];
}

// One workgroup per live row (the decode form's operation order).  With
// PER > 0 (width <= PER * NORM_THREADS) a thread requests its PER values,
// their residuals and norm weights together and keeps them in registers
// (one memory round trip before the reduction instead of one per value and
// a re-read of the stored sum); PER = 0 is the loop form for wider rows.
// Both forms do the same operations in the same order.
template <bool RESIDUAL, int PER>
__global__ __launch_bounds__(NORM_THREADS) void batch_rms_norm_kernel(const float* __restrict__ hidden,
                                                                      const float* __restrict__ residual,
                                                                      const float* __restrict__ weight,
                                                                      float* __restrict__ updated,
                                                                      float* __restrict__ out, int width, float eps,
                                                                      const int32_t* __restrict__ control)
{
    __shared__ float red[NORM_THREADS / 64];
    const int row = blockIdx.x;
    if (row >= control[1])
        return;   // the whole workgroup, before any barrier
    const int64_t base = static_cast<int64_t>(row) * width;
    float ss = 0.0f;
    if constexpr (PER > 0) {
        float v[PER], wt[PER];
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const int j = min(static_cast<int>(threadIdx.x) + k * NORM_THREADS, width - 1);   // clamped in the row
            v[k] = hidden[base + j];
            if (RESIDUAL)
                v[k] = v[k] + residual[base + j];
            wt[k] = weight[j];
        }
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const int j = static_cast<int>(threadIdx.x) + k * NORM_THREADS;
            if (j < width) {
                if (RESIDUAL)
                    updated[base + j] = v[k];
                ss = fmaf(v[k], v[k], ss);
            }
        }
        const float total = block_sum<NORM_THREADS>(ss, red);
        const float scale = 1.0f / sqrtf(total / static_cast<float>(width) + eps);
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const int j = static_cast<int>(threadIdx.x) + k * NORM_THREADS;
            if (j < width)
                out[base + j] = v[k] * scale * wt[k];
        }
        return;
    }
    for (int j = threadIdx.x; j < width; j += NORM_THREADS) {
        float v = hidden[base + j];
        if (RESIDUAL) {
            v = v + residual[base + j];
            updated[base + j] = v;
        }
        ss = fmaf(v, v, ss);
    }
    const float total = block_sum<NORM_THREADS>(ss, red);
    const float scale = 1.0f / sqrtf(total / static_cast<float>(width) + eps);
    for (int j = threadIdx.x; j < width; j += NORM_THREADS) {
        const float v = RESIDUAL ? updated[base + j] : hidden[base + j];   // written by this thread above
        out[base + j] = v * scale * weight[j];
    }
}

__global__ __launch_bounds__(THREADS) void batch_swiglu_kernel(const float* __restrict__ gate_up,
                                                               float* __restrict__ out, int width, int64_t total,
                                                               const int32_t* __restrict__ control)
{
    const int64_t e = static_cast<int64_t>(blockIdx.x) * THREADS + threadIdx.x;
    if (e >= total)
        return;
    const int row = static_cast<int>(e / width);
    if (row >= control[1])
        return;
    const int64_t src = e + static_cast<int64_t>(row) * width;   // row * 2 * width + column
    const float g = gate_up[src];
    out[e] = g / (1.0f + expf(-g)) * gate_up[src + width];
}

// One thread per value of the batch's qkv rows.
template <typename T>
__global__ __launch_bounds__(THREADS) void batch_rope_kv_write_kernel(BatchRopeArgs a, T* __restrict__ kc,
                                                                      T* __restrict__ vc)
{
    const int width = a.query_size + 2 * a.kv_size;
    const int64_t e = static_cast<int64_t>(blockIdx.x) * THREADS + threadIdx.x;
    if (e >= static_cast<int64_t>(a.batch) * width)
        return;
    const int row = static_cast<int>(e / width);
    const int64_t position = static_cast<int64_t>(a.control[0]) + row;
    if (row >= a.control[1] || position < 0 || position >= a.context)
        return;
    const int local = static_cast<int>(e - static_cast<int64_t>(row) * width);
    const int half = a.rotary_size / 2;
    auto rotate = [&](int in_head, float value) {
        const int d = in_head % a.head_size;
        if (d >= a.rotary_size)
            return value;
        const int ri = d < half ? d : d - half;
        const int64_t pair = d < half ? e + half : e - half;
        const float angle = static_cast<float>(position) * a.frequencies[ri];
        const float c = cosf(angle) * a.rope_scale, s = sinf(angle) * a.rope_scale;
        const float other = a.qkv[pair];
        return d < half ? value * c - other * s : value * c + other * s;
    };
    const float value = a.qkv[e];
    if (local < a.query_size) {
        a.query[static_cast<int64_t>(row) * a.query_size + local] = rotate(local, value);
    } else if (local < a.query_size + a.kv_size) {
        const int c = local - a.query_size;
        store_cache<T>(kc, position * a.kv_size + c, rotate(c, value));
    } else {
        const int c = local - a.query_size - a.kv_size;
        store_cache<T>(vc, position * a.kv_size + c, value);
    }
}

// ---- attention ---------------------------------------------------------------------------

// Scores: one workgroup per (KV head, 64 cache positions).  Wave w takes
// positions j0 + 16 w + n (n < 16) as the 16 columns of its
// v_mfma_f32_16x16x4_f32 products and the live queries (query qi = row *
// group + head in group) 16 a pass as the rows.  Lane (n, c) = (l % 16,
// l / 16) holds dims 32 c .. 32 c + 31 of position n's key and of the
// pass's query n; instruction s (s < 32) takes dim 32 c + s from lane group
// c, so the 32 products add up all 128 dims of each query-key dot product
// (in another order).  D[i][n] (query 16 p + i, position n) is element i % 4
// of lane n + 16 (i / 4).  The next pass's queries are requested before the
// current pass's products.  Positions past a row's own position get
// -FLT_MAX; a chunk wholly past the batch's last position writes only those,
// with coalesced stores and no products.
template <typename T>
__global__ __launch_bounds__(THREADS) void batch_gqa_scores_kernel(BatchAttentionArgs a, const T* __restrict__ kc)
{
    const int g = blockIdx.x, chunk = blockIdx.y;
    const int group = a.query_heads / a.kv_heads;
    const int start = a.control[0], valid = min(a.control[1], a.batch);
    const int nq = max(valid, 0) * group;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int j0 = chunk * BATCH_CHUNK;
    const int64_t last = static_cast<int64_t>(start) + valid - 1;   // the batch's last position
    if (nq == 0 || last < 0 || j0 > last) {
        // every score of the chunk is masked: coalesced -FLT_MAX stores, no products
        const int jn = min(BATCH_CHUNK, a.context - j0);
        for (int i = t; i < nq * BATCH_CHUNK; i += THREADS) {
            const int qi = i / BATCH_CHUNK, jj = i % BATCH_CHUNK;
            const int r = qi / group, h = g * group + qi % group;
            if (jj < jn)
                a.out[(static_cast<int64_t>(r) * a.query_heads + h) * a.context + j0 + jj] = -FLT_MAX;
        }
        return;
    }
    const int n = lane & 15, c = lane >> 4;
    const int j = j0 + 16 * wave + n;   // this lane's key position
    float k[32];
    {
        const T* src = kc + (static_cast<int64_t>(min(j, a.context - 1)) * a.kv_heads + g) * BATCH_HEAD + 32 * c;
#pragma unroll
        for (int i = 0; i < 4; i++)
            load8(src + 8 * i, k + 8 * i);
    }
    auto load_q = [&](int p, float* q) {
        const int qi = 16 * p + n;
        if (qi < nq) {
            const int r = qi / group, h = g * group + qi % group;
            const float* src = a.query + (static_cast<int64_t>(r) * a.query_heads + h) * BATCH_HEAD + 32 * c;
#pragma unroll
            for (int i = 0; i < 4; i++)
                load8(src + 8 * i, q + 8 * i);
        } else {
#pragma unroll
            for (int i = 0; i < 32; i++)
                q[i] = 0.0f;
        }
    };
    const float scale = 1.0f / sqrtf(static_cast<float>(BATCH_HEAD));
    auto run = [&](int p, const float* q) {
        floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 32; s++)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(q[s], k[s], acc, 0, 0, 0);
        if (j >= a.context)
            return;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int qi = 16 * p + 4 * c + e;
            if (qi < nq) {
                const int r = qi / group, h = g * group + qi % group;
                const int64_t active = static_cast<int64_t>(start) + r;
                a.out[(static_cast<int64_t>(r) * a.query_heads + h) * a.context + j] =
                    active >= 0 && j <= active ? acc[e] * scale : -FLT_MAX;
            }
        }
    };
    const int passes = (nq + 15) / 16;
    float q0[32], q1[32];
    load_q(0, q0);
    for (int p = 0; p < passes; p += 2) {
        if (p + 1 < passes)
            load_q(p + 1, q1);
        run(p, q0);
        if (p + 2 < passes)
            load_q(p + 2, q0);
        if (p + 1 < passes)
            run(p + 1, q1);
    }
}

// One workgroup per (live row, query head).  Up to SOFTMAX_HELD positions a
// thread (context up to THREADS * SOFTMAX_HELD) the scores are read once and
// held in registers for the max, the sum and the write; longer rows read
// them three times.
constexpr int SOFTMAX_HELD = 16;

__global__ __launch_bounds__(THREADS) void batch_causal_softmax_kernel(const float* __restrict__ scores,
                                                                       float* __restrict__ probs, int heads,
                                                                       int context,
                                                                       const int32_t* __restrict__ control)
{
    __shared__ float red[THREADS / 64];
    const int r = blockIdx.x / heads, h = blockIdx.x % heads;
    if (r >= control[1])
        return;   // the whole workgroup
    const int64_t active = static_cast<int64_t>(control[0]) + r;
    const int last = active < 0 ? -1 : static_cast<int>(min(active, static_cast<int64_t>(context) - 1));
    const int64_t base = (static_cast<int64_t>(r) * heads + h) * context;
    const int t = threadIdx.x;
    if (last < THREADS * SOFTMAX_HELD) {
        float v[SOFTMAX_HELD];
        float m = -FLT_MAX;
#pragma unroll
        for (int i = 0; i < SOFTMAX_HELD; i++) {
            const int j = t + THREADS * i;
            v[i] = j <= last ? scores[base + j] : -FLT_MAX;
            m = fmaxf(m, v[i]);
        }
        m = block_max<THREADS>(m, red);
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < SOFTMAX_HELD; i++) {
            const int j = t + THREADS * i;
            v[i] = j <= last ? expf(v[i] - m) : 0.0f;
            sum += v[i];
        }
        sum = block_sum<THREADS>(sum, red);
#pragma unroll
        for (int i = 0; i < SOFTMAX_HELD; i++) {
            const int j = t + THREADS * i;
            if (j < context)
                probs[base + j] = j <= last ? v[i] / sum : 0.0f;
        }
        for (int j = t + THREADS * SOFTMAX_HELD; j < context; j += THREADS)
            probs[base + j] = 0.0f;
        return;
    }
    float m = -FLT_MAX;
    for (int j = t; j <= last; j += THREADS)
        m = fmaxf(m, scores[base + j]);
    m = block_max<THREADS>(m, red);
    float sum = 0.0f;
    for (int j = t; j <= last; j += THREADS)
        sum += expf(scores[base + j] - m);
    sum = block_sum<THREADS>(sum, red);
    for (int j = t; j < context; j += THREADS)
        probs[base + j] = j <= last ? expf(scores[base + j] - m) / sum : 0.0f;
}

// Values, first pass: one workgroup per (KV head, 64 cache positions).  Wave
// w takes channels 32 w .. 32 w + 31 as two 16-column tiles of its
// v_mfma_f32_16x16x4_f32 products, column n of tile u being channel 32 w +
// 2 n + u (one channel pair per lane and position), and the live queries 16
// a pass as the rows.  Instruction s (s < 16) takes position j0 + 16 c + s
// from lane group c = l / 16, so a lane's probabilities are 16 consecutive
// floats of its query's row.  Positions past the batch's last position (or
// the context) take probability 0 and value 0, whatever the cache holds
// there.  Partial sums go to the workspace [chunk][row][head][128]; the
// second pass adds the chunks up to each row's own position in order.
template <typename T>
__global__ __launch_bounds__(THREADS) void batch_gqa_values_partial_kernel(BatchAttentionArgs a,
                                                                           const T* __restrict__ vc)
{
    const int g = blockIdx.x, chunk = blockIdx.y;
    const int group = a.query_heads / a.kv_heads;
    const int start = a.control[0], valid = min(a.control[1], a.batch);
    const int nq = max(valid, 0) * group;
    const int64_t last = static_cast<int64_t>(start) + valid - 1;
    const int j0 = chunk * BATCH_CHUNK;
    if (nq == 0 || last < 0 || j0 > last)
        return;   // the whole workgroup: no live position in this chunk
    const int jl = static_cast<int>(min(last, static_cast<int64_t>(a.context) - 1));   // last position read
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = lane & 15, c = lane >> 4;
    const int jc = j0 + 16 * c;   // the lane group's first position
    float2 v[16];
    {
        const T* src = vc + static_cast<int64_t>(g) * BATCH_HEAD + 32 * wave + 2 * n;
        const int64_t stride = static_cast<int64_t>(a.kv_heads) * BATCH_HEAD;
#pragma unroll
        for (int s = 0; s < 16; s++) {
            const float2 f = load2(src + min(jc + s, jl) * stride);   // rows past jl: read jl's, use 0
            v[s] = jc + s <= jl ? f : make_float2(0.0f, 0.0f);
        }
    }
    const bool whole = jc + 15 <= jl && (a.context & 3) == 0 &&
                       (reinterpret_cast<uintptr_t>(a.probabilities) & 15) == 0;
    auto load_p = [&](int p, float* pr) {
        const int qi = 16 * p + n;
        if (qi < nq) {
            const int r = qi / group, h = g * group + qi % group;
            const float* src = a.probabilities + (static_cast<int64_t>(r) * a.query_heads + h) * a.context + jc;
            if (whole) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 f = reinterpret_cast<const float4*>(src)[i];
                    pr[4 * i] = f.x; pr[4 * i + 1] = f.y; pr[4 * i + 2] = f.z; pr[4 * i + 3] = f.w;
                }
            } else {
#pragma unroll
                for (int s = 0; s < 16; s++) {
                    const float f = src[max(min(s, jl - jc), j0 - jc)];   // inside the row
                    pr[s] = jc + s <= jl ? f : 0.0f;
                }
            }
        } else {
#pragma unroll
            for (int s = 0; s < 16; s++)
                pr[s] = 0.0f;
        }
    };
    auto run = [&](int p, const float* pr) {
        floatx4 lo = {0.0f, 0.0f, 0.0f, 0.0f}, hi = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 16; s++) {
            lo = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[s], v[s].x, lo, 0, 0, 0);
            hi = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[s], v[s].y, hi, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int qi = 16 * p + 4 * c + e;
            if (qi < nq) {
                const int r = qi / group, h = g * group + qi % group;
                float* dst = a.workspace + ((static_cast<int64_t>(chunk) * a.batch + r) * a.query_heads + h) *
                                               BATCH_HEAD + 32 * wave + 2 * n;
                *reinterpret_cast<float2*>(dst) = make_float2(lo[e], hi[e]);
            }
        }
    };
    const int passes = (nq + 15) / 16;
    float p0[16], p1[16];
    load_p(0, p0);
    for (int p = 0; p < passes; p += 2) {
        if (p + 1 < passes)
            load_p(p + 1, p1);
        run(p, p0);
        if (p + 2 < passes)
            load_p(p + 2, p0);
        if (p + 1 < passes)
            run(p + 1, p1);
    }
}

// Values, second pass: one workgroup per (live row, query head); the chunk
// partials are requested VALUES_BATCH at a time and added in chunk order.
constexpr int VALUES_BATCH = 8;

__global__ __launch_bounds__(BATCH_HEAD) void batch_gqa_values_reduce_kernel(BatchAttentionArgs a)
{
    const int r = blockIdx.x / a.query_heads, h = blockIdx.x % a.query_heads;
    if (r >= min(a.control[1], a.batch))
        return;
    const int64_t active = static_cast<int64_t>(a.control[0]) + r;
    float sum = 0.0f;
    if (active >= 0) {
        const int n = static_cast<int>(min(active, static_cast<int64_t>(a.context) - 1) / BATCH_CHUNK) + 1;
        const float* src = a.workspace + (static_cast<int64_t>(r) * a.query_heads + h) * BATCH_HEAD + threadIdx.x;
        const int64_t cstride = static_cast<int64_t>(a.batch) * a.query_heads * BATCH_HEAD;
        for (int c0 = 0; c0 < n; c0 += VALUES_BATCH) {
            float part[VALUES_BATCH];
#pragma unroll
            for (int i = 0; i < VALUES_BATCH; i++)
                part[i] = c0 + i < n ? src[(c0 + i) * cstride] : 0.0f;
#pragma unroll
            for (int i = 0; i < VALUES_BATCH; i++)
                sum += part[i];
        }
    }
    a.out[(static_cast<int64_t>(r) * a.query_heads + h) * BATCH_HEAD + threadIdx.x] = sum;
}

// ---- scores, causal softmax and values in two launches ------------------------------------
//
// First pass: one workgroup per (KV head, 64 positions) holding a live
// position.  The group's scores of the chunk come from the matrix cores as
// in batch_gqa_scores_kernel (positions past a row's own position, or past
// the batch's last one, -inf) into an LDS tile; one wave per query turns its
// row of the tile into exp(s - m), m the row's largest score in the chunk, and
// l, their sum; the tile times the chunk's V rows (requested before the
// scores) as in batch_gqa_values_partial_kernel goes to the workspace with
// (m, l).  Second pass: per (row, head), the chunks up to the row's own
// position merge as sum_c exp(m_c - M) acc_c / sum_c exp(m_c - M) l_c, M the
// largest m_c: the causal softmax's weighted sum, rounded in another order.
// A row with no position of the chunk at or before its own gets m = -inf,
// l = 0, and a zero row of P; the merge never reads such a chunk for it.
constexpr int FLASH_PITCH = BATCH_CHUNK + 4;   // floats per query row of the tile (rows 4 banks apart)

template <typename T>
__global__ __launch_bounds__(THREADS) void batch_gqa_flash_partial_kernel(BatchAttentionArgs a,
                                                                          const T* __restrict__ kc,
                                                                          const T* __restrict__ vc)
{
    __shared__ __align__(16) float tile[BATCH_MAX * BATCH_GROUP_MAX * FLASH_PITCH];
    const int g = blockIdx.x, chunk = blockIdx.y;
    const int group = a.query_heads / a.kv_heads;
    const int start = a.control[0], valid = min(a.control[1], a.batch);
    const int nq = max(valid, 0) * group;
    const int64_t last = static_cast<int64_t>(start) + valid - 1;
    const int j0 = chunk * BATCH_CHUNK;
    if (nq == 0 || last < 0 || j0 > last)
        return;   // the whole workgroup: no live position in this chunk
    const int jl = static_cast<int>(min(last, static_cast<int64_t>(a.context) - 1));   // last position read
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 15, c = lane >> 4;
    const int64_t entries = static_cast<int64_t>(a.batch) * a.query_heads;
    const int64_t chunks = (a.context + BATCH_CHUNK - 1) / BATCH_CHUNK;
    // V rows: positions jc + s (s < 16) of lane group c, channels 32 wave + 2n and + 1
    const int jc = j0 + 16 * c;
    float2 v[16];
    {
        const T* src = vc + static_cast<int64_t>(g) * BATCH_HEAD + 32 * wave + 2 * n;
        const int64_t stride = static_cast<int64_t>(a.kv_heads) * BATCH_HEAD;
#pragma unroll
        for (int s = 0; s < 16; s++) {
            const float2 f = load2(src + min(jc + s, jl) * stride);   // rows past jl: read jl's, use 0
            v[s] = jc + s <= jl ? f : make_float2(0.0f, 0.0f);
        }
    }
    // keys: position j of this lane, dims 32c .. 32c + 31
    const int j = j0 + 16 * wave + n;
    float k[32];
    {
        const T* src = kc + (static_cast<int64_t>(min(j, jl)) * a.kv_heads + g) * BATCH_HEAD + 32 * c;
#pragma unroll
        for (int i = 0; i < 4; i++)
            load8(src + 8 * i, k + 8 * i);
    }
    auto load_q = [&](int p, float* q) {
        const int qi = 16 * p + n;
        if (qi < nq) {
            const int r = qi / group, h = g * group + qi % group;
            const float* src = a.query + (static_cast<int64_t>(r) * a.query_heads + h) * BATCH_HEAD + 32 * c;
#pragma unroll
            for (int i = 0; i < 4; i++)
                load8(src + 8 * i, q + 8 * i);
        } else {
#pragma unroll
            for (int i = 0; i < 32; i++)
                q[i] = 0.0f;
        }
    };
    const float scale = 1.0f / sqrtf(static_cast<float>(BATCH_HEAD));
    auto score_pass = [&](int p, const float* q) {
        floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};   // two product chains
#pragma unroll
        for (int s = 0; s < 32; s += 2) {
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(q[s], k[s], acc, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(q[s + 1], k[s + 1], acc1, 0, 0, 0);
        }
        acc += acc1;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int qi = 16 * p + 4 * c + e;
            if (qi < nq) {
                const int64_t active = static_cast<int64_t>(start) + qi / group;
                tile[qi * FLASH_PITCH + 16 * wave + n] = j <= jl && j <= active ? acc[e] * scale : -INFINITY;
            }
        }
    };
    const int passes = (nq + 15) / 16;
    {
        float q0[32], q1[32];
        load_q(0, q0);
        for (int p = 0; p < passes; p += 2) {
            if (p + 1 < passes)
                load_q(p + 1, q1);
            score_pass(p, q0);
            if (p + 2 < passes)
                load_q(p + 2, q0);
            if (p + 1 < passes)
                score_pass(p + 1, q1);
        }
    }
    __syncthreads();
    float* ml = a.workspace + chunks * entries * BATCH_HEAD;   // (m, l) per [chunk][row][head]
    // four queries a wave at a time (queries wave, wave + 4, ... ), their
    // reductions interleaved
    constexpr int SQ = 4;
    for (int q0 = wave; q0 < nq; q0 += SQ * (THREADS / 64)) {
        float sc[SQ], m[SQ], e[SQ], l[SQ];
#pragma unroll
        for (int u = 0; u < SQ; u++) {
            const int qi = q0 + u * (THREADS / 64);
            sc[u] = qi < nq ? tile[qi * FLASH_PITCH + lane] : -INFINITY;
            m[u] = sc[u];
        }
#pragma unroll
        for (int u = 0; u < SQ; u++)
            m[u] = rows_max(row_max<16>(m[u]));   // DPP within rows of 16, then across the 4 rows
#pragma unroll
        for (int u = 0; u < SQ; u++) {
            e[u] = m[u] == -INFINITY ? 0.0f : expf(sc[u] - m[u]);
            l[u] = e[u];
        }
#pragma unroll
        for (int u = 0; u < SQ; u++)
            l[u] = rows_sum(row_sum<16>(l[u]));
#pragma unroll
        for (int u = 0; u < SQ; u++) {
            const int qi = q0 + u * (THREADS / 64);
            if (qi < nq) {
                tile[qi * FLASH_PITCH + lane] = e[u];
                if (lane == 0) {
                    const int r = qi / group, h = g * group + qi % group;
                    float* dst = ml + ((static_cast<int64_t>(chunk) * a.batch + r) * a.query_heads + h) * 2;
                    dst[0] = m[u];
                    dst[1] = l[u];
                }
            }
        }
    }
    __syncthreads();
    auto load_p = [&](int p, float* pr) {
        const int qi = 16 * p + n;
        if (qi < nq) {
            const float4* src = reinterpret_cast<const float4*>(tile + qi * FLASH_PITCH + 16 * c);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 f = src[i];
                pr[4 * i] = f.x; pr[4 * i + 1] = f.y; pr[4 * i + 2] = f.z; pr[4 * i + 3] = f.w;
            }
        } else {
#pragma unroll
            for (int s = 0; s < 16; s++)
                pr[s] = 0.0f;
        }
    };
    for (int p = 0; p < passes; p++) {
        float pr[16];
        load_p(p, pr);
        floatx4 lo = {0.0f, 0.0f, 0.0f, 0.0f}, hi = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < 16; s++) {
            lo = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[s], v[s].x, lo, 0, 0, 0);
            hi = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[s], v[s].y, hi, 0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int qi = 16 * p + 4 * c + e;
            if (qi < nq) {
                const int r = qi / group, h = g * group + qi % group;
                float* dst = a.workspace + ((static_cast<int64_t>(chunk) * a.batch + r) * a.query_heads + h) *
                                               BATCH_HEAD + 32 * wave + 2 * n;
                *reinterpret_cast<float2*>(dst) = make_float2(lo[e], hi[e]);
            }
        }
    }
}

// Second pass: one workgroup per (live row, query head), a thread per
// channel.  The chunks' (m, l) are read at once (thread t takes chunks t and
// t + 128: a context of at most 16384 positions has 256 chunks), the weights
// exp(m_c - M) go through LDS, and the partial sums are requested
// VALUES_BATCH chunks at a time.
constexpr int FLASH_MAX_CHUNKS = 2 * BATCH_HEAD;

__global__ __launch_bounds__(BATCH_HEAD) void batch_gqa_flash_merge_kernel(BatchAttentionArgs a)
{
    __shared__ float weight[FLASH_MAX_CHUNKS];
    __shared__ float red[BATCH_HEAD / 64];
    const int r = blockIdx.x / a.query_heads, h = blockIdx.x % a.query_heads;
    if (r >= min(a.control[1], a.batch))
        return;
    const int64_t active = static_cast<int64_t>(a.control[0]) + r;
    const int64_t o = (static_cast<int64_t>(r) * a.query_heads + h) * BATCH_HEAD + threadIdx.x;
    if (active < 0) {   // the whole workgroup
        a.out[o] = 0.0f;
        return;
    }
    const int t = threadIdx.x;
    const int nch = static_cast<int>(min(active, static_cast<int64_t>(a.context) - 1) / BATCH_CHUNK) + 1;
    const int64_t entries = static_cast<int64_t>(a.batch) * a.query_heads;
    const int64_t chunks = (a.context + BATCH_CHUNK - 1) / BATCH_CHUNK;
    const int64_t e0 = static_cast<int64_t>(r) * a.query_heads + h;
    const float* ml = a.workspace + chunks * entries * BATCH_HEAD + 2 * e0;
    float m[2], l[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int c = t + BATCH_HEAD * i;
        const float2 f = c < nch ? *reinterpret_cast<const float2*>(ml + c * 2 * entries) : make_float2(-INFINITY, 0.0f);
        m[i] = f.x;
        l[i] = f.y;
    }
    const float M = block_max<BATCH_HEAD>(fmaxf(m[0], m[1]), red);   // finite: chunk 0 holds position 0
    float lsum = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int c = t + BATCH_HEAD * i;
        if (c < nch) {
            const float w = m[i] == -INFINITY ? 0.0f : expf(m[i] - M);
            weight[c] = w;
            lsum += w * l[i];
        }
    }
    const float L = block_sum<BATCH_HEAD>(lsum, red);   // its barriers publish the weights
    const float* part = a.workspace + e0 * BATCH_HEAD + t;
    float acc = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += VALUES_BATCH) {
        float pv[VALUES_BATCH];
#pragma unroll
        for (int i = 0; i < VALUES_BATCH; i++)
            pv[i] = part[static_cast<int64_t>(min(c0 + i, nch - 1)) * entries * BATCH_HEAD];
#pragma unroll
        for (int i = 0; i < VALUES_BATCH; i++)
            if (c0 + i < nch)
                acc += weight[c0 + i] * pv[i];
    }
    a.out[o] = acc / L;
}

__global__ __launch_bounds__(THREADS) void batch_select_last_kernel(const float* __restrict__ input,
                                                                    float* __restrict__ out, int batch, int width,
                                                                    const int32_t* __restrict__ control)
{
    const int c = static_cast<int>(blockIdx.x) * THREADS + threadIdx.x;
    const int valid = control[1];
    if (c < width && valid > 0 && valid <= batch)
        out[c] = input[static_cast<int64_t>(valid - 1) * width + c];
}

// ---- batched matrix-vector product on the FP32 matrix cores ------------------------------


typedef uint32_t u32_a2 __attribute__((aligned(2)));   // 4 bytes at a 2-byte aligned address

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }
__device__ __forceinline__ uint32_t ld_u32_a2(const uint8_t* p) { return *reinterpret_cast<const u32_a2*>(p); }

// Raw words of elements 8g .. 8g + 7 of one 32-column block of a row (plain
// word loads; every bit extraction happens in decode8, so a pass can issue
// the loads of all its blocks before it decodes the first):
//   F32: 8 floats; F16: 8 halves (4 words); Q8_0 {fp16 d; int8 q[32]}: d and
//   q[8g..8g+7]; Q4_0 {fp16 d; u8 qs[16]}: d and qs[8 (g % 2) ..] (elements
//   0..15 are the low nibbles, 16..31 the high ones); Q4_K: the super-block's
//   16-byte header (d, dmin, 12 scale bytes) and the 8 quant bytes of the
//   sub-block's chunk.
template <int FMT>
struct Raw8 {
    uint32_t w[FMT == FMT_F32 ? 8 : FMT == FMT_Q4_K ? 6 : 4];
};

template <int FMT>
__device__ __forceinline__ Raw8<FMT> load_raw8(const uint8_t* row, int blk, int g)
{
    Raw8<FMT> r;
    if constexpr (FMT == FMT_F32) {
        const uint4* p = reinterpret_cast<const uint4*>(row + 128 * static_cast<int64_t>(blk) + 32 * g);
        const uint4 a = p[0], b = p[1];
        r.w[0] = a.x; r.w[1] = a.y; r.w[2] = a.z; r.w[3] = a.w;
        r.w[4] = b.x; r.w[5] = b.y; r.w[6] = b.z; r.w[7] = b.w;
    } else if constexpr (FMT == FMT_F16) {
        const uint4 a = *reinterpret_cast<const uint4*>(row + 64 * static_cast<int64_t>(blk) + 16 * g);
        r.w[0] = a.x; r.w[1] = a.y; r.w[2] = a.z; r.w[3] = a.w;
    } else if constexpr (FMT == FMT_Q8_0) {
        const uint8_t* b = row + 34 * static_cast<int64_t>(blk);
        r.w[0] = ld_u16(b);
        r.w[1] = ld_u32_a2(b + 2 + 8 * g);
        r.w[2] = ld_u32_a2(b + 6 + 8 * g);
    } else if constexpr (FMT == FMT_Q4_0) {
        const uint8_t* b = row + 18 * static_cast<int64_t>(blk);
        r.w[0] = ld_u16(b);
        r.w[1] = ld_u32_a2(b + 2 + 8 * (g & 1));
        r.w[2] = ld_u32_a2(b + 6 + 8 * (g & 1));
    } else {
        const uint8_t* sb = row + 144 * static_cast<int64_t>(blk >> 3);
        const uint4 h = *reinterpret_cast<const uint4*>(sb);
        const uint2 q = *reinterpret_cast<const uint2*>(sb + 16 + 32 * ((blk & 7) >> 1) + 8 * g);
        r.w[0] = h.x; r.w[1] = h.y; r.w[2] = h.z; r.w[3] = h.w;
        r.w[4] = q.x; r.w[5] = q.y;
    }
    return r;
}

// The 8 values dequantised as the CpuVm decode does (one rounding per
// operation).
template <int FMT>
__device__ __forceinline__ void decode8(const Raw8<FMT>& r, int blk, int g, float* w)
{
    if constexpr (FMT == FMT_F32) {
#pragma unroll
        for (int i = 0; i < 8; i++)
            w[i] = __uint_as_float(r.w[i]);
    } else if constexpr (FMT == FMT_F16) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            w[2 * k] = half_bits(r.w[k]);
            w[2 * k + 1] = half_bits(r.w[k] >> 16);
        }
    } else if constexpr (FMT == FMT_Q8_0) {
        const float d = half_bits(r.w[0]);
#pragma unroll
        for (int i = 0; i < 8; i++)
            w[i] = d * static_cast<float>(static_cast<int8_t>((r.w[1 + i / 4] >> (8 * (i & 3))) & 0xffu));
    } else if constexpr (FMT == FMT_Q4_0) {
        const float d = half_bits(r.w[0]);
        const int sh = g < 2 ? 0 : 4;   // elements 0..15: low nibbles, 16..31: high nibbles
#pragma unroll
        for (int i = 0; i < 8; i++)
            w[i] = d * static_cast<float>(static_cast<int>((r.w[1 + i / 4] >> (8 * (i & 3) + sh)) & 15u) - 8);
    } else {
        const int j = blk & 7;   // sub-block: chunk j / 2, low nibbles for even j
        auto sbyte = [&](int i) { return static_cast<int>((r.w[1 + (i >> 2)] >> (8 * (i & 3))) & 0xffu); };
        int sc, m;
        if (j < 4) {
            sc = sbyte(j) & 63;
            m = sbyte(j + 4) & 63;
        } else {
            sc = (sbyte(j + 4) & 15) | ((sbyte(j - 4) >> 6) << 4);
            m = (sbyte(j + 4) >> 4) | ((sbyte(j) >> 6) << 4);
        }
        const float d1 = __fmul_rn(half_bits(r.w[0]), static_cast<float>(sc));
        const float m1 = __fmul_rn(half_bits(r.w[0] >> 16), static_cast<float>(m));
        const int sh = (j & 1) * 4;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float n = static_cast<float>((r.w[4 + i / 4] >> (8 * (i & 3) + sh)) & 15u);
            w[i] = __fsub_rn(__fmul_rn(d1, n), m1);
        }
    }
}

constexpr int MV_PASS = 2;   // blocks per wave and pass

// One workgroup = 16 output rows x 16 batch rows, its four waves splitting
// the 32-column blocks (wave w takes blocks w, w + 4, ...) and adding their
// 16 x 16 tiles through LDS in a fixed order.  Per block, lane (r, g) = (l %
// 16, l / 16) dequantises elements 8g..8g+7 of row o0 + r and loads the same
// columns of batch row t0 + r; eight v_mfma_f32_16x16x4_f32 take k = 8g + s
// (s < 8) from lane group g: the sum over k is the row's dot product in any
// order.  D[i][j] of the tile (batch row t0 + i, output row o0 + j) is held
// by lane j + 16 (i / 4), element i % 4.  A wave works in passes of MV_PASS
// blocks over two register sets: the W words and X values of the next pass
// are requested before the current one is decoded (block indexes past the
// row are clamped and their products skipped), so each pass's round trip
// overlaps the previous pass's products; a grid holds only one to four
// workgroups per CU, too few waves to hide the round trips otherwise (one
// set of eight blocks per pass, not overlapped: 112.7 against 97.8 us for
// the Phi-4 layer's four Q4_K products at 16 rows).
template <int FMT>
__global__ __launch_bounds__(THREADS) void batch_matvec_kernel(const uint8_t* __restrict__ W,
                                                               const float* __restrict__ X, float* __restrict__ Y,
                                                               int batch, int rows, int cols, int64_t row_bytes,
                                                               const int32_t* __restrict__ control)
{
    __shared__ floatx4 red[4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int o0 = static_cast<int>(blockIdx.x) * 16, t0 = static_cast<int>(blockIdx.y) * 16;
    const int live = min(control[1], batch) - t0;   // live batch rows of this tile
    if (live <= 0)
        return;   // the whole workgroup, before the barrier
    const uint8_t* wrow = W + static_cast<int64_t>(min(o0 + r, rows - 1)) * row_bytes;
    const bool tok = r < live;
    const float* xrow = X + static_cast<int64_t>(t0 + (tok ? r : 0)) * cols + 8 * g;
    const int nb = cols / 32;
    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    Raw8<FMT> raw[2][MV_PASS];
    float x[2][MV_PASS][8];
    auto load_pass = [&](int b0, int set) {
#pragma unroll
        for (int u = 0; u < MV_PASS; u++) {
            const int b = min(b0 + 4 * u, nb - 1);
            raw[set][u] = load_raw8<FMT>(wrow, b, g);
            load8(xrow + 32 * b, x[set][u]);
        }
    };
    auto run_pass = [&](int b0, int set) {
#pragma unroll
        for (int u = 0; u < MV_PASS; u++) {
            const int b = b0 + 4 * u;
            if (b < nb) {   // uniform across the wave
                float w[8];
                decode8<FMT>(raw[set][u], b, g, w);
#pragma unroll
                for (int s = 0; s < 8; s++)
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(tok ? x[set][u][s] : 0.0f, w[s], acc, 0, 0, 0);
            }
        }
    };
    constexpr int STEP = 4 * MV_PASS;   // blocks of one pass of the workgroup
    int b0 = wave;
    load_pass(b0, 0);
    for (; b0 + STEP < nb; b0 += 2 * STEP) {
        load_pass(b0 + STEP, 1);
        run_pass(b0, 0);
        if (b0 + 2 * STEP < nb)
            load_pass(b0 + 2 * STEP, 0);
        run_pass(b0 + STEP, 1);
    }
    if (b0 < nb)   // set 0 holds this pass (loaded when b0 < nb)
        run_pass(b0, 0);
    red[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
        const floatx4 v = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
        const int o = o0 + r;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int i = 4 * g + m;
            if (i < live && o < rows)
                Y[static_cast<int64_t>(t0 + i) * rows + o] = v[m];
        }
    }
}


// ---- the same product over per-wave LDS rings filled by asynchronous loads ----------------
//
// For Q4_0, Q8_0 and Q4_K with columns % 256 == 0.  A workgroup of WAVES
// (8, or 16 for grids that leave CUs without a second workgroup) owns 16
// output rows x 16 batch rows; wave w multiplies the 32-column blocks w,
// w + WAVES, w + 2 WAVES, ... (for Q4_K always sub-block w % 8 of a
// super-block) and copies exactly the bytes it
// multiplies into a ring of its own in LDS with global_load_lds_dwordx4: each
// lane's 16 bytes land at the instruction's LDS base + 16 x lane, no VGPR is
// held while a copy is in flight, and RING - 1 blocks are requested ahead of
// the one being multiplied.  A wave waits only for its own copies (s_waitcnt
// vmcnt), so the loop has no barrier and the waves of a CU drift freely,
// overlapping one's decode with another's matrix products.  Against X and W
// fragments loaded into registers one pass ahead, the Phi-4 layer's four
// Q4_K products at 16 rows take 74 instead of 102 us (Q4_0: 68 against 116);
// a ring shared by the workgroup, with a barrier per 256 columns, took 84.
//
// One stage per block: X of the 16 batch rows (2 copies of 1 KB; copy h,
// lane i holds row 8h + i/8, 16-byte piece (i % 8) ^ ((row >> 1) & 7) of the
// block, so a read of piece p by the 16 rows hits 16 distinct 4-bank groups)
// and the 16 weight rows' bytes of the block (one copy, three 16-byte pieces
// a row, 48 bytes apart: Q4_K the super-block header and the 32 quant bytes
// of the sub-block pair; Q4_0 / Q8_0 the aligned 32 / 48 bytes around the
// 18- / 34-byte block, which never pass the end of its 8-block group, a
// multiple of 16 bytes).  Lane (r, g) = (l % 16, l / 16) multiplies columns
// 4g..4g+3 and 16+4g..16+4g+3 of the block: eight v_mfma_f32_16x16x4_f32 on
// two accumulators (even and odd instructions), added at the end.
constexpr int RING_WAVES = 8;                  // waves of the default workgroup
constexpr int RING_XBYTES = 16 * 32 * 4;        // X bytes of a stage
constexpr int RING_WPITCH = 48;                 // bytes per weight row of a stage
constexpr int RING_STAGE = RING_XBYTES + 16 * RING_WPITCH;
constexpr int RING_COPIES = 3;                  // copy instructions per stage

__device__ __forceinline__ uint32_t lds_u16(const uint8_t* p) { return *reinterpret_cast<const uint16_t*>(p); }
__device__ __forceinline__ uint32_t lds_u32(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }

// One asynchronous 16-byte copy per lane from global memory into LDS at
// lds_base + 16 x lane.  The wave-uniform LDS base goes in M0 (the compiler
// writes it there as the operand's register); the s_nop is the wait state an
// LDS-bound load needs after an M0 write.
__device__ __forceinline__ void copy16_to_lds(const void* src, uint32_t lds_base)
{
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds_base) : "memory");
}

// Waits until at most N of this wave's memory loads (copies included) are in
// flight.
template <int N>
__device__ __forceinline__ void wait_copies()
{
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Source of weight piece j (0..2) of block b in a row: Q4_K the header (j =
// 0) and the quant bytes of the sub-block pair; Q4_0 the 16-byte aligned 32
// bytes holding the block (piece 2 repeats piece 1); Q8_0 the aligned 48.
template <int FMT>
__device__ __forceinline__ int64_t ring_piece(int b, int j)
{
    if constexpr (FMT == FMT_Q4_K)
        return 144 * static_cast<int64_t>(b >> 3) + (j == 0 ? 0 : 16 + 32 * ((b & 7) >> 1) + 16 * (j - 1));
    else if constexpr (FMT == FMT_Q4_0)
        return ((18 * static_cast<int64_t>(b)) & ~int64_t{15}) + 16 * min(j, 1);
    else
        return ((34 * static_cast<int64_t>(b)) & ~int64_t{15}) + 16 * j;
}

// The four bytes of a word as floats, one v_cvt_f32_ubyteN each (written
// out: the compiler folds a preceding nibble mask into per-byte bit-field
// extracts otherwise).
__device__ __forceinline__ void bytes_to_float(uint32_t v, float* f)
{
    asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f[0]) : "v"(v));
    asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f[1]) : "v"(v));
    asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f[2]) : "v"(v));
    asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f[3]) : "v"(v));
}

// The 8 weights of block b at columns 4g..4g+3 and 16+4g..16+4g+3 from its
// staged row pieces, dequantised as decode8 does.
template <int FMT>
__device__ __forceinline__ void decode_staged(const uint8_t* row, int b, int g, float* w)
{
    if constexpr (FMT == FMT_Q8_0) {
        const uint8_t* blk = row + ((34 * b) & 15);
        const float d = half_bits(lds_u16(blk));
        const uint32_t lo = lds_u16(blk + 2 + 4 * g) | (lds_u16(blk + 4 + 4 * g) << 16);
        const uint32_t hi = lds_u16(blk + 18 + 4 * g) | (lds_u16(blk + 20 + 4 * g) << 16);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            w[e] = d * static_cast<float>(static_cast<int8_t>((lo >> (8 * e)) & 0xffu));
            w[4 + e] = d * static_cast<float>(static_cast<int8_t>((hi >> (8 * e)) & 0xffu));
        }
    } else if constexpr (FMT == FMT_Q4_0) {
        const uint8_t* blk = row + ((18 * b) & 15);
        const float d = half_bits(lds_u16(blk));
        const uint32_t q = lds_u16(blk + 2 + 4 * g) | (lds_u16(blk + 4 + 4 * g) << 16);   // qs[4g..4g+3]
        float nl[4], nh[4];
        bytes_to_float(q & 0x0F0F0F0Fu, nl);          // one nibble per byte
        bytes_to_float((q >> 4) & 0x0F0F0F0Fu, nh);
#pragma unroll
        for (int e = 0; e < 4; e++) {   // n - 8 and d (n - 8) are exact in FP32
            w[e] = d * (nl[e] - 8.0f);       // element 4g+e
            w[4 + e] = d * (nh[e] - 8.0f);   // element 16+4g+e
        }
    } else {   // Q4_K sub-block j of the super-block (j is the same for the whole wave)
        const int j = b & 7;
        const uint4 h = *reinterpret_cast<const uint4*>(row);   // d, dmin; 12 scale bytes
        const int sh8 = 8 * (j & 3);                              // byte j % 4 of a scale word
        int sc, m;
        if (j < 4) {
            sc = static_cast<int>(__builtin_amdgcn_ubfe(h.y, sh8, 6));
            m = static_cast<int>(__builtin_amdgcn_ubfe(h.z, sh8, 6));
        } else {
            const int both = static_cast<int>(__builtin_amdgcn_ubfe(h.w, sh8, 8));
            sc = (both & 15) | (static_cast<int>(__builtin_amdgcn_ubfe(h.y, sh8 + 6, 2)) << 4);
            m = (both >> 4) | (static_cast<int>(__builtin_amdgcn_ubfe(h.z, sh8 + 6, 2)) << 4);
        }
        const float d1 = __fmul_rn(half_bits(h.x), static_cast<float>(sc));
        const float m1 = __fmul_rn(half_bits(h.x >> 16), static_cast<float>(m));
        const int sh = (j & 1) * 4;   // low nibbles for even sub-blocks
        const uint32_t lo = (lds_u32(row + 16 + 4 * g) >> sh) & 0x0F0F0F0Fu;   // one nibble per byte
        const uint32_t hi = (lds_u32(row + 32 + 4 * g) >> sh) & 0x0F0F0F0Fu;
        float nl[4], nh[4];
        bytes_to_float(lo, nl);
        bytes_to_float(hi, nh);
#pragma unroll
        for (int e = 0; e < 4; e++) {
            w[e] = __fsub_rn(__fmul_rn(d1, nl[e]), m1);
            w[4 + e] = __fsub_rn(__fmul_rn(d1, nh[e]), m1);
        }
    }
}

template <int FMT, int RING, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void batch_matvec_ring_kernel(
    const uint8_t* __restrict__ W, const float* __restrict__ X, float* __restrict__ Y, int batch, int rows, int cols,
    int64_t row_bytes, const int32_t* __restrict__ control)
{
    constexpr int WAVE_RING = RING * RING_STAGE;
    static_assert(RING >= 2 && (RING - 2) * RING_COPIES < 64, "vmcnt range");
    __shared__ __align__(16) uint8_t ring[WAVES * WAVE_RING];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r = lane & 15, g = lane >> 4;
    const int o0 = static_cast<int>(blockIdx.x) * 16, t0 = static_cast<int>(blockIdx.y) * 16;
    const int live = min(control[1], batch) - t0;   // live batch rows of this tile
    if (live <= 0)
        return;   // the whole workgroup, before any copy or barrier
    const int nk = cols / (32 * WAVES);        // blocks of each wave: b = wave + WAVES k
    const int wv = __builtin_amdgcn_readfirstlane(wave);   // the wave index as a scalar: block indexes are wave-uniform
    const uint32_t base = __builtin_amdgcn_readfirstlane(
        static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ring)) + wv * WAVE_RING);
    // per-lane sources of block wv (k = 0); block wv + WAVES k is WAVES
    // blocks further along the same rows (for the weights a fixed byte step:
    // WAVES blocks of 8-block groups, each group a multiple of 16 bytes)
    const int xrow = lane >> 3, xslot = lane & 7;   // X copy lane: row 8h + xrow, slot xslot
    const float* xsrc[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int row = 8 * h + xrow, piece = xslot ^ ((row >> 1) & 7);   // rows past the live ones repeat the last
        xsrc[h] = X + static_cast<int64_t>(t0 + min(row, live - 1)) * cols + 32 * wv + 4 * piece;
    }
    const int wrow = lane / 3, wpiece = lane % 3;   // weight copy lane (lanes < 48)
    const uint8_t* wsrc = W + static_cast<int64_t>(min(o0 + wrow, rows - 1)) * row_bytes + ring_piece<FMT>(wv, wpiece);
    constexpr int64_t WSTEP = FMT == FMT_Q4_K ? 144 * WAVES / 8 : (FMT == FMT_Q4_0 ? 18 : 34) * WAVES;
    auto request = [&](int k) {   // block wv + WAVES k into stage k % RING
        const uint32_t st = base + static_cast<uint32_t>((k % RING) * RING_STAGE);
#pragma unroll
        for (int h = 0; h < 2; h++)
            copy16_to_lds(xsrc[h] + static_cast<int64_t>(32 * WAVES) * k, st + 1024 * h);
        if (lane < 48)
            copy16_to_lds(wsrc + WSTEP * k, st + RING_XBYTES);
    };
    floatx4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int k = 0; k < RING - 1 && k < nk; k++)
        request(k);
    const int sw = (r >> 1) & 7;
    // this lane's read offsets inside a stage
    const int xo0 = 128 * r + 16 * (g ^ sw), xo1 = 128 * r + 16 * ((4 + g) ^ sw), wo = RING_XBYTES + RING_WPITCH * r;
    const uint8_t* ring_w = ring + wv * WAVE_RING;
    for (int k = 0; k < nk; k++) {
        if (k + RING - 2 < nk)
            wait_copies<(RING - 2) * RING_COPIES>();   // blocks k + 1 .. k + RING - 2 may stay in flight
        else
            wait_copies<0>();
        if (k + RING - 1 < nk)
            request(k + RING - 1);   // into the stage of block k - 1, whose reads have returned
        const uint8_t* st = ring_w + (k % RING) * RING_STAGE;
        const float4 x0 = *reinterpret_cast<const float4*>(st + xo0);
        const float4 x1 = *reinterpret_cast<const float4*>(st + xo1);
        const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        float w[8];
        decode_staged<FMT>(st + wo, wv + WAVES * k, g, w);
#pragma unroll
        for (int s = 0; s < 8; s += 2) {
            acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[s], w[s], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(xv[s + 1], w[s + 1], acc1, 0, 0, 0);
        }
    }
    __syncthreads();   // every wave is done with its ring
    floatx4* red = reinterpret_cast<floatx4*>(ring);
    red[wave * 64 + lane] = acc0 + acc1;
    __syncthreads();
    if (wave == 0) {
        floatx4 v = red[lane];
#pragma unroll
        for (int k = 1; k < WAVES; k++)
            v += red[k * 64 + lane];
        const int o = o0 + r;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int i = 4 * g + m;
            if (i < live && o < rows)
                Y[static_cast<int64_t>(t0 + i) * rows + o] = v[m];
        }
    }
}

}  // namespace

int64_t batch_values_workspace_floats(int batch, int query_heads, int context)
{
    // chunk partials [chunk][row][head][128], then the fused form's (m, l) per [chunk][row][head]
    return static_cast<int64_t>((context + BATCH_CHUNK - 1) / BATCH_CHUNK) * batch * query_heads * (BATCH_HEAD + 2);
}

hipError_t launch_batch_gather_rows(const float* table, int64_t table_rows, int width, const int32_t* control,
                                    float* out, int batch, hipStream_t s)
{
    const int64_t total = static_cast<int64_t>(batch) * width;
    hipLaunchKernelGGL(batch_gather_rows_kernel, dim3(static_cast<unsigned>((total + THREADS - 1) / THREADS)),
                       dim3(THREADS), 0, s, table, table_rows, width, control, out, total);
    return hipGetLastError();
}

hipError_t launch_batch_rms_norm(const float* hidden, const float* residual, const float* weight, float* updated,
                                 float* out, int batch, int width, float eps, const int32_t* control, hipStream_t s)
{
    auto go = [&](auto per) {
        constexpr int PER = decltype(per)::value;
        if (residual)
            hipLaunchKernelGGL((batch_rms_norm_kernel<true, PER>), dim3(static_cast<unsigned>(batch)),
                               dim3(NORM_THREADS), 0, s, hidden, residual, weight, updated, out, width, eps, control);
        else
            hipLaunchKernelGGL((batch_rms_norm_kernel<false, PER>), dim3(static_cast<unsigned>(batch)),
                               dim3(NORM_THREADS), 0, s, hidden, nullptr, weight, nullptr, out, width, eps, control);
    };
    if (width <= NORM_THREADS)
        go(std::integral_constant<int, 1>{});
    else if (width <= 2 * NORM_THREADS)
        go(std::integral_constant<int, 2>{});
    else if (width <= 4 * NORM_THREADS)
        go(std::integral_constant<int, 4>{});
    else if (width <= 8 * NORM_THREADS)
        go(std::integral_constant<int, 8>{});
    else
        go(std::integral_constant<int, 0>{});
    return hipGetLastError();
}

hipError_t launch_batch_swiglu(const float* gate_up, float* out, int batch, int width, const int32_t* control,
                               hipStream_t s)
{
    const int64_t total = static_cast<int64_t>(batch) * width;
    hipLaunchKernelGGL(batch_swiglu_kernel, dim3(static_cast<unsigned>((total + THREADS - 1) / THREADS)), dim3(THREADS),
                       0, s, gate_up, out, width, total, control);
    return hipGetLastError();
}

hipError_t launch_batch_rope_kv_write(const BatchRopeArgs& a, hipStream_t s)
{
    const int64_t total = static_cast<int64_t>(a.batch) * (a.query_size + 2 * a.kv_size);
    const dim3 grid(static_cast<unsigned>((total + THREADS - 1) / THREADS));
    if (a.cache_fp16)
        hipLaunchKernelGGL((batch_rope_kv_write_kernel<__half>), grid, dim3(THREADS), 0, s, a,
                           static_cast<__half*>(a.key_cache), static_cast<__half*>(a.value_cache));
    else
        hipLaunchKernelGGL((batch_rope_kv_write_kernel<float>), grid, dim3(THREADS), 0, s, a,
                           static_cast<float*>(a.key_cache), static_cast<float*>(a.value_cache));
    return hipGetLastError();
}

hipError_t launch_batch_gqa_scores(const BatchAttentionArgs& a, hipStream_t s)
{
    const dim3 grid(static_cast<unsigned>(a.kv_heads),
                    static_cast<unsigned>((a.context + BATCH_CHUNK - 1) / BATCH_CHUNK));
    if (a.cache_fp16)
        hipLaunchKernelGGL((batch_gqa_scores_kernel<__half>), grid, dim3(THREADS), 0, s, a,
                           static_cast<const __half*>(a.cache));
    else
        hipLaunchKernelGGL((batch_gqa_scores_kernel<float>), grid, dim3(THREADS), 0, s, a,
                           static_cast<const float*>(a.cache));
    return hipGetLastError();
}

hipError_t launch_batch_causal_softmax(const float* scores, float* probabilities, int batch, int heads, int context,
                                       const int32_t* control, hipStream_t s)
{
    hipLaunchKernelGGL(batch_causal_softmax_kernel, dim3(static_cast<unsigned>(batch * heads)), dim3(THREADS), 0, s,
                       scores, probabilities, heads, context, control);
    return hipGetLastError();
}

hipError_t launch_batch_gqa_values(const BatchAttentionArgs& a, hipStream_t s)
{
    const dim3 grid(static_cast<unsigned>(a.kv_heads),
                    static_cast<unsigned>((a.context + BATCH_CHUNK - 1) / BATCH_CHUNK));
    if (a.cache_fp16)
        hipLaunchKernelGGL((batch_gqa_values_partial_kernel<__half>), grid, dim3(THREADS), 0, s, a,
                           static_cast<const __half*>(a.cache));
    else
        hipLaunchKernelGGL((batch_gqa_values_partial_kernel<float>), grid, dim3(THREADS), 0, s, a,
                           static_cast<const float*>(a.cache));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    hipLaunchKernelGGL(batch_gqa_values_reduce_kernel, dim3(static_cast<unsigned>(a.batch * a.query_heads)),
                       dim3(BATCH_HEAD), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_batch_gqa_attention(const BatchAttentionArgs& a, const void* value_cache, hipStream_t s)
{
    const dim3 grid(static_cast<unsigned>(a.kv_heads),
                    static_cast<unsigned>((a.context + BATCH_CHUNK - 1) / BATCH_CHUNK));
    if (a.cache_fp16)
        hipLaunchKernelGGL((batch_gqa_flash_partial_kernel<__half>), grid, dim3(THREADS), 0, s, a,
                           static_cast<const __half*>(a.cache), static_cast<const __half*>(value_cache));
    else
        hipLaunchKernelGGL((batch_gqa_flash_partial_kernel<float>), grid, dim3(THREADS), 0, s, a,
                           static_cast<const float*>(a.cache), static_cast<const float*>(value_cache));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    hipLaunchKernelGGL(batch_gqa_flash_merge_kernel, dim3(static_cast<unsigned>(a.batch * a.query_heads)),
                       dim3(BATCH_HEAD), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_batch_select_last(const float* input, float* out, int batch, int width, const int32_t* control,
                                    hipStream_t s)
{
    hipLaunchKernelGGL(batch_select_last_kernel, dim3(static_cast<unsigned>((width + THREADS - 1) / THREADS)),
                       dim3(THREADS), 0, s, input, out, batch, width, control);
    return hipGetLastError();
}

hipError_t launch_batch_matvec(int fmt, const void* w, const float* x, float* y, int batch, int64_t rows,
                               int64_t cols, const int32_t* control, hipStream_t s)
{
    const dim3 grid(static_cast<unsigned>((rows + 15) / 16), static_cast<unsigned>((batch + 15) / 16));
    const uint8_t* wb = static_cast<const uint8_t*>(w);
    const int64_t rb = row_bytes(fmt, cols);
    const int r = static_cast<int>(rows), c = static_cast<int>(cols);
    if (cols % (32 * RING_WAVES) == 0) {   // weight and input are 16-byte aligned (checked by the ABI)
        // grids of more than one workgroup per CU: 8 waves with three stages
        // each (67.6 KB of LDS, two workgroups a CU); smaller grids: 16 waves
        // (four a SIMD on the CUs they occupy) when the blocks divide, else 8
        // waves with four stages
        const bool small = (rows + 15) / 16 <= 256;
        const bool wide = small && cols % (32 * 2 * RING_WAVES) == 0;
#define SI_RING_LAUNCH(F)                                                                                              \
    do {                                                                                                              \
        if (wide)                                                                                                     \
            hipLaunchKernelGGL((batch_matvec_ring_kernel<F, 3, 2 * RING_WAVES>), grid, dim3(128 * RING_WAVES), 0, s,  \
                               wb, x, y, batch, r, c, rb, control);                                                   \
        else if (small)                                                                                               \
            hipLaunchKernelGGL((batch_matvec_ring_kernel<F, 4, RING_WAVES>), grid, dim3(64 * RING_WAVES), 0, s, wb,   \
                               x, y, batch, r, c, rb, control);                                                       \
        else                                                                                                          \
            hipLaunchKernelGGL((batch_matvec_ring_kernel<F, 3, RING_WAVES>), grid, dim3(64 * RING_WAVES), 0, s, wb,   \
                               x, y, batch, r, c, rb, control);                                                       \
        return hipGetLastError();                                                                                     \
    } while (0)
        switch (fmt) {
        case FMT_Q8_0: SI_RING_LAUNCH(FMT_Q8_0);
        case FMT_Q4_0: SI_RING_LAUNCH(FMT_Q4_0);
        case FMT_Q4_K: SI_RING_LAUNCH(FMT_Q4_K);
        default: break;
        }
#undef SI_RING_LAUNCH
    }
    switch (fmt) {
    case FMT_Q8_0: hipLaunchKernelGGL((batch_matvec_kernel<FMT_Q8_0>), grid, dim3(THREADS), 0, s, wb, x, y, batch, r, c, rb, control); break;
    case FMT_Q4_0: hipLaunchKernelGGL((batch_matvec_kernel<FMT_Q4_0>), grid, dim3(THREADS), 0, s, wb, x, y, batch, r, c, rb, control); break;
    case FMT_Q4_K: hipLaunchKernelGGL((batch_matvec_kernel<FMT_Q4_K>), grid, dim3(THREADS), 0, s, wb, x, y, batch, r, c, rb, control); break;
    case FMT_F16: hipLaunchKernelGGL((batch_matvec_kernel<FMT_F16>), grid, dim3(THREADS), 0, s, wb, x, y, batch, r, c, rb, control); break;
    case FMT_F32: hipLaunchKernelGGL((batch_matvec_kernel<FMT_F32>), grid, dim3(THREADS), 0, s, wb, x, y, batch, r, c, rb, control); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace si
