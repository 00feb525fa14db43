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
#include "si_lanes.hpp"

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

// head_size 128, group G <= 4: one workgroup = one KV head x 128 cache rows
// (the decode step's register-resident form, without its rotary and
// append: rope-kv-write has already rotated the query and written the row).
// Thread (wave w, lane l) takes the 8-value slice l % 16 of rows
// 32 w + l / 16 + 4 j (j < 8) for both the scores and the values, so the
// softmax weights stay in its registers: each wave keeps its maximum and
// sum, sums across its four rows with lane swaps, and the four waves merge
// (with rescaling) through LDS at one barrier.  Rows past the active range
// count as absent.  Partials (m, l, o) of each query head and chunk go to
// the workspace at the 64-row layout's index (chunk < its chunk count).
constexpr int GQA_FCHUNK = 128;

template <typename T>
struct CacheSlice {   // 8 consecutive values of one cache row as loaded
    uint4 w[sizeof(T) == 2 ? 1 : 2];
};
template <typename T>
__device__ __forceinline__ CacheSlice<T> load_slice(const T* p)
{
    CacheSlice<T> r;
#pragma unroll
    for (int i = 0; i < (sizeof(T) == 2 ? 1 : 2); i++)
        r.w[i] = reinterpret_cast<const uint4*>(p)[i];
    return r;
}
__device__ __forceinline__ void unpack_slice(const CacheSlice<__half>& r, float* f)
{
    const uint32_t w[4] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
        f[2 * k] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[k] & 0xffffu)));
        f[2 * k + 1] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[k] >> 16)));
    }
}
__device__ __forceinline__ void unpack_slice(const CacheSlice<float>& r, float* f)
{
    f[0] = __uint_as_float(r.w[0].x); f[1] = __uint_as_float(r.w[0].y);
    f[2] = __uint_as_float(r.w[0].z); f[3] = __uint_as_float(r.w[0].w);
    f[4] = __uint_as_float(r.w[1].x); f[5] = __uint_as_float(r.w[1].y);
    f[6] = __uint_as_float(r.w[1].z); f[7] = __uint_as_float(r.w[1].w);
}

template <typename T, int G>
__global__ __launch_bounds__(GQA_THREADS) void gqa_chunk_kernel(GqaArgs a, const T* __restrict__ kc,
                                                                const T* __restrict__ vc)
{
    constexpr int HEAD = 128, PPL = GQA_FCHUNK / 16;   // rows per lane
    const int g = blockIdx.x, chunk = blockIdx.y;
    const int start = chunk * GQA_FCHUNK;
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int dg = lane & 15, row = lane >> 4;
    float q[G][8];
#pragma unroll
    for (int h = 0; h < G; h++)
        load8(a.query + static_cast<int64_t>(g * G + h) * HEAD + 8 * dg, q[h]);
    const int active = min(max(*a.position, 0), a.context - 1);
    const bool valid = start <= active;
    const int count = min(GQA_FCHUNK, active + 1 - start);
    const int64_t row_stride = static_cast<int64_t>(a.kv_heads) * HEAD;
    const T* kb = kc + static_cast<int64_t>(g) * HEAD + 8 * dg;
    const T* vb = vc + static_cast<int64_t>(g) * HEAD + 8 * dg;
    CacheSlice<T> kr[PPL], vr[PPL];
    if (valid) {   // a chunk past the active rows loads nothing and stores nothing
#pragma unroll
        for (int j = 0; j < PPL; j++) {
            const int64_t r = min(start + wave * (GQA_FCHUNK / 4) + row + 4 * j, a.context - 1);
            kr[j] = load_slice(kb + r * row_stride);
            vr[j] = load_slice(vb + r * row_stride);
        }
    }
    // scores q.k / sqrt(128) (a 16-lane row holds one cache row), masked
    // past the count; exponentials with the hardware exp2 (__expf)
    const float rscale = 1.0f / sqrtf(static_cast<float>(HEAD));
    float sc[G][PPL];
#pragma unroll
    for (int j = 0; j < PPL; j++) {
        const int p = wave * (GQA_FCHUNK / 4) + row + 4 * j;
        float k8[8];
        unpack_slice(kr[j], k8);
#pragma unroll
        for (int h = 0; h < G; h++) {
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++)
                d = fmaf(q[h][e], k8[e], d);
            d = row_sum<16>(d);
            sc[h][j] = p < count ? d * rscale : -INFINITY;
        }
    }
    float m[G], l[G], acc[G][8];
#pragma unroll
    for (int h = 0; h < G; h++) {
        float mh = sc[h][0];
#pragma unroll
        for (int j = 1; j < PPL; j++)
            mh = fmaxf(mh, sc[h][j]);
        mh = rows_max(mh);
        m[h] = mh;
        float lh = 0.0f;
#pragma unroll
        for (int j = 0; j < PPL; j++) {
            const float e = sc[h][j] == -INFINITY ? 0.0f : __expf(sc[h][j] - mh);
            sc[h][j] = e;
            lh += e;
        }
        l[h] = lh;
#pragma unroll
        for (int e = 0; e < 8; e++)
            acc[h][e] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < PPL; j++) {
        const int p = wave * (GQA_FCHUNK / 4) + row + 4 * j;
        float v8[8];
        unpack_slice(vr[j], v8);
#pragma unroll
        for (int e = 0; e < 8; e++)
            v8[e] = p < count ? v8[e] : 0.0f;   // rows past the count may hold anything
#pragma unroll
        for (int h = 0; h < G; h++)
#pragma unroll
            for (int e = 0; e < 8; e++)
                acc[h][e] = fmaf(sc[h][j], v8[e], acc[h][e]);
    }
    __shared__ float red[4][G][HEAD];
    __shared__ float wm[4][G], wl[4][G];
#pragma unroll
    for (int h = 0; h < G; h++) {
        l[h] = rows_sum(l[h]);
#pragma unroll
        for (int e = 0; e < 8; e++)
            acc[h][e] = rows_sum(acc[h][e]);
    }
    if (row == 0) {
#pragma unroll
        for (int h = 0; h < G; h++)
#pragma unroll
            for (int e = 0; e < 8; e++)
                red[wave][h][8 * dg + e] = acc[h][e];
        if (dg == 0)
#pragma unroll
            for (int h = 0; h < G; h++) {
                wm[wave][h] = m[h];
                wl[wave][h] = l[h];
            }
    }
    __syncthreads();
    if (!valid)
        return;
    for (int i = t; i < G * HEAD; i += GQA_THREADS) {
        const int h = i / HEAD, d = i % HEAD;
        const float M = fmaxf(fmaxf(wm[0][h], wm[1][h]), fmaxf(wm[2][h], wm[3][h]));   // finite: row start is active
        float o = 0.0f, lsum = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float f = wm[w][h] == -INFINITY ? 0.0f : __expf(wm[w][h] - M);   // a wave without active rows adds nothing
            o = fmaf(red[w][h][d], f, o);
            lsum = fmaf(wl[w][h], f, lsum);
        }
        float* dst = a.workspace + (static_cast<int64_t>(g * G + h) * a.chunks + chunk) * (HEAD + 2);
        dst[2 + d] = o;
        if (d == 0) {
            dst[0] = M;
            dst[1] = lsum;
        }
    }
}

// The merge of CHUNK-row partials: one workgroup per query head, batches of
// 8 chunks requested together, merged online (m, l, o rescaled per batch).
template <int HEAD, int CHUNK>
__global__ __launch_bounds__(HEAD) void gqa_merge_chunks_kernel(GqaArgs a)
{
    const int head = blockIdx.x, d = threadIdx.x;
    const int active = min(max(*a.position, 0), a.context - 1);
    const int n = active / CHUNK + 1;
    const float* src = a.workspace + static_cast<int64_t>(head) * a.chunks * (HEAD + 2);
    float m = -INFINITY, L = 0.0f, O = 0.0f;
    for (int c0 = 0; c0 < n; c0 += 8) {
        float mc[8], lc[8], oc[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float* pc = src + static_cast<int64_t>(min(c0 + u, n - 1)) * (HEAD + 2);
            mc[u] = pc[0];
            lc[u] = pc[1];
            oc[u] = pc[2 + d];
        }
        float bm = m;
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (c0 + u < n)
                bm = fmaxf(bm, mc[u]);
        const float r = __expf(m - bm);   // m = -inf before the first batch: r = 0
        L *= r;
        O *= r;
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (c0 + u < n) {
                const float e = __expf(mc[u] - bm);
                L = fmaf(lc[u], e, L);
                O = fmaf(oc[u], e, O);
            }
        m = bm;
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
    const int group = a.kv_heads > 0 ? a.query_heads / a.kv_heads : 0;
    if (a.head_size == 128 && group >= 1 && group <= 4 && group * a.kv_heads == a.query_heads) {
        // the register-resident form over 128-row chunks
        const dim3 fgrid(static_cast<unsigned>(a.kv_heads), static_cast<unsigned>((a.context + GQA_FCHUNK - 1) / GQA_FCHUNK));
        switch (group * 2 + (a.cache_fp16 ? 1 : 0)) {
#define SI_GQA_CHUNK(G, F, T)                                                                                     \
    case G * 2 + F:                                                                                               \
        hipLaunchKernelGGL((gqa_chunk_kernel<T, G>), fgrid, dim3(GQA_THREADS), 0, s, a,                          \
                           static_cast<const T*>(a.key_cache), static_cast<const T*>(a.value_cache));            \
        break;
        SI_GQA_CHUNK(1, 0, float)
        SI_GQA_CHUNK(2, 0, float)
        SI_GQA_CHUNK(3, 0, float)
        SI_GQA_CHUNK(4, 0, float)
        SI_GQA_CHUNK(1, 1, __half)
        SI_GQA_CHUNK(2, 1, __half)
        SI_GQA_CHUNK(3, 1, __half)
        SI_GQA_CHUNK(4, 1, __half)
#undef SI_GQA_CHUNK
        default: return hipErrorInvalidValue;
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess)
            return e;
        hipLaunchKernelGGL((gqa_merge_chunks_kernel<128, GQA_FCHUNK>), heads, dim3(128), 0, s, a);
        return hipGetLastError();
    }
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
