// Decode-step operators around the quantized products: embedding row
// gather, grouped-query attention over an fp16 KV cache with the rotary
// embedding and the cache append fused in, and argmax.
//
// Semantics follow the Phi-4 text model of the reference
// (SharpInference.Architectures.Phi4/Phi4TextModel.cs): Embed :44-53,
// ApplyRotary :212-229 (rotate-half over the first `rotary_dim` values of
// each head, cos/sin scaled by rope_scale), ComputeAttention :231-273
// (scores q.k / sqrt(head_dim) over every cached token including the new
// one, softmax, weighted sum of values), and the D3D12 program's argmax
// (GpuTransformerInstructionCollection.cs:697-748: first index of the
// maximum) and gather-row (GpuTierZeroInstruction.cs:397-405: an index
// outside the table yields NaN).  The benchmark decode step keeps K and V in
// fp16: new rows are rounded to fp16 when appended and attention reads the
// rounded values back.
#include "si_internal.hpp"
#include "si_decode.hpp"
#include "si_rows.hpp"
#include "si_lanes.hpp"

#include <hip/hip_fp16.h>

#include <map>
#include <mutex>
#include <type_traits>

namespace si {
namespace {

// Attention workspace of the allocation-free entry point: chunk partials
// and the rotary table, as a caller-provided workspace holds them.  Every
// context on one GPU shares this array; it keeps the last call's contents,
// and nothing in it has to start at zero (each call writes every partial
// and table entry it reads).  Host code never passes `scratch` itself to a
// kernel: it passes the address attention_scratch() looked up.
static __device__ __align__(256) float scratch[ATTENTION_SCRATCH_FLOATS];

constexpr int HEAD_DIM = 128;
constexpr int CHUNK = 64;          // cache positions per workgroup of the staged partial kernel (workspace layout)
constexpr int FCHUNK = 128;        // cache positions per workgroup of the register-resident chunk kernel
constexpr int FPPL = FCHUNK / 16;  // positions per lane of the chunk kernel
constexpr int ATT_THREADS = 256;
constexpr int PART = HEAD_DIM + 2; // per head and chunk: max, sum, 128 weighted values

// ---- embedding gather -------------------------------------------------------

// Row `*index` of the table into out (columns strided over `blocks`
// workgroups of 256 threads, this one `block`); an index outside the table
// yields NaN.
template <int FMT>
__device__ __forceinline__ void gather_row(const uint8_t* __restrict__ table, int rows, int cols, int64_t row_bytes,
                                           const int32_t* __restrict__ index, float* __restrict__ out, int block,
                                           int blocks)
{
    const int row = *index;
    const bool valid = row >= 0 && row < rows;
    const uint8_t* rp = table + static_cast<int64_t>(valid ? row : 0) * row_bytes;
    for (int c = block * 256 + threadIdx.x; c < cols; c += blocks * 256)
        out[c] = valid ? row_value<FMT>(rp, c) : __int_as_float(0x7fc00000);
}

template <int FMT>
__global__ __launch_bounds__(256) void gather_row_kernel(const uint8_t* __restrict__ table, int rows, int cols,
                                                         int64_t row_bytes, const int32_t* __restrict__ index,
                                                         float* __restrict__ out)
{
    gather_row<FMT>(table, rows, cols, row_bytes, index, out, blockIdx.x, gridDim.x);
}

// ---- attention ------------------------------------------------------------------

// Workspace of one attention launch: per query head and chunk the partial
// (max, sum, 128 weighted values), then the rotary table of the current
// position (cos at [0, R/2), sin at [64, 64 + R/2), both already scaled).
__host__ __device__ inline int64_t att_rope(int heads, int max_chunks)
{
    return (static_cast<int64_t>(heads) * max_chunks * PART + 63) / 64 * 64;
}

// Rotary embedding of one pair in place (values in LDS): pairs (i, i + R/2)
// for i < R/2 with the precomputed cos / sin of the position.
__device__ __forceinline__ void rotate_pair(float* h, int i, int rotary, const float* rope)
{
    const float c = rope[i], s = rope[64 + i];
    const float left = h[i], right = h[i + rotary / 2];
    h[i] = left * c - right * s;
    h[i + rotary / 2] = right * c + left * s;
}

// 8 values already rounded to fp16 precision, as the cache words hold them.
__device__ __forceinline__ uint4 pack8(const float* f)
{
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
        w[i] = static_cast<uint32_t>(__half_as_ushort(__float2half_rn(f[2 * i]))) |
               (static_cast<uint32_t>(__half_as_ushort(__float2half_rn(f[2 * i + 1]))) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ uint4 select4(bool c, const uint4& a, const uint4& b)
{
    return make_uint4(c ? a.x : b.x, c ? a.y : b.y, c ? a.z : b.z, c ? a.w : b.w);
}

__device__ __forceinline__ void unpack8(const uint4& r, float* f)
{
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f[2 * i] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[i] & 0xffffu)));
        f[2 * i + 1] = __half2float(__ushort_as_half(static_cast<unsigned short>(w[i] >> 16)));
    }
}


// Once per step: the rotary table of the new position (frequency
// 1 / base^(2i / R), cos / sin scaled by rope_scale), shared by every layer
// that attends at that position.
__device__ __forceinline__ void rope_table(const AttentionArgs& a, int t)
{
    const int P = *a.position;
    float* rope = a.workspace + att_rope(a.heads, a.max_chunks);
    if (t < a.rotary_dim / 2) {
        const float freq = 1.0f / powf(a.rope_base, 2.0f * static_cast<float>(t) / static_cast<float>(a.rotary_dim));
        const float angle = static_cast<float>(P) * freq;
        rope[t] = cosf(angle) * a.rope_scale;
        rope[64 + t] = sinf(angle) * a.rope_scale;
    }
}

__global__ __launch_bounds__(64) void attention_prep_kernel(AttentionArgs a) { rope_table(a, threadIdx.x); }

// The decode step's first launch: the embedding row of the token (every
// workgroup but the last) and the step's rotary table (the last
// workgroup); both read only the step's control values.
template <int FMT>
__global__ __launch_bounds__(256) void step_start_kernel(const uint8_t* __restrict__ table, int rows, int cols,
                                                         int64_t row_bytes, const int32_t* __restrict__ index,
                                                         float* __restrict__ out, AttentionArgs a)
{
    const int gather_blocks = static_cast<int>(gridDim.x) - 1;
    if (static_cast<int>(blockIdx.x) == gather_blocks) {
        if (threadIdx.x < 64)
            rope_table(a, threadIdx.x);
        return;
    }
    gather_row<FMT>(table, rows, cols, row_bytes, index, out, blockIdx.x, gather_blocks);
}

constexpr int MAX_CHUNKS = 256;

// One workgroup per query head merges the chunk partials (m_c, l_c, o_c):
// out = sum_c o_c e^(m_c - M) / sum_c l_c e^(m_c - M) with M = max_c m_c.
// Thread (half, d) takes chunks half, half + 2, ... in batches of
// COMBINE_BATCH, every load of a batch issued together, and merges the
// batches online; the two halves merge through LDS.  The first batch is
// written ahead of the position read (slots past the position hold stale
// partials and are masked), but the compiler issues its loads inside the
// merge's branch, after the position check: a cache of up to
// 2 * COMBINE_BATCH chunks costs the position's round trip and one more.
// (A branch-free merge that keeps them ahead of the position measured
// slower; merging inside the last partial workgroup needs a device-scope
// release per workgroup, which writes back the XCD's L2 and costs far more
// than this launch.)
constexpr int COMBINE_BATCH = 16;

struct CombineBatch {
    float m[COMBINE_BATCH], l[COMBINE_BATCH], o[COMBINE_BATCH];
};

__device__ __forceinline__ void load_combine_batch(const float* src, int base, int max_chunks, int d, CombineBatch& b)
{
#pragma unroll
    for (int i = 0; i < COMBINE_BATCH; i++) {
        const int c = base + 2 * i;
        const float* p = src + static_cast<int64_t>(c < max_chunks ? c : 0) * PART;
        b.m[i] = p[0];
        b.l[i] = p[1];
        b.o[i] = p[2 + d];
    }
}

// Folds the batch's chunks below `chunks` into (m, l, acc).
__device__ __forceinline__ void merge_combine_batch(const CombineBatch& b, int base, int chunks, float& m, float& l,
                                                    float& acc)
{
    float bm = m;
#pragma unroll
    for (int i = 0; i < COMBINE_BATCH; i++)
        if (base + 2 * i < chunks)
            bm = fmaxf(bm, b.m[i]);
    const float r = __expf(m - bm);   // m = -inf before the first batch: r = 0
    float bl = 0.0f, bo = 0.0f;
#pragma unroll
    for (int i = 0; i < COMBINE_BATCH; i++) {
        if (base + 2 * i < chunks) {
            const float w = __expf(b.m[i] - bm);
            bl = fmaf(b.l[i], w, bl);
            bo = fmaf(b.o[i], w, bo);
        }
    }
    l = fmaf(l, r, bl);
    acc = fmaf(acc, r, bo);
    m = bm;
}

// The pointers arrive as preloaded scalar arguments; exponentials use the
// hardware exp2 (__expf), within a few ulp of expf.
__global__ __launch_bounds__(256) void attention_combine_kernel(const float* __restrict__ workspace,
                                                                const int32_t* __restrict__ position,
                                                                float* __restrict__ out, int capacity,
                                                                int max_chunks, int chunk_size)
{
    const int h = blockIdx.x, t = threadIdx.x;
    const int d = t & (HEAD_DIM - 1), half = t >> 7;
    const float* src = workspace + static_cast<int64_t>(h) * max_chunks * PART;
    CombineBatch b;
    load_combine_batch(src, half, max_chunks, d, b);
    const int P = *position;
    if (P < 0 || P >= capacity) {
        if (t < HEAD_DIM)
            out[h * HEAD_DIM + t] = __int_as_float(0x7fc00000);   // position outside the cache
        return;
    }
    const int chunks = P / chunk_size + 1;
    float m = -INFINITY, l = 0.0f, acc = 0.0f;
    if (half < chunks)
        merge_combine_batch(b, half, chunks, m, l, acc);
    for (int base = half + 2 * COMBINE_BATCH; base < chunks; base += 2 * COMBINE_BATCH) {
        load_combine_batch(src, base, max_chunks, d, b);
        merge_combine_batch(b, base, chunks, m, l, acc);
    }
    __shared__ float other[HEAD_DIM + 2];
    if (half == 1) {
        other[d] = acc;
        if (d == 0) {
            other[HEAD_DIM] = m;
            other[HEAD_DIM + 1] = l;
        }
    }
    __syncthreads();
    if (half == 0) {
        const float m1 = other[HEAD_DIM];
        const float M = fmaxf(m, m1);
        const float e0 = __expf(m - M), e1 = __expf(m1 - M);   // half 1 without chunks: m1 = -inf, e1 = 0
        out[h * HEAD_DIM + d] = fmaf(acc, e0, other[d] * e1) / fmaf(l, e0, other[HEAD_DIM + 1] * e1);
    }
}

// One workgroup = one KV head x one chunk of 64 cache positions.  Writes
// per query head of the group: (max score, sum of exp, sum of exp * v).
// The inputs that do not depend on the position (the group's queries, the
// new K / V rows, the step's rotary table) are requested together with the
// position; then every K and V row of the chunk is requested (16-byte
// loads, one 8-value slice per lane), and the queries are staged and
// rotated while those loads are in flight.
template <int GROUP>
__global__ __launch_bounds__(ATT_THREADS) void attention_partial_kernel(AttentionArgs a)
{
    constexpr int QPT = (GROUP * HEAD_DIM + ATT_THREADS - 1) / ATT_THREADS;   // query values per thread
    const int g = blockIdx.x;                 // KV head
    const int chunk = blockIdx.y;
    const int start = chunk * CHUNK;
    const int koff = a.heads * HEAD_DIM, voff = koff + a.kv_heads * HEAD_DIM;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int dg = t & 15;                    // 8-value slice of a head row

    // 1. position-independent inputs, into registers
    float qr[QPT];
#pragma unroll
    for (int e = 0; e < QPT; e++) {
        const int i = t + e * ATT_THREADS;
        qr[e] = a.qkv[g * GROUP * HEAD_DIM + (i < GROUP * HEAD_DIM ? i : 0)];
    }
    const float* rope = a.workspace + att_rope(a.heads, a.max_chunks);
    const int ti = t & (HEAD_DIM - 1);
    const float kn = a.qkv[koff + g * HEAD_DIM + ti];
    const float vn = a.qkv[voff + g * HEAD_DIM + ti];
    const float rp = rope[ti];                // cos at [0, 64), sin at [64, 128)

    const int P = *a.position;                // index of the new token
    if (P < 0 || P >= a.capacity || start > P)
        return;                               // whole workgroup leaves together
    const int count = min(CHUNK, P + 1 - start);
    const int newp = P - start;               // the new token's slot in this chunk (< CHUNK when owned)
    const bool owns_new = newp < CHUNK;

    __half* kc = a.k_cache + static_cast<int64_t>(g) * a.capacity * HEAD_DIM;
    __half* vc = a.v_cache + static_cast<int64_t>(g) * a.capacity * HEAD_DIM;

    // 2. K rows for the scores (wave w: positions 16w..16w+15) and V rows
    //    for the weighted sum (position slot t/16 + 16j).  The loads are
    //    unconditional (rows clamped into the cache) so that all eight are
    //    in flight at once; rows past the chunk's count and the new token's
    //    slot are masked afterwards (V to zero, K through the score mask).
    uint4 kr[4], vr[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int pk = wave * 16 + (lane >> 4) + 4 * j;
        const int pv = (t >> 4) + 16 * j;
        kr[j] = *reinterpret_cast<const uint4*>(kc + static_cast<int64_t>(min(start + pk, a.capacity - 1)) * HEAD_DIM +
                                                8 * dg);
        vr[j] = *reinterpret_cast<const uint4*>(vc + static_cast<int64_t>(min(start + pv, a.capacity - 1)) * HEAD_DIM +
                                                8 * dg);
    }

    __shared__ float q[GROUP][HEAD_DIM];
    __shared__ float knew[HEAD_DIM];
    __shared__ float vnew[HEAD_DIM];
    __shared__ float rope_s[HEAD_DIM];
    __shared__ float prob[GROUP][CHUNK];
    __shared__ float mx[GROUP];
    __shared__ float lsum[GROUP];
    __shared__ float red[4][GROUP][HEAD_DIM];

    // 3. rotated queries of the group; the new row, rotated, rounded, appended
#pragma unroll
    for (int e = 0; e < QPT; e++) {
        const int i = t + e * ATT_THREADS;
        if (i < GROUP * HEAD_DIM)
            q[i / HEAD_DIM][i % HEAD_DIM] = qr[e];
    }
    if (t < HEAD_DIM) {
        knew[t] = kn;
        vnew[t] = vn;
        rope_s[t] = rp;
    }
    __syncthreads();
    const int half_rot = a.rotary_dim / 2;
    for (int i = t; i < GROUP * half_rot; i += ATT_THREADS)
        rotate_pair(q[i / half_rot], i % half_rot, a.rotary_dim, rope_s);
    if (owns_new && t < half_rot)
        rotate_pair(knew, t, a.rotary_dim, rope_s);
    __syncthreads();
    if (owns_new && t < HEAD_DIM) {
        const __half kh = __float2half_rn(knew[t]), vh = __float2half_rn(vnew[t]);
        kc[static_cast<int64_t>(P) * HEAD_DIM + t] = kh;
        vc[static_cast<int64_t>(P) * HEAD_DIM + t] = vh;
        knew[t] = __half2float(kh);
        vnew[t] = __half2float(vh);
    }
    __syncthreads();

    // 3. scores: a 16-lane row holds one position's 128 values
    float qv[GROUP][8];
#pragma unroll
    for (int h = 0; h < GROUP; h++)
#pragma unroll
        for (int e = 0; e < 8; e++)
            qv[h][e] = q[h][8 * dg + e];
    const float inv_scale = sqrtf(static_cast<float>(HEAD_DIM));
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int p = wave * 16 + (lane >> 4) + 4 * j;
        float k8[8];
        if (p == newp) {
#pragma unroll
            for (int e = 0; e < 8; e++)
                k8[e] = knew[8 * dg + e];
        } else {
            unpack8(kr[j], k8);
        }
#pragma unroll
        for (int h = 0; h < GROUP; h++) {
            float sdot = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; e++)
                sdot = fmaf(qv[h][e], k8[e], sdot);
            sdot = row_sum<16>(sdot);
            if (dg == 0)
                prob[h][p] = p < count ? sdot / inv_scale : -INFINITY;
        }
    }
    __syncthreads();

    // 4. per-head max and exponentials (wave h takes head h)
    if (wave < GROUP) {
        const float v = prob[wave][lane];
        float m = v;
        for (int off = 32; off > 0; off >>= 1)
            m = fmaxf(m, __shfl_xor(m, off));
        const float e = lane < count ? expf(v - m) : 0.0f;
        float l = e;
        for (int off = 32; off > 0; off >>= 1)
            l += __shfl_xor(l, off);
        prob[wave][lane] = e;
        if (lane == 0) {
            mx[wave] = m;
            lsum[wave] = l;
        }
    }
    __syncthreads();

    // 5. weighted values: thread (slot t/16, slice t%16) over 4 positions,
    //    then a sum over the 16 position slots
    float acc[GROUP][8];
#pragma unroll
    for (int h = 0; h < GROUP; h++)
#pragma unroll
        for (int e = 0; e < 8; e++)
            acc[h][e] = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int p = (t >> 4) + 16 * j;
        float v8[8];
        if (p == newp) {
#pragma unroll
            for (int e = 0; e < 8; e++)
                v8[e] = vnew[8 * dg + e];
        } else {
            unpack8(p < count ? vr[j] : make_uint4(0, 0, 0, 0), v8);   // rows past the count may hold anything
        }
#pragma unroll
        for (int h = 0; h < GROUP; h++) {
            const float w = prob[h][p];
#pragma unroll
            for (int e = 0; e < 8; e++)
                acc[h][e] = fmaf(w, v8[e], acc[h][e]);
        }
    }
#pragma unroll
    for (int h = 0; h < GROUP; h++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float v = acc[h][e];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            acc[h][e] = v;
        }
    if (lane < 16) {
#pragma unroll
        for (int h = 0; h < GROUP; h++)
#pragma unroll
            for (int e = 0; e < 8; e++)
                red[wave][h][8 * dg + e] = acc[h][e];
    }
    __syncthreads();
    float* part_out = a.workspace;
    for (int i = t; i < GROUP * HEAD_DIM; i += ATT_THREADS) {
        const int h = i / HEAD_DIM, d = i % HEAD_DIM;
        const float o = (red[0][h][d] + red[1][h][d]) + (red[2][h][d] + red[3][h][d]);
        float* dst = part_out + (static_cast<int64_t>(g * GROUP + h) * a.max_chunks + chunk) * PART;
        dst[2 + d] = o;
        if (d == 0) {
            dst[0] = mx[h];
            dst[1] = lsum[h];
        }
    }
}


__device__ __forceinline__ void load8(const float* p, float* f)
{
    const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}

// Rotate-half of a thread's 8-value slice dg of one head row (rotary width
// R, a multiple of 16 so that a slice and its partner slice are whole):
// for i < R/2, h[i] = h[i] c_i - h[i + R/2] s_i; for R/2 <= i < R,
// h[i] = h[i] c_{i-R/2} + h[i - R/2] s_{i-R/2}; other values unchanged.
// `own` holds the slice, `partner` the slice R/2 away, cs / sn the table
// values of the pair.
__device__ __forceinline__ void rotate8(float* own, const float* partner, const float* cs, const float* sn, int dg,
                                        int rotary)
{
    const int i0 = 8 * dg;
    if (i0 < rotary / 2) {
#pragma unroll
        for (int e = 0; e < 8; e++)
            own[e] = own[e] * cs[e] - partner[e] * sn[e];
    } else if (i0 < rotary) {
#pragma unroll
        for (int e = 0; e < 8; e++)
            own[e] = own[e] * cs[e] + partner[e] * sn[e];
    }
}

// One workgroup = one KV head x one chunk of 128 cache positions, the same
// function as attention_partial_kernel with every intermediate kept in
// registers.  Thread (wave w, lane l) takes the 8-value slice dg = l % 16
// of positions 32 w + l / 16 + 4 j (j < 8) for both the scores and the
// values, so its softmax weights never leave its registers: each wave keeps
// its own running maximum and sum, sums across its four rows with lane
// swaps, and the four waves merge (with rescaling) through LDS at one
// barrier.  The queries, the new K / V rows and their rotary partners are
// read straight from the step's qkv vector and rotated in registers; the
// 16 lanes holding the new token's position round it to fp16 and append it.
// The pointers a wave needs first arrive as preloaded scalar arguments.
// BOUNDED: the grid holds only chunks that start at or below every position
// the caller replays it with (a step recorded for a range of positions), so
// every chunk's K / V rows are requested together with the position instead
// of after it.
template <int GROUP, bool BOUNDED>
__global__ __launch_bounds__(ATT_THREADS) void attention_chunk_kernel(const float* __restrict__ qkv,
                                                                      const int32_t* __restrict__ position,
                                                                      __half* k_cache, __half* v_cache,
                                                                      float* __restrict__ workspace, int capacity,
                                                                      int rotary, int max_chunks)
{
    // max_chunks: the workspace's partials per head (its 64-position layout);
    // this grid has ceil(capacity / 128) chunks
    const int g = blockIdx.x;                 // KV head
    const int kv_heads = gridDim.x;
    const int heads = GROUP * kv_heads;
    const int chunk = blockIdx.y;
    const int start = chunk * FCHUNK;
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int dg = lane & 15, row = lane >> 4;
    const int half = rotary / 2;
    const bool rot = 8 * dg < rotary;
    // the partner slice of a rotated slice (any valid slice otherwise)
    const int pdg = !rot ? dg : (8 * dg < half ? dg + half / 8 : dg - half / 8);
    const int tdg = 8 * dg < half ? dg : (rot ? dg - half / 8 : 0);   // table slice of the pair

    // 1. position-independent inputs: queries, new K / V slices, rotary table
    const float* qg = qkv + static_cast<int64_t>(g) * GROUP * HEAD_DIM;
    const float* kn_row = qkv + static_cast<int64_t>(heads) * HEAD_DIM + g * HEAD_DIM;
    const float* vn_row = kn_row + static_cast<int64_t>(kv_heads) * HEAD_DIM;
    const float* rope = workspace + att_rope(heads, max_chunks);
    float q[GROUP][8], qp[GROUP][8], kn[8], knp[8], vn[8], cs[8], sn[8];
#pragma unroll
    for (int h = 0; h < GROUP; h++) {
        load8(qg + h * HEAD_DIM + 8 * dg, q[h]);
        load8(qg + h * HEAD_DIM + 8 * pdg, qp[h]);
    }
    load8(kn_row + 8 * dg, kn);
    load8(kn_row + 8 * pdg, knp);
    load8(vn_row + 8 * dg, vn);
    load8(rope + 8 * tdg, cs);
    load8(rope + 64 + 8 * tdg, sn);

    // A chunk past the position (or a position outside the cache) loads no
    // cache rows and stores nothing, but runs the same straight-line code:
    // with an early return the compiler would move the loads above (used
    // only on the valid path) behind the position's round trip.
    const int P = *position;                  // index of the new token
    const bool valid = P >= 0 && P < capacity && start <= P;
    const int count = min(FCHUNK, P + 1 - start);
    const int newp = valid ? P - start : FCHUNK;   // the new token's slot in this chunk (< FCHUNK when owned)

    // 2. K and V rows of this thread's positions (rows clamped into the
    //    cache; positions past the count are masked below)
    __half* kc = k_cache + static_cast<int64_t>(g) * capacity * HEAD_DIM;
    __half* vc = v_cache + static_cast<int64_t>(g) * capacity * HEAD_DIM;
    //    (an invalid chunk leaves them unloaded: its results are not stored)
    uint4 kr[FPPL], vr[FPPL];
    if (BOUNDED || valid) {
#pragma unroll
        for (int j = 0; j < FPPL; j++) {
            const int64_t r = min(start + wave * (FCHUNK / 4) + row + 4 * j, capacity - 1);
            kr[j] = *reinterpret_cast<const uint4*>(kc + r * HEAD_DIM + 8 * dg);
            vr[j] = *reinterpret_cast<const uint4*>(vc + r * HEAD_DIM + 8 * dg);
        }
    }

    // 3. rotate the queries and the new key; the new row in fp16
#pragma unroll
    for (int h = 0; h < GROUP; h++)
        rotate8(q[h], qp[h], cs, sn, dg, rotary);
    rotate8(kn, knp, cs, sn, dg, rotary);
#pragma unroll
    for (int e = 0; e < 8; e++) {
        kn[e] = __half2float(__float2half_rn(kn[e]));
        vn[e] = __half2float(__float2half_rn(vn[e]));
    }

    // 4. scores of the thread's four positions (a 16-lane row holds one
    //    position), masked past the count
    // scores q.k / sqrt(head_dim) as q.k * (1 / sqrt(head_dim)), and
    // exponentials with the hardware exp2 (__expf): both within a few ulp
    // of the exact forms, far inside the attention tolerance
    // 5. the wave's maximum and exponentials per head; weighted values
    //
    // A chunk that ends at or before the new position (every chunk but the
    // last) has all its positions cached and does not hold the new one: it
    // takes the form without masks.  The last chunk puts the new row's fp16
    // words in place of the loaded cache words at its position and zeroes
    // the words past the count with selects (no divergent branches), then
    // runs the same arithmetic, so both forms give the same values.
    const float rscale = 1.0f / sqrtf(static_cast<float>(HEAD_DIM));
    float sc[GROUP][FPPL];
    float m[GROUP], l[GROUP], acc[GROUP][8];
    auto attend = [&](auto whole_chunk) {
        constexpr bool WHOLE = decltype(whole_chunk)::value;
        uint4 knw = make_uint4(0, 0, 0, 0), vnw = knw;
        if constexpr (!WHOLE) {
            knw = pack8(kn);
            vnw = pack8(vn);
        }
#pragma unroll
        for (int j = 0; j < FPPL; j++) {
            const int p = wave * (FCHUNK / 4) + row + 4 * j;
            float k8[8];
            unpack8(WHOLE ? kr[j] : select4(p == newp, knw, kr[j]), k8);
#pragma unroll
            for (int h = 0; h < GROUP; h++) {
                float sdot = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++)
                    sdot = fmaf(q[h][e], k8[e], sdot);
                sdot = row_sum<16>(sdot);
                sc[h][j] = WHOLE || p < count ? sdot * rscale : -INFINITY;
            }
        }
#pragma unroll
        for (int h = 0; h < GROUP; h++) {
            float mh = sc[h][0];
#pragma unroll
            for (int j = 1; j < FPPL; j++)
                mh = fmaxf(mh, sc[h][j]);
            mh = rows_max(mh);
            m[h] = mh;
            float lh = 0.0f;
#pragma unroll
            for (int j = 0; j < FPPL; j++) {
                const float e = !WHOLE && sc[h][j] == -INFINITY ? 0.0f : __expf(sc[h][j] - mh);
                sc[h][j] = e;
                lh += e;
            }
            l[h] = lh;
#pragma unroll
            for (int e = 0; e < 8; e++)
                acc[h][e] = 0.0f;
        }
#pragma unroll
        for (int j = 0; j < FPPL; j++) {
            const int p = wave * (FCHUNK / 4) + row + 4 * j;
            float v8[8];
            // rows past the count may hold anything
            unpack8(WHOLE ? vr[j] : select4(p == newp, vnw, select4(p < count, vr[j], make_uint4(0, 0, 0, 0))), v8);
#pragma unroll
            for (int h = 0; h < GROUP; h++)
#pragma unroll
                for (int e = 0; e < 8; e++)
                    acc[h][e] = fmaf(sc[h][j], v8[e], acc[h][e]);
        }
    };
    if (__builtin_amdgcn_readfirstlane(static_cast<int>(valid && start + FCHUNK <= P)))
        attend(std::true_type{});
    else
        attend(std::false_type{});

    // the owner's 16 lanes append the new row (positions of a lane are
    // wave * 32 + row + 4 j, so the new one is in row newp % 4 of wave newp / 32)
    if (newp < FCHUNK && newp / (FCHUNK / 4) == wave && (newp & 3) == row) {   // newp < FCHUNK only when valid
        __half kh[8], vh[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
            kh[e] = __float2half_rn(kn[e]);
            vh[e] = __float2half_rn(vn[e]);
        }
        *reinterpret_cast<uint4*>(kc + static_cast<int64_t>(P) * HEAD_DIM + 8 * dg) = *reinterpret_cast<const uint4*>(kh);
        *reinterpret_cast<uint4*>(vc + static_cast<int64_t>(P) * HEAD_DIM + 8 * dg) = *reinterpret_cast<const uint4*>(vh);
    }

    // 6. every 16-lane row's sums into LDS, then the rows and the four
    //    waves merged there: (r0 + r2) + (r1 + r3) per wave, the order of a
    //    swap of the wave's halves followed by a swap of row pairs, so the
    //    cross-lane swaps (and their register copies) are left out
    __shared__ float4 red4[4][4][GROUP][HEAD_DIM / 4];
    __shared__ float wm[4][GROUP], wl[4][4][GROUP];
#pragma unroll
    for (int h = 0; h < GROUP; h++) {
        red4[wave][row][h][2 * dg] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
        red4[wave][row][h][2 * dg + 1] = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
    }
    if (dg == 0)
#pragma unroll
        for (int h = 0; h < GROUP; h++) {
            wl[wave][row][h] = l[h];
            if (row == 0)
                wm[wave][h] = m[h];
        }
    __syncthreads();
    if (!valid)
        return;
    const float* red = reinterpret_cast<const float*>(red4);
    auto part = [&](int w, int r, int h, int d) { return red[((w * 4 + r) * GROUP + h) * HEAD_DIM + d]; };
    for (int i = t; i < GROUP * HEAD_DIM; i += ATT_THREADS) {
        const int h = i / HEAD_DIM, d = i % HEAD_DIM;
        const float M = fmaxf(fmaxf(wm[0][h], wm[1][h]), fmaxf(wm[2][h], wm[3][h]));
        float o = 0.0f, lsum = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float f = wm[w][h] == -INFINITY ? 0.0f : __expf(wm[w][h] - M);   // a wave without valid positions adds nothing
            const float ow = (part(w, 0, h, d) + part(w, 2, h, d)) + (part(w, 1, h, d) + part(w, 3, h, d));
            const float lw = (wl[w][0][h] + wl[w][2][h]) + (wl[w][1][h] + wl[w][3][h]);
            o = fmaf(ow, f, o);
            lsum = fmaf(lw, f, lsum);
        }
        float* dst = workspace + (static_cast<int64_t>(g * GROUP + h) * max_chunks + chunk) * PART;
        dst[2 + d] = o;
        if (d == 0) {
            dst[0] = M;
            dst[1] = lsum;
        }
    }
}

// ---- argmax ----------------------------------------------------------------------------

constexpr int AM_BLOCKS = 256;

__device__ __forceinline__ void better(float& bv, int& bi, float v, int i)
{
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// better() over the lane that DPP control CTRL reads from.
template <int CTRL>
__device__ __forceinline__ void better_dpp(float& bv, int& bi)
{
    const float ov = dpp_row<CTRL>(bv);
    const int oi = dpp_row<CTRL>(bi);
    better(bv, bi, ov, oi);
}

// The wave's best (value, index) in every lane: DPP inside quads and rows,
// then the swaps between halves and row pairs.  better() is a total order
// (larger value, then smaller index; NaN never wins), so the result does
// not depend on the pairing.
__device__ __forceinline__ void wave_best(float& bv, int& bi)
{
    better_dpp<0xB1>(bv, bi);    // quad_perm 1,0,3,2
    better_dpp<0x4E>(bv, bi);    // quad_perm 2,3,0,1
    better_dpp<0x141>(bv, bi);   // row_half_mirror
    better_dpp<0x140>(bv, bi);   // row_mirror
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(bv), __float_as_uint(bv), false, false);
    const auto ai = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(bi), static_cast<unsigned>(bi), false, false);
    bv = __uint_as_float(a[0]);
    bi = static_cast<int>(ai[0]);
    better(bv, bi, __uint_as_float(a[1]), static_cast<int>(ai[1]));
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(bv), __float_as_uint(bv), false, false);
    const auto bi2 = __builtin_amdgcn_permlane16_swap(static_cast<unsigned>(bi), static_cast<unsigned>(bi), false, false);
    bv = __uint_as_float(b[0]);
    bi = static_cast<int>(bi2[0]);
    better(bv, bi, __uint_as_float(b[1]), static_cast<int>(bi2[1]));
}

// The four waves' results through LDS at one barrier; thread 0 returns the
// workgroup's best.
__device__ __forceinline__ void block_best(float& bv, int& bi)
{
    __shared__ float sv[4];
    __shared__ int si[4];
    wave_best(bv, bi);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[wave] = bv;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0)
        for (int w = 1; w < 4; w++)
            better(bv, bi, sv[w], si[w]);
}

// The first AM_PER values of a thread are requested together (indices
// clamped into the vector, n >= 1), the rest (vectors longer than
// AM_PER * AM_BLOCKS * 256) one after another.
constexpr int AM_PER = 4;

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float* __restrict__ v, int n,
                                                             float* __restrict__ pv, int* __restrict__ pi)
{
    constexpr int STRIDE = AM_BLOCKS * 256;
    const int i0 = blockIdx.x * 256 + threadIdx.x;
    float vals[AM_PER];
#pragma unroll
    for (int k = 0; k < AM_PER; k++)
        vals[k] = v[min(i0 + k * STRIDE, n - 1)];
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int k = 0; k < AM_PER; k++)
        if (i0 + k * STRIDE < n)
            better(bv, bi, vals[k], i0 + k * STRIDE);
    for (int64_t i = i0 + AM_PER * STRIDE; i < n; i += STRIDE)
        better(bv, bi, v[i], static_cast<int>(i));
    block_best(bv, bi);
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = bv;
        pi[blockIdx.x] = bi;
    }
}

__global__ __launch_bounds__(256) void argmax_final_kernel(const float* __restrict__ pv, const int* __restrict__ pi,
                                                           int32_t* __restrict__ out)
{
    float bv = pv[threadIdx.x];
    int bi = pi[threadIdx.x];
    block_best(bv, bi);
    if (threadIdx.x == 0)
        *out = bi == 0x7fffffff ? 0 : bi;
}

}  // namespace

int64_t attention_workspace_floats(int heads, int capacity)
{
    return att_rope(heads, (capacity + CHUNK - 1) / CHUNK) + 2 * 64;
}

int64_t argmax_workspace_bytes() { return AM_BLOCKS * 8; }

hipError_t attention_scratch(int device, float** out)
{
    static std::mutex lock;
    static std::map<int, float*> address;   // one copy of the array per GPU
    std::lock_guard<std::mutex> hold(lock);
    const auto it = address.find(device);
    if (it != address.end()) {
        *out = it->second;
        return hipSuccess;
    }
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
        return e != hipSuccess ? e : hipErrorInvalidSymbol;
    address[device] = static_cast<float*>(p);
    *out = static_cast<float*>(p);
    return hipSuccess;
}

hipError_t launch_gather_row(int fmt, const void* table, int64_t rows, int64_t cols, const int32_t* index, float* out,
                             hipStream_t s)
{
    const int64_t rb = row_bytes(fmt, cols);
    const int64_t nblk = (cols + 255) / 256;
    const dim3 grid(static_cast<unsigned>(nblk < 64 ? nblk : 64));
    const uint8_t* t = static_cast<const uint8_t*>(table);
    switch (fmt) {
    case FMT_Q8_0: hipLaunchKernelGGL((gather_row_kernel<FMT_Q8_0>), grid, dim3(256), 0, s, t, static_cast<int>(rows), static_cast<int>(cols), rb, index, out); break;
    case FMT_Q4_0: hipLaunchKernelGGL((gather_row_kernel<FMT_Q4_0>), grid, dim3(256), 0, s, t, static_cast<int>(rows), static_cast<int>(cols), rb, index, out); break;
    case FMT_Q4_K: hipLaunchKernelGGL((gather_row_kernel<FMT_Q4_K>), grid, dim3(256), 0, s, t, static_cast<int>(rows), static_cast<int>(cols), rb, index, out); break;
    case FMT_F16: hipLaunchKernelGGL((gather_row_kernel<FMT_F16>), grid, dim3(256), 0, s, t, static_cast<int>(rows), static_cast<int>(cols), rb, index, out); break;
    case FMT_F32: hipLaunchKernelGGL((gather_row_kernel<FMT_F32>), grid, dim3(256), 0, s, t, static_cast<int>(rows), static_cast<int>(cols), rb, index, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_step_start(int fmt, const void* table, int64_t rows, int64_t cols, const int32_t* index, float* out,
                             const AttentionArgs& a, hipStream_t s)
{
    const int64_t rb = row_bytes(fmt, cols);
    const int64_t nblk = (cols + 255) / 256;
    const dim3 grid(static_cast<unsigned>((nblk < 64 ? nblk : 64) + 1));
    const uint8_t* t = static_cast<const uint8_t*>(table);
    const int r = static_cast<int>(rows), c = static_cast<int>(cols);
    switch (fmt) {
    case FMT_Q8_0: hipLaunchKernelGGL((step_start_kernel<FMT_Q8_0>), grid, dim3(256), 0, s, t, r, c, rb, index, out, a); break;
    case FMT_Q4_0: hipLaunchKernelGGL((step_start_kernel<FMT_Q4_0>), grid, dim3(256), 0, s, t, r, c, rb, index, out, a); break;
    case FMT_Q4_K: hipLaunchKernelGGL((step_start_kernel<FMT_Q4_K>), grid, dim3(256), 0, s, t, r, c, rb, index, out, a); break;
    case FMT_F16: hipLaunchKernelGGL((step_start_kernel<FMT_F16>), grid, dim3(256), 0, s, t, r, c, rb, index, out, a); break;
    case FMT_F32: hipLaunchKernelGGL((step_start_kernel<FMT_F32>), grid, dim3(256), 0, s, t, r, c, rb, index, out, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_attention_prep(const AttentionArgs& a, hipStream_t s)
{
    hipLaunchKernelGGL(attention_prep_kernel, dim3(1), dim3(64), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_attention(const AttentionArgs& a, hipStream_t s, bool prep)
{
    if (a.head_dim != HEAD_DIM || a.kv_heads <= 0 || a.heads % a.kv_heads != 0 || a.max_chunks > MAX_CHUNKS ||
        a.rotary_dim > HEAD_DIM)
        return hipErrorInvalidValue;
    if (prep) {
        const hipError_t e = launch_attention_prep(a, s);
        if (e != hipSuccess)
            return e;
    }
    const int group = a.heads / a.kv_heads;
    const dim3 grid(static_cast<unsigned>(a.kv_heads), static_cast<unsigned>(a.max_chunks));
    if (a.rotary_dim % 16 == 0) {
        const int all = (a.capacity + FCHUNK - 1) / FCHUNK;
        const bool bounded = a.chunk_bound > 0;
        if (bounded && a.chunk_bound > all)
            return hipErrorInvalidValue;
        const dim3 fgrid(static_cast<unsigned>(a.kv_heads), static_cast<unsigned>(bounded ? a.chunk_bound : all));
        // slices of 8 values and their rotary partners are whole
        switch (group * 2 + (bounded ? 1 : 0)) {
#define SI_CHUNK(G, B)                                                                                            \
    case G * 2 + B:                                                                                               \
        hipLaunchKernelGGL((attention_chunk_kernel<G, B>), fgrid, dim3(ATT_THREADS), 0, s, a.qkv, a.position,     \
                           a.k_cache, a.v_cache, a.workspace, a.capacity, a.rotary_dim, a.max_chunks);           \
        break;
        SI_CHUNK(1, 0)
        SI_CHUNK(2, 0)
        SI_CHUNK(3, 0)
        SI_CHUNK(4, 0)
        SI_CHUNK(1, 1)
        SI_CHUNK(2, 1)
        SI_CHUNK(3, 1)
        SI_CHUNK(4, 1)
#undef SI_CHUNK
        default: return hipErrorInvalidValue;
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess)
            return e;
        // positions past the chunks of a bounded grid count as outside the cache
        const int limit = bounded ? min(a.capacity, a.chunk_bound * FCHUNK) : a.capacity;
        hipLaunchKernelGGL(attention_combine_kernel, dim3(static_cast<unsigned>(a.heads)), dim3(256), 0, s, a.workspace,
                       a.position, a.out, limit, a.max_chunks, FCHUNK);
        return hipGetLastError();
    }
    if (a.chunk_bound > 0)
        return hipErrorNotSupported;   // the bounded grid is built for rotary widths that are multiples of 16
    switch (group) {
    case 1: hipLaunchKernelGGL((attention_partial_kernel<1>), grid, dim3(ATT_THREADS), 0, s, a); break;
    case 2: hipLaunchKernelGGL((attention_partial_kernel<2>), grid, dim3(ATT_THREADS), 0, s, a); break;
    case 3: hipLaunchKernelGGL((attention_partial_kernel<3>), grid, dim3(ATT_THREADS), 0, s, a); break;
    case 4: hipLaunchKernelGGL((attention_partial_kernel<4>), grid, dim3(ATT_THREADS), 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    hipLaunchKernelGGL(attention_combine_kernel, dim3(static_cast<unsigned>(a.heads)), dim3(256), 0, s, a.workspace,
                       a.position, a.out, a.capacity, a.max_chunks, CHUNK);
    return hipGetLastError();
}

hipError_t launch_argmax(const float* values, int64_t n, void* workspace, int32_t* out, hipStream_t s)
{
    if (n <= 0 || n > INT32_MAX)
        return hipErrorInvalidValue;
    float* pv = static_cast<float*>(workspace);
    int* pi = reinterpret_cast<int*>(pv + AM_BLOCKS);
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(AM_BLOCKS), dim3(256), 0, s, values, static_cast<int>(n), pv, pi);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, s, pv, pi, out);
    return hipGetLastError();
}

}  // namespace si
