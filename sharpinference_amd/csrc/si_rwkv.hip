// RWKV-7 time-mix core, LayerNorm and FP32 batched mat-vec kernels.
//
// The reference expresses one layer's WKV step as ~40 unfused portable
// tensor nodes (PortableRwkv7GraphProvider.cs:224-276): decay and
// adaptation from their LoRA outputs, key normalisation per head, key and
// value adjustment, the state update
//   S'[h,i,j] = S[h,i,j] w[h,j] + v[h,i] k[h,j] - (sum_l S[h,i,l] kn[h,l]) kn[h,j] a[h,j]
// (two batched mat-vecs and two head outer products), the readout S' . r,
// GroupNorm, the r_k bonus and the gate.  Here one workgroup owns one head:
// its 64x64 FP32 state (16 KB) is read once and written once, and every
// per-head vector lives in LDS.
#include "si_rwkv.hpp"

namespace si {
namespace {

constexpr int WKV_THREADS = 256;   // 4 threads per state row, 16 columns each

__device__ __forceinline__ float sigm(float v) { return 1.0f / (1.0f + expf(-v)); }

// Sums over the 4 lanes of a quad and over the wave, left in every lane:
// DPP moves inside quads and 16-lane rows, then swaps between the wave's
// halves and between row pairs (v_permlane32_swap / v_permlane16_swap), so
// no step waits for an LDS round trip.
__device__ __forceinline__ float quad_sum(float v)
{
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
    return v;
}

__device__ __forceinline__ float wave_sum(float v)
{
    v = quad_sum(v);
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false));  // row_half_mirror
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false));  // row_mirror
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__global__ __launch_bounds__(WKV_THREADS) void rwkv_wkv_kernel(WkvArgs a)
{
    constexpr int N = RWKV_HEAD;
    __shared__ float s_decay[N], s_key[N], s_value[N], s_kn[N], s_ak[N], s_r[N], s_y[N];
    __shared__ float s_bonus;
    const int h = blockIdx.x;
    const int t = threadIdx.x;
    const int o = h * N;
    float* S = a.state + static_cast<int64_t>(h) * N * N;
    const int i = t >> 2;              // state row
    const int j0 = (t & 3) * 16;       // first of this thread's 16 columns

    // Every global load is issued here, before any result is waited for:
    // the state tile, then (wave 0, one element per lane) the head vectors,
    // the GroupNorm affine and gate, and the side copy's value.  Loads are
    // unconditional (the first layer's value inputs read v instead of the
    // v_lora / v0 / v_first it does not use), so no branch holds them back
    // behind an earlier round trip; the side copy is stored at the end.
    float4 sv[4];
#pragma unroll
    for (int q = 0; q < 4; q++)
        sv[q] = *reinterpret_cast<const float4*>(S + i * N + j0 + 4 * q);
    const int e = o + (t & (N - 1));
    const bool first = a.first_layer != 0;
    float kk = 0.0f, wl = 0.0f, w0 = 0.0f, al = 0.0f, a0 = 0.0f, kkk = 0.0f, kka = 0.0f, vv = 0.0f, vf = 0.0f,
          vl = 0.0f, v0 = 0.0f, rr = 0.0f, rk = 0.0f, lw = 0.0f, lb = 0.0f, gt = 0.0f, cp = 0.0f;
    if (t < N) {
        kk = a.k[e];
        wl = a.w_lora[e];
        w0 = a.w0[e];
        al = a.a_lora[e];
        a0 = a.a0[e];
        kkk = a.k_k[e];
        kka = a.k_a[e];
        vv = a.v[e];
        vf = (first ? a.v : a.v_first)[e];
        vl = (first ? a.v : a.v_lora)[e];
        v0 = (first ? a.v : a.v0)[e];
        rr = a.r[e];
        rk = a.r_k[e];
        lw = a.lnx_weight[e];
        lb = a.lnx_bias[e];
        gt = a.gate[e];
        cp = (a.copy_src ? a.copy_src : a.v)[e];
    }

    if (t < N) {   // wave 0: one element of each head vector per lane
        const float decay = expf(-0.606531f * sigm(wl + w0));                      // :232-234
        const float ad = sigm(al + a0);                                           // :235-237
        const float sk = kk * kkk;                                                // :241-246
        const float squares = wave_sum(sk * sk);
        const float kn = sk * (1.0f / sqrtf(squares > 1e-24f ? squares : 1e-24f));
        const float ka = kk * kka;                                                // :247-248
        const float key = (kk + ad * ka) - ka;
        const float value = first ? vv : vv + (vf - vv) * sigm(vl + v0);          // :249-257
        if (first)
            a.v_first[e] = vv;
        const float bonus = wave_sum((key * rr) * rk);                           // :274-275
        s_decay[t] = decay;
        s_key[t] = key;
        s_value[t] = value;
        s_kn[t] = kn;
        s_ak[t] = kn * ad;                                                       // adaptedKey :254
        s_r[t] = rr;
        if (t == 0)
            s_bonus = bonus;
    }
    __syncthreads();

    // proj_i = sum_l S[i][l] kn[l] over the old state
    float p = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int j = j0 + 4 * q;
        p = fmaf(sv[q].x, s_kn[j], p);
        p = fmaf(sv[q].y, s_kn[j + 1], p);
        p = fmaf(sv[q].z, s_kn[j + 2], p);
        p = fmaf(sv[q].w, s_kn[j + 3], p);
    }
    const float negp = 0.0f - quad_sum(p);
    const float vi = s_value[i];
    float y = 0.0f;
    auto upd = [&](float s, int j) {
        const float n = (s * s_decay[j] + vi * s_key[j]) + negp * s_ak[j];
        y = fmaf(n, s_r[j], y);
        return n;
    };
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int j = j0 + 4 * q;
        sv[q].x = upd(sv[q].x, j);
        sv[q].y = upd(sv[q].y, j + 1);
        sv[q].z = upd(sv[q].z, j + 2);
        sv[q].w = upd(sv[q].w, j + 3);
        *reinterpret_cast<float4*>(S + i * N + j) = sv[q];
    }
    y = quad_sum(y);
    if ((t & 3) == 0)
        s_y[i] = y;
    __syncthreads();

    if (t < N) {   // GroupNorm (eps 64e-5) + ln_x affine, bonus, gate (:272-276)
        const float yv = s_y[t];
        const float mean = wave_sum(yv) / static_cast<float>(N);
        const float c = yv - mean;
        const float var = wave_sum(c * c) / static_cast<float>(N);
        const float ln = c * (1.0f / sqrtf(var + 64e-5f)) * lw + lb;
        a.out[o + t] = (ln + s_value[t] * s_bonus) * gt;
        if (a.copy_src)
            a.copy_dst[o + t] = cp;
    }
}

constexpr int LN_THREADS = 1024;
constexpr int LN_MAX = 8192;

__device__ __forceinline__ float block_sum(float v, float* red)
{
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < LN_THREADS / 64; k++)
        s += red[k];
    return s;
}

__global__ __launch_bounds__(LN_THREADS) void layernorm_kernel(const float* __restrict__ x, const float* w,
                                                                 const float* b, int n, float eps, float* out)
{
    constexpr int PER = LN_MAX / LN_THREADS;
    __shared__ float red1[LN_THREADS / 64], red2[LN_THREADS / 64];
    float v[PER];
    float s1 = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int e = threadIdx.x + k * LN_THREADS;
        v[k] = e < n ? x[e] : 0.0f;
        s1 += v[k];
    }
    const float mean = block_sum(s1, red1) / static_cast<float>(n);
    float s2 = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int e = threadIdx.x + k * LN_THREADS;
        v[k] = e < n ? v[k] - mean : 0.0f;
        s2 += v[k] * v[k];
    }
    const float inv = 1.0f / sqrtf(block_sum(s2, red2) / static_cast<float>(n) + eps);
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int e = threadIdx.x + k * LN_THREADS;
        if (e < n)
            out[e] = v[k] * inv * w[e] + b[e];
    }
}

// One wave per output row; lanes stride over the columns.
__global__ __launch_bounds__(256) void batched_matvec_kernel(const float* __restrict__ m, const float* __restrict__ v,
                                                             float* __restrict__ out, int batch, int rows, int cols)
{
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= static_cast<int64_t>(batch) * rows)
        return;   // whole wave leaves together; no barrier follows
    const int bt = static_cast<int>(row / rows);
    const float* mr = m + row * cols;
    const float* vb = v + static_cast<int64_t>(bt) * cols;
    float acc = 0.0f;
    for (int c = lane; c < cols; c += 64)
        acc = fmaf(mr[c], vb[c], acc);
    acc = wave_sum(acc);
    if (lane == 0)
        out[row] = acc;
}

}  // namespace

hipError_t launch_rwkv_wkv(const WkvArgs& a, hipStream_t s)
{
    if (a.heads <= 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(rwkv_wkv_kernel, dim3(static_cast<unsigned>(a.heads)), dim3(WKV_THREADS), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_layernorm(const float* x, const float* w, const float* b, int n, float eps, float* out,
                            hipStream_t s)
{
    if (n <= 0 || n > LN_MAX)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(layernorm_kernel, dim3(1), dim3(LN_THREADS), 0, s, x, w, b, n, eps, out);
    return hipGetLastError();
}

hipError_t launch_batched_matvec(const float* m, const float* v, float* out, int batch, int rows, int cols,
                                 hipStream_t s)
{
    const int64_t total = static_cast<int64_t>(batch) * rows;
    if (batch <= 0 || rows <= 0 || cols <= 0 || (total + 3) / 4 > 0x7fffffff)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(batched_matvec_kernel, dim3(static_cast<unsigned>((total + 3) / 4)), dim3(256), 0, s, m, v,
                       out, batch, rows, cols);
    return hipGetLastError();
}

}  // namespace si
