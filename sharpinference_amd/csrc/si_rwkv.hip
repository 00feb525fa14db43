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
#include "si_lanes.hpp"
#include "si_internal.hpp"
#include "si_planes.hpp"
#include "si_rows.hpp"

#include <hip/hip_fp16.h>

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
    v += dpp_row<0xB1>(v);   // quad_perm 1,0,3,2
    v += dpp_row<0x4E>(v);   // quad_perm 2,3,0,1
    return v;
}

__device__ __forceinline__ float wave_sum(float v)
{
    v = quad_sum(v);
    v += dpp_row<0x141>(v);  // row_half_mirror
    v += dpp_row<0x140>(v);  // row_mirror
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// The LoRA outputs of one head formed in the kernel (lora_fmt Q8_0 /
// Q4_0): the head's 64 rows of each up matrix (contiguous, 64 * row bytes,
// a multiple of 16) are staged into LDS with 16-byte loads and the hidden
// vectors as int8 digit planes (encode_planes); each (block, row) product
// is one v_dot4_i32_i8 block product, a wave taking one block column of a
// matrix with one row per lane, and the blocks of a row are summed in
// order.  A block's bytes start at an even LDS offset: its quant words are
// read as aligned dwords from the first quant byte's dword and realigned
// with v_alignbit.
constexpr int LORA_THREADS = 512;
constexpr int LORA_MAX_BLOCKS = WKV_LORA_MAX_ITEMS / RWKV_HEAD;   // hidden blocks (32 values) of the four vectors

// One block of an up-matrix row (bytes at LDS offset `off`) times its
// hidden block: the digit-plane product (planes P, inv = 2^-s, sum8 =
// 8 sum(X)) when the block's planes are valid (inv not NaN), else the
// per-weight FP32 form over the block's FP32 values x.
template <int FMT>
__device__ __forceinline__ float lora_block(const uint32_t* lw, int off, const uint32_t* P, float inv, int sum8,
                                            const float* x)
{
    const uint8_t* lb = reinterpret_cast<const uint8_t*>(lw);
    const float d = __half2float(__ushort_as_half(*reinterpret_cast<const unsigned short*>(lb + off)));
    const int q0 = off + 2;
    const uint32_t* W = lw + (q0 >> 2);
    const uint32_t sh = static_cast<uint32_t>(q0 & 3) * 8u;   // 0 or 16
    if constexpr (FMT == FMT_Q8_0) {
        uint32_t w[9], q[8];
#pragma unroll
        for (int k = 0; k < 9; k++)
            w[k] = W[k];
#pragma unroll
        for (int k = 0; k < 8; k++)
            q[k] = __builtin_amdgcn_alignbit(w[k + 1], w[k], sh);
        if (__builtin_expect(inv == inv, 1))
            return d * (q8_planes_sum(q, P) * inv);
        float acc = 0.0f;   // a = fma(q_i, x_i, a) for i = 0..31, then d * a
        for (int k = 0; k < 8; k++)
            for (int b = 0; b < 4; b++)
                acc = fmaf(static_cast<float>(static_cast<int8_t>(q[k] >> (8 * b))), x[4 * k + b], acc);
        return d * acc;
    } else {
        uint32_t w[5], q[4], lo[4], hi[4];
#pragma unroll
        for (int k = 0; k < 5; k++)
            w[k] = W[k];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            q[k] = __builtin_amdgcn_alignbit(w[k + 1], w[k], sh);
            lo[k] = q[k] & 0x0f0f0f0fu;
            hi[k] = (q[k] >> 4) & 0x0f0f0f0fu;
        }
        if (__builtin_expect(inv == inv, 1))
            return (d * inv) * static_cast<float>(q4_planes_sum(lo, hi, P) - sum8);
        float acc = 0.0f;   // a = fma(lo_i - 8, x_i, a); a = fma(hi_i - 8, x_(i+16), a) for i = 0..15
        for (int i = 0; i < 16; i++) {
            const uint32_t byte = (q[i >> 2] >> (8 * (i & 3))) & 0xffu;
            acc = fmaf(static_cast<float>(static_cast<int>(byte & 15u) - 8), x[i], acc);
            acc = fmaf(static_cast<float>(static_cast<int>(byte >> 4) - 8), x[i + 16], acc);
        }
        return d * acc;
    }
}

// LF = 0: the LoRA outputs are read from memory (256 threads).  LF = FMT_Q8_0
// / FMT_Q4_0: they are formed here (512 threads; waves 4..7 take part in the
// LoRA products only).
template <int LF>
__global__ __launch_bounds__(LF ? LORA_THREADS : WKV_THREADS) void rwkv_wkv_kernel(WkvArgs a)
{
    constexpr int N = RWKV_HEAD;
    constexpr int THREADS = LF ? LORA_THREADS : WKV_THREADS;
    constexpr int BB = LF ? block_bytes(LF) : 4;
    constexpr int HB = LF ? LORA_MAX_BLOCKS : 1;
    __shared__ float s_decay[N], s_key[N], s_value[N], s_kn[N], s_ak[N], s_r[N], s_y[N];
    __shared__ float s_bonus;
    // LoRA staging (LF only): the up rows (+16 bytes: a block's last window
    // word may lie past the staged bytes); the hidden blocks as planes
    // (plane p word w of the concatenation at 8 * HB * p + w), their 2^-s
    // (NaN: per-weight form) and 8 sum(X), and as FP32; the block products
    // [block][row]
    __shared__ uint4 s_up[LF ? WKV_LORA_LDS_BYTES / 16 + 1 : 1];
    __shared__ uint4 s_hp[3 * 2 * HB];
    __shared__ float4 s_hx[8 * HB];
    __shared__ float s_hinv[HB];
    __shared__ int s_hsum[HB];
    __shared__ float s_part[LF ? WKV_LORA_MAX_ITEMS : 1];
    const int h = blockIdx.x;
    const int t = threadIdx.x;
    const int o = h * N;
    float* S = a.state + static_cast<int64_t>(h) * N * N;
    const bool state_thread = t < WKV_THREADS;
    const int i = (t & (WKV_THREADS - 1)) >> 2;   // state row
    const int j0 = (t & 3) * 16;                  // first of this thread's 16 columns

    // LoRA staging (LF only), issued first: the up matrices' rows are the
    // largest and coldest reads of the kernel
    constexpr int UPT = LF ? (WKV_LORA_LDS_BYTES / 16 + THREADS - 1) / THREADS : 1;
    uint4 ch[UPT];
    float4 hx = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    int nb[4] = {}, cb[4] = {}, u_end[4] = {};
    int nblk = 0;
    if constexpr (LF != 0) {
        // per matrix m: blocks per row, its first hidden block, the end of
        // its chunk (uint4 units) in the staged concatenation
        int uc = 0;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            nb[m] = a.rank[m] / 32;
            cb[m] = nblk;
            nblk += nb[m];
            uc += N * nb[m] * BB / 16;
            u_end[m] = uc;
        }
        // head h's chunk of matrix m starts h * (its units) units into the
        // matrix (an absent v2 is never selected: its units are empty); the
        // matrix of a unit is chosen by sequential selects, so every load
        // below is issued before the first wait
        const uint4* const c0 = static_cast<const uint4*>(a.up[0]) + static_cast<int64_t>(h) * u_end[0];
        const uint4* const c1 = static_cast<const uint4*>(a.up[1]) + static_cast<int64_t>(h) * (u_end[1] - u_end[0]);
        const uint4* const c2 = static_cast<const uint4*>(a.up[2]) + static_cast<int64_t>(h) * (u_end[2] - u_end[1]);
        const uint4* const c3 =
            a.up[3] ? static_cast<const uint4*>(a.up[3]) + static_cast<int64_t>(h) * (u_end[3] - u_end[2]) : c0;
        // chunk loads: at most WKV_LORA_LDS_BYTES / 16 / THREADS per thread,
        // unconditional (the index clamped into the staged units) and all
        // issued before any is stored; the stores are unconditional too:
        // slots past the staged units (inside the array) take copies of the
        // last unit, which no block reads
        static_assert(THREADS * UPT <= WKV_LORA_LDS_BYTES / 16 + 1, "staging slots stay inside s_up");
#pragma unroll
        for (int j = 0; j < UPT; j++) {
            const int u = min(t + j * THREADS, uc - 1);
            const uint4* p = c0 + u;
            p = u >= u_end[0] ? c1 + (u - u_end[0]) : p;
            p = u >= u_end[1] ? c2 + (u - u_end[1]) : p;
            p = u >= u_end[2] ? c3 + (u - u_end[2]) : p;
            ch[j] = *p;
        }
        // the hidden vectors: 4 values per lane of waves 0..3 (a block's
        // 32 values in 8 consecutive lanes; the index clamped as above)
        static_assert(8 * LORA_MAX_BLOCKS <= WKV_THREADS, "waves 0..3 hold every hidden value");
        if (state_thread) {
            const int f = min(t, 8 * nblk - 1);
            const float* p = a.hid[0] + 4 * f;
            p = f >= 8 * cb[1] ? a.hid[1] + 4 * (f - 8 * cb[1]) : p;
            p = f >= 8 * cb[2] ? a.hid[2] + 4 * (f - 8 * cb[2]) : p;
            p = f >= 8 * cb[3] && a.hid[3] ? a.hid[3] + 4 * (f - 8 * cb[3]) : p;
            hx = *reinterpret_cast<const float4*>(p);
        }
    }

    // Every global load is issued here, before any result is waited for:
    // the state tile, then (wave 0, one element per lane) the head vectors,
    // the GroupNorm affine and gate, and the side copies' values.  Loads are
    // unconditional (the first layer's value inputs read v instead of the
    // v_lora / v0 / v_first it does not use), so no branch holds them back
    // behind an earlier round trip; the side copies are stored at the end.
    float4 sv[4];
    if (state_thread) {
#pragma unroll
        for (int q = 0; q < 4; q++)
            sv[q] = *reinterpret_cast<const float4*>(S + i * N + j0 + 4 * q);
    }
    const int e = o + (t & (N - 1));
    const bool first = a.first_layer != 0;
    float kk = 0.0f, wl = 0.0f, w0 = 0.0f, al = 0.0f, a0 = 0.0f, kkk = 0.0f, kka = 0.0f, vv = 0.0f, vf = 0.0f,
          vl = 0.0f, v0 = 0.0f, rr = 0.0f, rk = 0.0f, lw = 0.0f, lb = 0.0f, gt = 0.0f, cp = 0.0f, cp2 = 0.0f;
    if (t < N) {
        kk = a.k[e];
        w0 = a.w0[e];
        a0 = a.a0[e];
        kkk = a.k_k[e];
        kka = a.k_a[e];
        vv = a.v[e];
        vf = (first ? a.v : a.v_first)[e];
        v0 = (first ? a.v : a.v0)[e];
        rr = a.r[e];
        rk = a.r_k[e];
        lw = a.lnx_weight[e];
        lb = a.lnx_bias[e];
        cp = (a.copy_src ? a.copy_src : a.v)[e];
        cp2 = (a.copy2_src ? a.copy2_src : a.v)[e];
        if constexpr (LF == 0) {
            wl = a.w_lora[e];
            al = a.a_lora[e];
            vl = (first ? a.v : a.v_lora)[e];
            gt = a.gate[e];
        }
    }

    if constexpr (LF != 0) {
#pragma unroll
        for (int j = 0; j < UPT; j++)
            s_up[t + j * THREADS] = ch[j];
        if (state_thread) {   // whole waves: every lane of a block's group takes part
            const PlaneWords pl = encode_planes(hx);
            if (t < 8 * nblk) {
                uint32_t* hp = reinterpret_cast<uint32_t*>(s_hp);
                hp[t] = pl.p[0];
                hp[8 * HB + t] = pl.p[1];
                hp[16 * HB + t] = pl.p[2];
                s_hx[t] = hx;
                if ((t & 7) == 0) {
                    s_hinv[t >> 3] = pl.exact ? __builtin_nanf("") : pl.inv;
                    s_hsum[t >> 3] = 8 * pl.sum;
                }
            }
        }
        __syncthreads();
        // block products: wave w takes the block columns blk of matrix m
        // with (first block of m + blk) % 8 == w, one row per lane
        const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
        const int row = t & 63;
        const uint32_t* lwd = reinterpret_cast<const uint32_t*>(s_up);
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int base = m == 0 ? 0 : u_end[m - 1] * 16;   // LDS byte offset of matrix m's rows
            for (int blk = (wave - cb[m]) & 7; blk < nb[m]; blk += 8) {
                const int gb = cb[m] + blk;
                uint32_t P[24];
#pragma unroll
                for (int p = 0; p < 3; p++) {
                    const uint4 x0 = s_hp[(8 * HB * p + 8 * gb) / 4], x1 = s_hp[(8 * HB * p + 8 * gb) / 4 + 1];
                    P[8 * p] = x0.x; P[8 * p + 1] = x0.y; P[8 * p + 2] = x0.z; P[8 * p + 3] = x0.w;
                    P[8 * p + 4] = x1.x; P[8 * p + 5] = x1.y; P[8 * p + 6] = x1.z; P[8 * p + 7] = x1.w;
                }
                s_part[gb * N + row] = lora_block<LF>(lwd, base + (row * nb[m] + blk) * BB, P, s_hinv[gb],
                                                      s_hsum[gb], reinterpret_cast<const float*>(s_hx + 8 * gb));
            }
        }
        __syncthreads();
        if (t < N) {
            // the row's blocks in order, read 8 at a time ahead of their
            // sums (reads past the row are replaced by +0, which leaves a sum
            // that starts at +0 unchanged)
            float sum[4];
#pragma unroll
            for (int m = 0; m < 4; m++) {
                float v = 0.0f;
                for (int k0 = 0; k0 < nb[m]; k0 += 8) {
                    float p[8];
#pragma unroll
                    for (int k = 0; k < 8; k++)
                        p[k] = s_part[min(cb[m] + k0 + k, LORA_MAX_BLOCKS - 1) * N + t];
#pragma unroll
                    for (int k = 0; k < 8; k++)
                        v += k0 + k < nb[m] ? p[k] : 0.0f;
                }
                sum[m] = v;
            }
            wl = sum[0];
            al = sum[1];
            gt = sum[2];
            vl = first ? vv : sum[3];
        }
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

    if (state_thread) {
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
    }
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
        if (a.copy2_src)
            a.copy2_dst[o + t] = cp2;
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

// LayerNorm of x, or (FMT >= 0) of row *index of a GGUF table (the
// embedding gather of the same step; an index outside the table gives a
// row of NaN, as the gather does).
template <int FMT>
__global__ __launch_bounds__(LN_THREADS) void layernorm_kernel(const float* __restrict__ x, const float* w,
                                                                 const float* b, int n, float eps, float* out,
                                                                 const uint8_t* __restrict__ table, int rows,
                                                                 int64_t row_bytes, const int32_t* __restrict__ index)
{
    constexpr int PER = LN_MAX / LN_THREADS;
    __shared__ float red1[LN_THREADS / 64], red2[LN_THREADS / 64];
    float v[PER];
    float s1 = 0.0f;
    const uint8_t* rp = nullptr;
    bool valid = true;
    if constexpr (FMT >= 0) {
        const int row = *index;
        valid = row >= 0 && row < rows;
        rp = table + static_cast<int64_t>(valid ? row : 0) * row_bytes;
    }
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int e = threadIdx.x + k * LN_THREADS;
        if constexpr (FMT >= 0)
            v[k] = e < n ? (valid ? row_value<FMT>(rp, e) : __int_as_float(0x7fc00000)) : 0.0f;
        else
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

bool wkv_lora_supported(const WkvArgs& a)
{
    if (a.lora_fmt != FMT_Q8_0 && a.lora_fmt != FMT_Q4_0)
        return false;
    auto a16 = [](const void* p) { return p && (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    int blocks = 0;
    for (int m = 0; m < 4; m++) {
        const bool absent = m == 3 && a.first_layer;
        if (absent ? a.rank[m] != 0 : (a.rank[m] <= 0 || a.rank[m] % 32 != 0 || !a16(a.up[m]) || !a16(a.hid[m])))
            return false;
        blocks += a.rank[m] / 32;
    }
    return static_cast<int64_t>(RWKV_HEAD) * blocks * block_bytes(a.lora_fmt) <= WKV_LORA_LDS_BYTES &&
           RWKV_HEAD * blocks <= WKV_LORA_MAX_ITEMS;
}

hipError_t launch_rwkv_wkv(const WkvArgs& a, hipStream_t s)
{
    if (a.heads <= 0)
        return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(a.heads));
    if (a.lora_fmt == 0)
        hipLaunchKernelGGL(rwkv_wkv_kernel<0>, grid, dim3(WKV_THREADS), 0, s, a);
    else if (!wkv_lora_supported(a))
        return hipErrorInvalidValue;
    else if (a.lora_fmt == FMT_Q8_0)
        hipLaunchKernelGGL(rwkv_wkv_kernel<FMT_Q8_0>, grid, dim3(LORA_THREADS), 0, s, a);
    else
        hipLaunchKernelGGL(rwkv_wkv_kernel<FMT_Q4_0>, grid, dim3(LORA_THREADS), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_layernorm(const float* x, const float* w, const float* b, int n, float eps, float* out,
                            hipStream_t s)
{
    if (n <= 0 || n > LN_MAX)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL((layernorm_kernel<-1>), dim3(1), dim3(LN_THREADS), 0, s, x, w, b, n, eps, out, nullptr, 0,
                       int64_t{0}, nullptr);
    return hipGetLastError();
}

hipError_t launch_gather_layernorm(int fmt, const void* table, int64_t rows, int64_t cols, const int32_t* index,
                                   const float* w, const float* b, float eps, float* out, hipStream_t s)
{
    const int64_t rb = row_bytes(fmt, cols);
    if (cols <= 0 || cols > LN_MAX || rb < 0 || rows <= 0 || rows > INT32_MAX)
        return hipErrorInvalidValue;
    const uint8_t* t = static_cast<const uint8_t*>(table);
    const int n = static_cast<int>(cols), r = static_cast<int>(rows);
    switch (fmt) {
    case FMT_Q8_0: hipLaunchKernelGGL((layernorm_kernel<FMT_Q8_0>), dim3(1), dim3(LN_THREADS), 0, s, nullptr, w, b, n, eps, out, t, r, rb, index); break;
    case FMT_Q4_0: hipLaunchKernelGGL((layernorm_kernel<FMT_Q4_0>), dim3(1), dim3(LN_THREADS), 0, s, nullptr, w, b, n, eps, out, t, r, rb, index); break;
    case FMT_Q4_K: hipLaunchKernelGGL((layernorm_kernel<FMT_Q4_K>), dim3(1), dim3(LN_THREADS), 0, s, nullptr, w, b, n, eps, out, t, r, rb, index); break;
    case FMT_F16: hipLaunchKernelGGL((layernorm_kernel<FMT_F16>), dim3(1), dim3(LN_THREADS), 0, s, nullptr, w, b, n, eps, out, t, r, rb, index); break;
    case FMT_F32: hipLaunchKernelGGL((layernorm_kernel<FMT_F32>), dim3(1), dim3(LN_THREADS), 0, s, nullptr, w, b, n, eps, out, t, r, rb, index); break;
    default: return hipErrorInvalidValue;
    }
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
