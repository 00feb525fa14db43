// Batched prefill product Y[m, n] = sum_k X[m, k] * W[n, k] on MFMA.
//
// W is a GGUF matrix [N, K] (Q4_0, Q8_0, Q4_K, or F16 / F32 with K a
// multiple of 32), X holds M
// token rows of bf16 activations [M, K], Y is FP32 [M, N] (one output row per
// token), FP32 accumulation.  Reference semantics: the transpose_right branch
// of CpuInstructionNumerics.MatrixMultiply
// (SharpInference.Instructions.Cpu/CpuInstructionNumerics.cs:66-77), i.e. one
// core.mat-vec per token row, and the batched prefill matvec of the D3D12
// transformer program (GpuBatchTransformerInstructions.cs:224-279), whose B=16
// token batch re-reads W per token.  Here every W element is decoded once per
// workgroup tile of 64, 128 or 256 tokens:
//
//   * a workgroup (4 waves) owns 32*NT rows of W and 4*MW token rows of X;
//   * per step of two 32-column blocks, the 256 threads decode the blocks of
//     each W row exactly as the CPU decoder does (FP32, one rounding per
//     operation), round them to bf16 and write a double-buffered LDS tile;
//     the raw bytes are loaded a step ahead;
//   * the workgroup's X tile of the step is loaded with coalesced 16-byte
//     loads (8 lanes per 128-byte token row, a step ahead; X is small and
//     stays in L2) into a swizzled LDS tile;
//   * each wave multiplies its MW token rows by the tile with
//     v_mfma_f32_32x32x16_bf16 (MW/32 x NT accumulator tiles of 32 x 32
//     FP32), both fragments read from LDS;
//   * the tile is the largest whose grid still covers the 256 CUs; grids
//     of 3072 x 512 outputs use a 16 x 16 block form (prefill_m16_kernel
//     below) whose 96-row x 64-token tiles give one workgroup per CU.
//
// Loading the fragments straight from global memory instead (each load
// instruction then spans 32 token or W rows, 32 cache lines) measured about
// half the speed of this form: the address / tag work of such loads, not
// the matrix cores or the decode, bounds it.  In this form the LDS fragment
// reads and the tile stores take most of the time; the matrix-core work is
// hidden under them.
//
// MFMA fragment layout (32x32x16 bf16): lane l holds A[l % 32][8*(l/32)+e]
// and B[8*(l/32)+e][l % 32] for e = 0..7; accumulator register r of lane l
// is C[8*(r/4) + 4*(l/32) + r%4][l % 32].
#include "si_internal.hpp"

#include <algorithm>

#include <hip/hip_fp16.h>

namespace si {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));   // 16 raw bytes

constexpr int PF_THREADS = 256;
// LDS W tile rows of 32 bf16 (four 16-byte chunks).  Padded: a row takes
// 40 bf16.  Compact (used when two workgroups share a CU, to fit two in
// 160 KiB): a row takes 32 bf16 and chunk c sits at c ^ ((r / 4) % 4).
// Both keep the fragment reads (32 consecutive rows, one chunk) and the
// decode stores free of bank conflicts; the padded form measured faster
// when a workgroup has its CU to itself.
template <bool COMPACT>
constexpr int ws_stride() { return COMPACT ? 32 : 40; }
template <bool COMPACT>
__device__ __forceinline__ int ws_off(int r, int c)
{
    return COMPACT ? r * 32 + 8 * (c ^ ((r >> 2) & 3)) : r * 40 + 8 * c;
}
constexpr int PF_DEPTH = 2;         // steps of loads in flight (even: LDS buffer = step parity)

// Raw words of one item of 16 values (half a 32-value block of one W row),
// loaded steps ahead of their decode.  The loads are plain word loads and
// every bit extraction happens at decode time, so a word in flight is never
// touched before its decode.  An F32 item is 16 words, every other format's
// at most 8.
template <int FMT>
struct RawW {
    uint32_t w[FMT == FMT_F32 ? 16 : 8];
};

typedef uint32_t u32_a2 __attribute__((aligned(2)));   // 4 bytes at a 2-byte aligned address

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p)
{
    return *reinterpret_cast<const unsigned short*>(p);
}
__device__ __forceinline__ uint32_t ld_u32_a2(const uint8_t* p) { return *reinterpret_cast<const u32_a2*>(p); }
__device__ __forceinline__ uint32_t ld_u32(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }

// Hides a value from the optimiser: keeps a 32-bit lane offset from being
// widened to 64 bits outside the loop (so loads keep the scalar-base
// addressing form), and keeps the known-zero bits of a masked word hidden
// (so each byte converts with one v_cvt_f32_ubyteN).
__device__ __forceinline__ uint32_t opaque(uint32_t v)
{
    asm("" : "+v"(v));
    return v;
}

// Loads address a block through a workgroup-uniform base (W plus the
// block's offset in a row) and a 32-bit lane offset (the row's offset), so
// they use the scalar-base addressing form and need no 64-bit vector
// address arithmetic.  Item h of a block:
//   Q4_0 {fp16 d; u8 qs[16]}: d and bytes 8h..8h+7 (elements 8h..8h+7 in the
//        low nibbles, 16+8h..16+8h+7 in the high nibbles);
//   Q8_0 {fp16 d; int8 q[32]}: d and q[16h..16h+15];
//   Q4_K {fp16 d, dmin; u8 scales[12]; u8 qs[128]} (16-byte aligned
//        super-blocks), sub-block j = blk % 8: d | dmin << 16, the three
//        scale words and the 16 quant bytes of elements 16h..16h+15 (nibble
//        j % 2 of qs[32 (j / 2) + 16h ..]).
template <int FMT>
__device__ __forceinline__ RawW<FMT> load_raw(const uint8_t* W, uint32_t row_off, int blk, int h);

template <>
__device__ __forceinline__ RawW<FMT_Q4_0> load_raw<FMT_Q4_0>(const uint8_t* W, uint32_t row_off, int blk, int h)
{
    const uint8_t* b = W + blk * 18;
    row_off = opaque(row_off);
    RawW<FMT_Q4_0> r;
    r.w[0] = ld_u16(b + row_off);
    r.w[1] = ld_u32_a2(b + (row_off + 2 + 8 * h));
    r.w[2] = ld_u32_a2(b + (row_off + 6 + 8 * h));
    return r;
}

template <>
__device__ __forceinline__ RawW<FMT_Q8_0> load_raw<FMT_Q8_0>(const uint8_t* W, uint32_t row_off, int blk, int h)
{
    const uint8_t* b = W + blk * 34;
    row_off = opaque(row_off);
    RawW<FMT_Q8_0> r;
    r.w[0] = ld_u16(b + row_off);
#pragma unroll
    for (int k = 0; k < 4; k++)
        r.w[1 + k] = ld_u32_a2(b + (row_off + 2 + 16 * h + 4 * k));
    return r;
}

template <>
__device__ __forceinline__ RawW<FMT_Q4_K> load_raw<FMT_Q4_K>(const uint8_t* W, uint32_t row_off, int blk, int h)
{
    const uint8_t* b = W + (blk >> 3) * 144;
    const int j = blk & 7;
    row_off = opaque(row_off);
    RawW<FMT_Q4_K> r;
    r.w[0] = ld_u32(b + row_off);
    r.w[1] = ld_u32(b + (row_off + 4));
    r.w[2] = ld_u32(b + (row_off + 8));
    r.w[3] = ld_u32(b + (row_off + 12));
#pragma unroll
    for (int k = 0; k < 4; k++)
        r.w[4 + k] = ld_u32(b + 16 + 32 * (j >> 1) + (row_off + 16 * h + 4 * k));
    return r;
}

// F16 / F32 (dense rows, a "block" is 32 consecutive elements): item h is
// elements 16h..16h+15, 8 words (F16) or 16 words (F32).
template <>
__device__ __forceinline__ RawW<FMT_F16> load_raw<FMT_F16>(const uint8_t* W, uint32_t row_off, int blk, int h)
{
    const uint8_t* b = W + blk * 64 + 32 * h;
    row_off = opaque(row_off);
    RawW<FMT_F16> r;
#pragma unroll
    for (int k = 0; k < 8; k++)
        r.w[k] = ld_u32(b + (row_off + 4 * k));
    return r;
}

template <>
__device__ __forceinline__ RawW<FMT_F32> load_raw<FMT_F32>(const uint8_t* W, uint32_t row_off, int blk, int h)
{
    const uint8_t* b = W + blk * 128 + 64 * h;
    row_off = opaque(row_off);
    RawW<FMT_F32> r;
#pragma unroll
    for (int k = 0; k < 16; k++)
        r.w[k] = ld_u32(b + (row_off + 4 * k));
    return r;
}

__device__ __forceinline__ float half_bits(uint32_t h)
{
    return __half2float(__ushort_as_half(static_cast<unsigned short>(h & 0xffffu)));
}

// Byte i of q as a float (v_cvt_f32_ubyteN).
__device__ __forceinline__ float ubyte(uint32_t q, int i) { return static_cast<float>((q >> (8 * i)) & 0xffu); }

// 8 values fma(a, byte, c) of two words, rounded to bf16 (RNE).
__device__ __forceinline__ bf16x8 decode8(uint32_t q0, uint32_t q1, float a, float c)
{
    f32x8 v;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[i] = fmaf(a, ubyte(q0, i), c);
        v[4 + i] = fmaf(a, ubyte(q1, i), c);
    }
    return __builtin_convertvector(v, bf16x8);
}

// The 16 values of an item in FP32 are bit-identical to the block decoder,
// each one fused multiply-add whose exact result needs no rounding or
// equals the decoder's single rounding:
//   Q8_0: d * q = fma(d, q + 128, -128 d)   (d * (q + 128) and 128 d exact)
//   Q4_0: d * (q - 8) = fma(d, q, -8 d)      (every term exact)
//   Q4_K: (d sc) q - dmin m = fma(d1, q, -m1) with d1 = d sc and m1 = dmin m
//         exact (11-bit by 6-bit products), d1 q exact, one rounding.
// High nibbles are masked in place (16 q per byte) and the factor 1/16 goes
// into the scale, which stays exact (a power of two).  The two halves of
// 8 values go to columns c0 and c1 of the block.
template <int FMT>
__device__ __forceinline__ void decode_raw(const RawW<FMT>& r, int blk, int h, bf16x8& v0, bf16x8& v1, int& c0,
                                           int& c1);

template <>
__device__ __forceinline__ void decode_raw<FMT_Q4_0>(const RawW<FMT_Q4_0>& r, int, int h, bf16x8& v0, bf16x8& v1, int& c0,
                                                     int& c1)
{
    const float d = half_bits(r.w[0]);
    const float c = -8.0f * d;
    v0 = decode8(opaque(r.w[1] & 0x0f0f0f0fu), opaque(r.w[2] & 0x0f0f0f0fu), d, c);
    v1 = decode8(opaque(r.w[1] & 0xf0f0f0f0u), opaque(r.w[2] & 0xf0f0f0f0u), d * 0.0625f, c);
    c0 = 8 * h;
    c1 = 16 + 8 * h;
}

template <>
__device__ __forceinline__ void decode_raw<FMT_Q8_0>(const RawW<FMT_Q8_0>& r, int, int h, bf16x8& v0, bf16x8& v1, int& c0,
                                                     int& c1)
{
    const float d = half_bits(r.w[0]);
    const float c = -128.0f * d;
    v0 = decode8(opaque(r.w[1] ^ 0x80808080u), opaque(r.w[2] ^ 0x80808080u), d, c);   // q + 128 as unsigned bytes
    v1 = decode8(opaque(r.w[3] ^ 0x80808080u), opaque(r.w[4] ^ 0x80808080u), d, c);
    c0 = 16 * h;
    c1 = 16 * h + 8;
}

// 6-bit scale and min of sub-block j (GGML get_scale_min_k4) from the
// scale words lo = scales[0..3], mid = scales[4..7], hi = scales[8..11].
template <>
__device__ __forceinline__ void decode_raw<FMT_Q4_K>(const RawW<FMT_Q4_K>& r, int blk, int h, bf16x8& v0, bf16x8& v1, int& c0,
                                                     int& c1)
{
    const int j = blk & 7;
    const float d = half_bits(r.w[0]), dmin = half_bits(r.w[0] >> 16);
    const int sh = 8 * (j & 3);
    const uint32_t lo = (r.w[1] >> sh) & 0xffu, mid = (r.w[2] >> sh) & 0xffu, hi = (r.w[3] >> sh) & 0xffu;
    int sc, m;
    if (j < 4) {
        sc = static_cast<int>(lo & 63u);
        m = static_cast<int>(mid & 63u);
    } else {
        sc = static_cast<int>((hi & 15u) | ((lo >> 6) << 4));
        m = static_cast<int>((hi >> 4) | ((mid >> 6) << 4));
    }
    const float d1 = __fmul_rn(d, static_cast<float>(sc));
    const float m1 = __fmul_rn(dmin, static_cast<float>(m));
    const bool high = (j & 1) != 0;
    const uint32_t mask = high ? 0xf0f0f0f0u : 0x0f0f0f0fu;
    const float a = high ? d1 * 0.0625f : d1;
    v0 = decode8(opaque(r.w[4] & mask), opaque(r.w[5] & mask), a, -m1);
    v1 = decode8(opaque(r.w[6] & mask), opaque(r.w[7] & mask), a, -m1);
    c0 = 16 * h;
    c1 = 16 * h + 8;
}

// F16: each value converted exactly to FP32, then rounded to bf16 (one
// rounding from the exact value).  F32: rounded to bf16.
template <>
__device__ __forceinline__ void decode_raw<FMT_F16>(const RawW<FMT_F16>& r, int, int h, bf16x8& v0, bf16x8& v1,
                                                    int& c0, int& c1)
{
    f32x8 a, b;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        a[2 * i] = half_bits(r.w[i]);
        a[2 * i + 1] = half_bits(r.w[i] >> 16);
        b[2 * i] = half_bits(r.w[4 + i]);
        b[2 * i + 1] = half_bits(r.w[4 + i] >> 16);
    }
    v0 = __builtin_convertvector(a, bf16x8);
    v1 = __builtin_convertvector(b, bf16x8);
    c0 = 16 * h;
    c1 = 16 * h + 8;
}

template <>
__device__ __forceinline__ void decode_raw<FMT_F32>(const RawW<FMT_F32>& r, int, int h, bf16x8& v0, bf16x8& v1,
                                                    int& c0, int& c1)
{
    f32x8 a, b;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        a[i] = __uint_as_float(r.w[i]);
        b[i] = __uint_as_float(r.w[8 + i]);
    }
    v0 = __builtin_convertvector(a, bf16x8);
    v1 = __builtin_convertvector(b, bf16x8);
    c0 = 16 * h;
    c1 = 16 * h + 8;
}

// Scheduling hint for one steady-state step: the step's matrix-core
// instructions are spread over the step, with the LDS fragment reads, the
// decode of the next step (vector ALU), its LDS stores and the loads of a
// later step placed between them, so a single wave keeps the matrix core
// busy while it decodes (the work of a step is independent of the next
// step's decode and stores, which go to the other LDS buffer).
template <int NMFMA>
__device__ __forceinline__ void interleave_step()
{
#pragma unroll
    for (int i = 0; i < NMFMA; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);   // vector ALU
    }
}

// MW token rows per wave (32 or 64: MW / 32 accumulator tiles along M),
// 4 * MW token rows and 32 * NT rows of W per workgroup tile, two
// 32-column blocks (64 columns) per step; KS groups of 4 waves split the
// steps of the tile (KS = 2: two waves per SIMD, whose LDS, decode and
// matrix-core phases overlap) and add their sums through LDS at the end.
//
//   * X: a group's 4 * MW x 64 bf16 tile of a step is loaded with
//     coalesced 16-byte loads (8 lanes per 128-byte token row) and stored
//     to LDS with its 16-byte chunks swizzled (chunk c of row r at
//     c ^ ((r >> 1) & 7)), so the MFMA fragment reads (32 rows, one chunk)
//     are free of bank conflicts;
//   * W: each lane loads the raw words of 16 values (half a block of one
//     row) and decodes them exactly into the group's bf16 LDS tile;
//   * both are loaded D steps ahead into a ring of register sets (the loop
//     is unrolled by D so each slot is one fixed register set) and written
//     to the other LDS buffer after the step's matrix-core work; one
//     barrier per step.
template <int FMT, int MW, int NT, int D, int KS, bool COMPACT>
__global__ __launch_bounds__(PF_THREADS * KS) void prefill_mfma_kernel(const uint8_t* __restrict__ W,
                                                                        const __bf16* __restrict__ X,
                                                                        float* __restrict__ Y, int M, int N, int K,
                                                                        int64_t row_bytes)
{
    constexpr int MT = MW / 32;                           // accumulator tiles along M per wave
    constexpr int NROWS = 32 * NT;                        // W rows per workgroup
    constexpr int TROWS = 4 * MW;                         // token rows per workgroup
    constexpr int BPS = 2;                                // 32-column blocks per step
    constexpr int WI = NROWS * BPS * 2 / PF_THREADS;      // 16-value W items per thread per step
    constexpr int XL = TROWS * 8 / PF_THREADS;            // 16-byte X chunks per thread per step
    static_assert(WI >= 1 && WI * PF_THREADS == NROWS * BPS * 2, "whole W items per thread");
    static_assert(D % 2 == 0, "ring groups start on even steps, so a slot's LDS buffer is fixed");
    static_assert(XL * PF_THREADS == TROWS * 8, "whole X chunks per thread");
    static_assert(KS == 1 || KS * 2 * TROWS * 8 * 16 >= PF_THREADS * (KS - 1) * MT * NT * 16 * 4,
                  "the X buffers hold the partial sums of the other step groups");
    __shared__ __attribute__((aligned(16))) __bf16 ws[KS][2][BPS][NROWS * ws_stride<COMPACT>()];
    __shared__ __attribute__((aligned(16))) u32x4 xs[KS][2][TROWS * 8];

    const int t = threadIdx.x % PF_THREADS;              // thread within the step group
    const int kh = threadIdx.x / PF_THREADS;             // step group
    const int lane = t & 63;
    const int wave = t >> 6;
    const int n0 = blockIdx.x * NROWS;
    const int mw0 = blockIdx.y * TROWS;                  // first token row of the workgroup
    const int m0 = mw0 + wave * MW;                       // first token row of this wave
    const int g = lane >> 5;          // K group of the fragment (0, 1)
    const int li = lane & 31;
    const int nblk = K / 32;
    const int nsteps_all = (nblk + BPS - 1) / BPS;
    const int nsteps = (nsteps_all + KS - 1) / KS;       // steps of each group (the launcher makes KS divide)
    const int step0 = kh * nsteps;

    // this thread's X chunks: token row, 16-byte chunk
    uint32_t xoff[XL];                                    // byte offset of the token row
    int xdst[XL];
    const int xcol = 8 * (t & 7);                         // the same chunk column for every e
#pragma unroll
    for (int e = 0; e < XL; e++) {
        const int item = t + e * PF_THREADS;
        const int r = item >> 3, c = item & 7;
        xoff[e] = static_cast<uint32_t>(min(mw0 + r, M - 1)) * static_cast<uint32_t>(2 * K);
        xdst[e] = r * 8 + (c ^ ((r >> 1) & 7));
    }
    const uint8_t* xbytes = reinterpret_cast<const uint8_t*>(X);

    // W item i of this thread: idx = t + 256 i -> half h = idx % 2, block
    // bo = (idx / 2) % 2 of the step, tile row idx / 4 (4 consecutive lanes
    // cover one row's two blocks)
    uint32_t wrow[WI];                                    // byte offset of the W row
#pragma unroll
    for (int i = 0; i < WI; i++) {
        const int r = (t + i * PF_THREADS) >> 2;
        wrow[i] = static_cast<uint32_t>(min(n0 + r, N - 1)) * static_cast<uint32_t>(row_bytes);
    }
    const int wh = t & 1, wbo = (t >> 1) & 1;

    f32x16 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
            acc[mt][nt] = f32x16{};

    // ring slot s % D holds the W words and X chunks of local step s
    RawW<FMT> raw[D][WI];
    u32x4 xr[D][XL];
    auto load_step = [&](int ls, RawW<FMT> (&wdst)[WI], u32x4 (&xdst_regs)[XL]) {
        const int step = step0 + ls;
        const int blk = min(BPS * step + wbo, nblk - 1);
#pragma unroll
        for (int i = 0; i < WI; i++)
            wdst[i] = load_raw<FMT>(W, wrow[i], blk, wh);
        // columns past K (the second block of a partial last step) re-read
        // the row's last chunk; their MFMAs are skipped
        const int col = min(BPS * 32 * step + xcol, K - 8);
#pragma unroll
        for (int e = 0; e < XL; e++)
            xdst_regs[e] = *reinterpret_cast<const u32x4*>(xbytes + (xoff[e] + static_cast<uint32_t>(2 * col)));
    };
    auto store_step = [&](int ls, const RawW<FMT> (&wsrc)[WI], const u32x4 (&xsrc_regs)[XL], int buf) {
        const int blk = min(BPS * (step0 + ls) + wbo, nblk - 1);
#pragma unroll
        for (int i = 0; i < WI; i++) {
            bf16x8 v0, v1;
            int c0, c1;
            decode_raw<FMT>(wsrc[i], blk, wh, v0, v1, c0, c1);
            const int r = (t + i * PF_THREADS) >> 2;
            *reinterpret_cast<bf16x8*>(&ws[kh][buf][wbo][ws_off<COMPACT>(r, c0 >> 3)]) = v0;
            *reinterpret_cast<bf16x8*>(&ws[kh][buf][wbo][ws_off<COMPACT>(r, c1 >> 3)]) = v1;
        }
#pragma unroll
        for (int e = 0; e < XL; e++)
            xs[kh][buf][xdst[e]] = xsrc_regs[e];
    };
    // matrix-core work of one local step from LDS buffer buf (= ls & 1);
    // only the last step of all can hold a block past K (guarded)
    auto mfma_step = [&](int ls, int buf, bool guarded) {
        const int step = step0 + ls;
#pragma unroll
        for (int bo = 0; bo < BPS; bo++) {
            if (!guarded || BPS * step + bo < nblk) {
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int c = 4 * bo + 2 * h + g;   // 16-byte chunk of the fragment
                    bf16x8 a[MT];
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) {
                        const int r = wave * MW + 32 * mt + li;
                        a[mt] = *reinterpret_cast<const bf16x8*>(&xs[kh][buf][r * 8 + (c ^ ((r >> 1) & 7))]);
                    }
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) {
                        const bf16x8 b = *reinterpret_cast<const bf16x8*>(
                            &ws[kh][buf][bo][ws_off<COMPACT>(32 * nt + li, 2 * h + g)]);
#pragma unroll
                        for (int mt = 0; mt < MT; mt++)
                            acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[mt], b, acc[mt][nt], 0, 0, 0);
                    }
                }
            }
        }
    };

    // prologue: local step 0 in LDS; steps 1..D in flight
    {
        RawW<FMT> w0[WI];
        u32x4 x0[XL];
        load_step(0, w0, x0);
#pragma unroll
        for (int u = 0; u < D; u++)
            load_step(min(u + 1, nsteps - 1), raw[(u + 1) % D], xr[(u + 1) % D]);
        store_step(0, w0, x0, 0);
    }
    __syncthreads();
    // Steady state: every step of a group has a successor and the loads are
    // unconditional (clamped step indexes), so each ring slot stays one
    // register set across the loop and no load is waited for early.
    int base = 0;
    for (; base + D < nsteps; base += D) {
#pragma unroll
        for (int u = 0; u < D; u++) {
            const int ls = base + u;
            const int next = (u + 1) % D;   // constant after unrolling
            mfma_step(ls, u & 1, false);                 // D is even: the buffers are constants
            store_step(ls + 1, raw[next], xr[next], (u + 1) & 1);
            load_step(min(ls + 1 + D, nsteps - 1), raw[next], xr[next]);
            interleave_step<BPS * 2 * MT * NT>();
            __syncthreads();
        }
    }
    // the last (at most D) steps: their loads are already in flight
#pragma unroll
    for (int u = 0; u < D; u++) {
        const int ls = base + u;
        if (ls < nsteps) {
            mfma_step(ls, u & 1, true);
            if (ls + 1 < nsteps)
                store_step(ls + 1, raw[(u + 1) % D], xr[(u + 1) % D], (u + 1) & 1);
            __syncthreads();
        }
    }

    // the other step groups add their sums into group 0 through LDS (the X
    // buffers are free after the last barrier)
    if constexpr (KS > 1) {
        float* red = reinterpret_cast<float*>(&xs[0][0][0]);
        constexpr int PER = MT * NT * 16;
        if (kh > 0) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        red[((kh - 1) * PER + (mt * NT + nt) * 16 + r) * PF_THREADS + t] = acc[mt][nt][r];
        }
        __syncthreads();
        if (kh > 0)
            return;
#pragma unroll
        for (int o = 1; o < KS; o++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        acc[mt][nt][r] += red[((o - 1) * PER + (mt * NT + nt) * 16 + r) * PF_THREADS + t];
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

// Warp-specialised form: 4 consumer waves issue only LDS fragment reads and
// MFMAs (wave w owns MW tokens x all 32 * NT rows of the tile), while 4
// producer waves load the raw W words and X chunks D steps ahead and decode
// / store the next step into the other LDS buffer, so a SIMD runs one
// wave's matrix-core work and another wave's decode at the same time.  One
// barrier per step; the same exact W decode and swizzled layouts as the
// kernel above.
//
// Split K (splits > 1, for grids with fewer tiles than CUs): workgroup z
// takes a contiguous range of the steps and stores its FP32 tile to `part`
// (the tile's slot of split z); prefill_reduce_kernel then adds each
// output's partial sums in split order 0, 1, ... (a fixed order, so results
// are reproducible run to run) and writes Y.
template <int FMT, int MW, int NT, int D>
__global__ __launch_bounds__(2 * PF_THREADS) void prefill_ws_kernel(const uint8_t* __restrict__ W,
                                                                    const __bf16* __restrict__ X,
                                                                    float* __restrict__ Y, int M, int N, int K,
                                                                    int64_t row_bytes, int splits,
                                                                    float4* __restrict__ part)
{
    constexpr int MT = MW / 32;
    constexpr int NROWS = 32 * NT;
    constexpr int TROWS = 4 * MW;
    constexpr int BPS = 2;
    constexpr int WI = NROWS * BPS * 2 / PF_THREADS;      // W items per producer thread per step
    constexpr int XL = TROWS * 8 / PF_THREADS;            // X chunks per producer thread per step
    static_assert(WI >= 1 && WI * PF_THREADS == NROWS * BPS * 2, "whole W items per thread");
    static_assert(XL * PF_THREADS == TROWS * 8, "whole X chunks per thread");
    static_assert(D % 2 == 0, "ring groups start on even steps, so a slot's LDS buffer is fixed");
    __shared__ __attribute__((aligned(16))) __bf16 ws[2][BPS][NROWS * ws_stride<true>()];
    __shared__ __attribute__((aligned(16))) u32x4 xs[2][TROWS * 8];

    // the role is the same for a whole wave; readfirstlane makes that
    // visible, so each wave runs one branch and both branches execute the
    // same sequence of barriers (1 + one per step)
    const bool consumer = __builtin_amdgcn_readfirstlane(threadIdx.x) < PF_THREADS;
    const int t = threadIdx.x % PF_THREADS;
    const int lane = t & 63, wave = t >> 6;
    const int n0 = blockIdx.x * NROWS;
    const int mw0 = blockIdx.y * TROWS;
    const int g = lane >> 5, li = lane & 31;
    const int nblk = K / 32;
    // this workgroup's steps: [s0, s0 + nsteps) of the K range (the
    // launcher keeps every split non-empty)
    const int steps_all = (nblk + BPS - 1) / BPS;
    const int per = (steps_all + splits - 1) / splits;
    const int s0 = static_cast<int>(blockIdx.z) * per;
    const int nsteps = min(per, steps_all - s0);
    constexpr int TILE4 = PF_THREADS * MT * NT * 4;       // float4 values of a tile's FP32 sums
    const int tile = blockIdx.x + gridDim.x * blockIdx.y;

    if (consumer) {
        f32x16 acc[MT][NT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int nt = 0; nt < NT; nt++)
                acc[mt][nt] = f32x16{};
        auto mfma_step = [&](int step, int buf, bool guarded) {
#pragma unroll
            for (int bo = 0; bo < BPS; bo++) {
                if (!guarded || BPS * (s0 + step) + bo < nblk) {
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const int c = 4 * bo + 2 * h + g;
                        bf16x8 a[MT], b[NT];
#pragma unroll
                        for (int mt = 0; mt < MT; mt++) {
                            const int r = wave * MW + 32 * mt + li;
                            a[mt] = *reinterpret_cast<const bf16x8*>(&xs[buf][r * 8 + (c ^ ((r >> 1) & 7))]);
                        }
#pragma unroll
                        for (int nt = 0; nt < NT; nt++)
                            b[nt] = *reinterpret_cast<const bf16x8*>(
                                &ws[buf][bo][ws_off<true>(32 * nt + li, 2 * h + g)]);
#pragma unroll
                        for (int nt = 0; nt < NT; nt++)
#pragma unroll
                            for (int mt = 0; mt < MT; mt++)
                                acc[mt][nt] =
                                    __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[mt], b[nt], acc[mt][nt], 0, 0, 0);
                    }
                }
            }
        };
        __syncthreads();                                  // step 0 stored
        int base = 0;
        for (; base + D < nsteps; base += D) {
#pragma unroll
            for (int u = 0; u < D; u++) {
                mfma_step(base + u, u & 1, false);
                __syncthreads();
            }
        }
#pragma unroll
        for (int u = 0; u < D; u++) {
            if (base + u < nsteps) {
                mfma_step(base + u, u & 1, true);
                __syncthreads();
            }
        }
        if (splits > 1) {
            // this split's sums: float4 j * 256 + t holds registers 4 (j % 4) ..
            // of accumulator tile j / 4 = mt * NT + nt of thread t
            float4* dst = part + (static_cast<int64_t>(tile) * splits + blockIdx.z) * TILE4;
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
#pragma unroll
                    for (int r4 = 0; r4 < 4; r4++) {
                        const f32x16& a = acc[mt][nt];
                        dst[((mt * NT + nt) * 4 + r4) * PF_THREADS + t] =
                            make_float4(a[4 * r4], a[4 * r4 + 1], a[4 * r4 + 2], a[4 * r4 + 3]);
                    }
        } else {
            const int m0 = mw0 + wave * MW;
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
    } else {
        uint32_t xoff[XL];
        int xdst[XL];
        const int xcol = 8 * (t & 7);
#pragma unroll
        for (int e = 0; e < XL; e++) {
            const int item = t + e * PF_THREADS;
            const int r = item >> 3, c = item & 7;
            xoff[e] = static_cast<uint32_t>(min(mw0 + r, M - 1)) * static_cast<uint32_t>(2 * K);
            xdst[e] = r * 8 + (c ^ ((r >> 1) & 7));
        }
        const uint8_t* xbytes = reinterpret_cast<const uint8_t*>(X);
        uint32_t wrow[WI];
#pragma unroll
        for (int i = 0; i < WI; i++) {
            const int r = (t + i * PF_THREADS) >> 2;
            wrow[i] = static_cast<uint32_t>(min(n0 + r, N - 1)) * static_cast<uint32_t>(row_bytes);
        }
        const int wh = t & 1, wbo = (t >> 1) & 1;
        RawW<FMT> raw[D][WI];
        u32x4 xr[D][XL];
        auto load_step = [&](int step, RawW<FMT> (&wdst)[WI], u32x4 (&xdst_regs)[XL]) {
            const int blk = min(BPS * (s0 + step) + wbo, nblk - 1);
#pragma unroll
            for (int i = 0; i < WI; i++)
                wdst[i] = load_raw<FMT>(W, wrow[i], blk, wh);
            const int col = min(BPS * 32 * (s0 + step) + xcol, K - 8);
#pragma unroll
            for (int e = 0; e < XL; e++)
                xdst_regs[e] = *reinterpret_cast<const u32x4*>(xbytes + (xoff[e] + static_cast<uint32_t>(2 * col)));
        };
        auto store_step = [&](int step, const RawW<FMT> (&wsrc)[WI], const u32x4 (&xsrc_regs)[XL], int buf) {
            const int blk = min(BPS * (s0 + step) + wbo, nblk - 1);
#pragma unroll
            for (int i = 0; i < WI; i++) {
                bf16x8 v0, v1;
                int c0, c1;
                decode_raw<FMT>(wsrc[i], blk, wh, v0, v1, c0, c1);
                const int r = (t + i * PF_THREADS) >> 2;
                *reinterpret_cast<bf16x8*>(&ws[buf][wbo][ws_off<true>(r, c0 >> 3)]) = v0;
                *reinterpret_cast<bf16x8*>(&ws[buf][wbo][ws_off<true>(r, c1 >> 3)]) = v1;
            }
#pragma unroll
            for (int e = 0; e < XL; e++)
                xs[buf][xdst[e]] = xsrc_regs[e];
        };
        {
            RawW<FMT> w0[WI];
            u32x4 x0[XL];
            load_step(0, w0, x0);
#pragma unroll
            for (int u = 0; u < D; u++)
                load_step(min(u + 1, nsteps - 1), raw[(u + 1) % D], xr[(u + 1) % D]);
            store_step(0, w0, x0, 0);
        }
        __syncthreads();                                  // step 0 stored
        int base = 0;
        for (; base + D < nsteps; base += D) {
#pragma unroll
            for (int u = 0; u < D; u++) {
                const int next = (u + 1) % D;
                store_step(base + u + 1, raw[next], xr[next], (u + 1) & 1);
                load_step(min(base + u + 1 + D, nsteps - 1), raw[next], xr[next]);
                __syncthreads();
            }
        }
#pragma unroll
        for (int u = 0; u < D; u++) {
            if (base + u < nsteps) {
                if (base + u + 1 < nsteps)
                    store_step(base + u + 1, raw[(u + 1) % D], xr[(u + 1) % D], (u + 1) & 1);
                __syncthreads();
            }
        }
    }
}

// Sums the split-K partials of prefill_ws_kernel in split order and writes
// Y: thread i of the grid takes float4 i % TILE4 of tile i / TILE4 (the
// layout the kernel's consumer threads store).
template <int MW, int NT>
__global__ __launch_bounds__(PF_THREADS) void prefill_reduce_kernel(const float4* __restrict__ part,
                                                                    float* __restrict__ Y, int M, int N, int splits,
                                                                    int tiles_n)
{
    constexpr int MT = MW / 32;
    constexpr int TILE4 = PF_THREADS * MT * NT * 4;
    const int64_t gi = static_cast<int64_t>(blockIdx.x) * PF_THREADS + threadIdx.x;
    const int tile = static_cast<int>(gi / TILE4), i = static_cast<int>(gi % TILE4);
    const float4* src = part + static_cast<int64_t>(tile) * splits * TILE4 + i;
    float4 v = src[0];
    for (int q = 1; q < splits; q++) {
        const float4 w = src[static_cast<int64_t>(q) * TILE4];
        v.x += w.x;
        v.y += w.y;
        v.z += w.z;
        v.w += w.w;
    }
    // float4 i = registers 4 r4 .. of accumulator tile (mt, nt) of consumer thread ct
    const int ct = i % PF_THREADS, j = i / PF_THREADS;
    const int r4 = j & 3, tnt = (j >> 2) % NT, tmt = (j >> 2) / NT;
    const int cw = ct >> 6, cl = ct & 63;
    const int n = (tile % tiles_n) * 32 * NT + 32 * tnt + (cl & 31);
    const int m = (tile / tiles_n) * 4 * MW + cw * MW + 32 * tmt + 8 * r4 + 4 * (cl >> 5);
    if (n < N) {
        if (m < M) Y[static_cast<int64_t>(m) * N + n] = v.x;
        if (m + 1 < M) Y[static_cast<int64_t>(m + 1) * N + n] = v.y;
        if (m + 2 < M) Y[static_cast<int64_t>(m + 2) * N + n] = v.z;
        if (m + 3 < M) Y[static_cast<int64_t>(m + 3) * N + n] = v.w;
    }
}

// 16 x 16 x 32 block form (v_mfma_f32_16x16x32_bf16; lane l holds
// A[l % 16][8 * (l / 16) + e], B[8 * (l / 16) + e][l % 16] and D rows
// 4 * (l / 16) + r of column l % 16, as checked on the GPU).  A group of 4
// waves in a 2 x 2 layout: wave (wn, wm) owns 16*WN W rows x 16*WM tokens of
// the 32*WN x 32*WM tile, so tiles such as 96 rows x 64 tokens give 256
// workgroups for a 3072 x 512 product (one per CU, where the 32 x 32 form
// above leaves a quarter of the CUs idle).  A step covers BPS blocks; KS
// groups of 4 waves split the steps (two waves per SIMD) and add through
// LDS.  The W and X tiles are stored as 16-byte chunks, chunk c of row r at
// c ^ (r & 15) (16 chunks a row) or c ^ ((r >> 1) & 7) (8 chunks), so the
// fragment reads (16 rows, one chunk) are free of bank conflicts.  Same
// exact decode, ring of D steps in flight and one barrier per step as the
// kernels above.
template <int BPS>
__device__ __forceinline__ int m16_off(int r, int c)
{
    constexpr int CPR = 4 * BPS;
    return r * CPR + (CPR == 8 ? (c ^ ((r >> 1) & 7)) : (c ^ (r & 15)));
}

template <int FMT, int WN, int WM, int BPS, int D, int KS>
__global__ __launch_bounds__(PF_THREADS * KS) void prefill_m16_kernel(const uint8_t* __restrict__ W,
                                                                       const __bf16* __restrict__ X,
                                                                       float* __restrict__ Y, int M, int N, int K,
                                                                       int64_t row_bytes)
{
    constexpr int NROWS = 32 * WN, TROWS = 32 * WM, CPR = 4 * BPS;
    constexpr int WI = NROWS * BPS * 2 / PF_THREADS;      // 16-value W items per thread per step
    constexpr int XL = TROWS * CPR / PF_THREADS;          // 16-byte X chunks per thread per step
    static_assert(WI * PF_THREADS == NROWS * BPS * 2 && XL * PF_THREADS == TROWS * CPR, "whole items per thread");
    static_assert(BPS == 2 || BPS == 4, "8 or 16 chunks a row");
    static_assert(D % 2 == 0, "ring groups start on even steps, so a slot's LDS buffer is fixed");
    constexpr int GROUP_CHUNKS = 2 * (NROWS + TROWS) * CPR;   // a step group's double-buffered W and X tiles
    static_assert((KS - 1) * WM * WN * 4 * PF_THREADS * 4 <= KS * GROUP_CHUNKS * 16, "the partial sums fit");
    __shared__ __attribute__((aligned(16))) u32x4 pool[KS * GROUP_CHUNKS];

    const int t = threadIdx.x % PF_THREADS, kh = threadIdx.x / PF_THREADS;
    const int lane = t & 63, wave = t >> 6;
    const int wn = wave & 1, wm = wave >> 1;
    const int li = lane & 15, lg = lane >> 4;
    const int n0 = blockIdx.x * NROWS, m0 = blockIdx.y * TROWS;
    const int nsteps = K / (32 * BPS) / KS;              // the launcher makes 32 * BPS * KS divide K
    const int step0 = kh * nsteps;
    u32x4* const gbase = pool + kh * GROUP_CHUNKS;
    auto wt = [&](int buf) { return gbase + buf * NROWS * CPR; };
    auto xt = [&](int buf) { return gbase + 2 * NROWS * CPR + buf * TROWS * CPR; };

    // X chunk e of this thread: token row item / CPR, chunk item % CPR
    uint32_t xoff[XL];
    int xdst[XL];
    const int xc = t % CPR;
#pragma unroll
    for (int e = 0; e < XL; e++) {
        const int r = (t + PF_THREADS * e) / CPR;
        xoff[e] = static_cast<uint32_t>(min(m0 + r, M - 1)) * static_cast<uint32_t>(2 * K) + 16u * xc;
        xdst[e] = m16_off<BPS>(r, xc);
    }
    const uint8_t* xbytes = reinterpret_cast<const uint8_t*>(X);
    // W item i: half t % 2 of block (t / 2) % BPS of tile row (t + 256 i) / (2 BPS)
    uint32_t wrow[WI];
    int wr[WI];
#pragma unroll
    for (int i = 0; i < WI; i++) {
        wr[i] = (t + PF_THREADS * i) / (2 * BPS);
        wrow[i] = static_cast<uint32_t>(min(n0 + wr[i], N - 1)) * static_cast<uint32_t>(row_bytes);
    }
    const int wh = t & 1, wbo = (t >> 1) % BPS;

    f32x4 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++)
            acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    RawW<FMT> raw[D][WI];
    u32x4 xr[D][XL];
    auto load_step = [&](int ls, RawW<FMT> (&wd)[WI], u32x4 (&xd)[XL]) {
        const int step = step0 + ls;
        const int blk = BPS * step + wbo;
#pragma unroll
        for (int i = 0; i < WI; i++)
            wd[i] = load_raw<FMT>(W, wrow[i], blk, wh);
        const uint32_t col_bytes = static_cast<uint32_t>(64 * BPS * step);
#pragma unroll
        for (int e = 0; e < XL; e++)
            xd[e] = *reinterpret_cast<const u32x4*>(xbytes + (xoff[e] + col_bytes));
    };
    auto store_step = [&](int ls, const RawW<FMT> (&wsrc)[WI], const u32x4 (&xsrc)[XL], int buf) {
        const int blk = BPS * (step0 + ls) + wbo;
#pragma unroll
        for (int i = 0; i < WI; i++) {
            bf16x8 v0, v1;
            int c0, c1;
            decode_raw<FMT>(wsrc[i], blk, wh, v0, v1, c0, c1);
            *reinterpret_cast<bf16x8*>(wt(buf) + m16_off<BPS>(wr[i], 4 * wbo + (c0 >> 3))) = v0;
            *reinterpret_cast<bf16x8*>(wt(buf) + m16_off<BPS>(wr[i], 4 * wbo + (c1 >> 3))) = v1;
        }
#pragma unroll
        for (int e = 0; e < XL; e++)
            xt(buf)[xdst[e]] = xsrc[e];
    };
    auto mfma_step = [&](int buf) {
#pragma unroll
        for (int kk = 0; kk < BPS; kk++) {
            const int c = 4 * kk + lg;                     // the fragment's chunk of the step
            bf16x8 a[WM], b[WN];
#pragma unroll
            for (int i = 0; i < WM; i++)
                a[i] = *reinterpret_cast<const bf16x8*>(xt(buf) + m16_off<BPS>(16 * (WM * wm + i) + li, c));
#pragma unroll
            for (int j = 0; j < WN; j++)
                b[j] = *reinterpret_cast<const bf16x8*>(wt(buf) + m16_off<BPS>(16 * (WN * wn + j) + li, c));
#pragma unroll
            for (int i = 0; i < WM; i++)
#pragma unroll
                for (int j = 0; j < WN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    };

    // prologue: local step 0 in LDS; steps 1..D in flight
    {
        RawW<FMT> w0[WI];
        u32x4 x0[XL];
        load_step(0, w0, x0);
#pragma unroll
        for (int u = 0; u < D; u++)
            load_step(min(u + 1, nsteps - 1), raw[(u + 1) % D], xr[(u + 1) % D]);
        store_step(0, w0, x0, 0);
    }
    __syncthreads();
    int base = 0;
    for (; base + D < nsteps; base += D) {
#pragma unroll
        for (int u = 0; u < D; u++) {
            const int ls = base + u;
            const int next = (u + 1) % D;
            mfma_step(u & 1);
            store_step(ls + 1, raw[next], xr[next], (u + 1) & 1);
            load_step(min(ls + 1 + D, nsteps - 1), raw[next], xr[next]);
            interleave_step<BPS * WM * WN>();
            __syncthreads();
        }
    }
#pragma unroll
    for (int u = 0; u < D; u++) {
        const int ls = base + u;
        if (ls < nsteps) {
            mfma_step(u & 1);
            if (ls + 1 < nsteps)
                store_step(ls + 1, raw[(u + 1) % D], xr[(u + 1) % D], (u + 1) & 1);
            __syncthreads();
        }
    }

    // the other step groups add their sums into group 0 through LDS (every
    // tile read ended at the last barrier)
    if constexpr (KS > 1) {
        constexpr int PER = WM * WN * 4;
        float* red = reinterpret_cast<float*>(pool);
        if (kh > 0) {
#pragma unroll
            for (int i = 0; i < WM; i++)
#pragma unroll
                for (int j = 0; j < WN; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        red[((kh - 1) * PER + (i * WN + j) * 4 + r) * PF_THREADS + t] = acc[i][j][r];
        }
        __syncthreads();
        if (kh > 0)
            return;
#pragma unroll
        for (int o = 1; o < KS; o++)
#pragma unroll
            for (int i = 0; i < WM; i++)
#pragma unroll
                for (int j = 0; j < WN; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        acc[i][j][r] += red[((o - 1) * PER + (i * WN + j) * 4 + r) * PF_THREADS + t];
    }
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++) {
            const int n = n0 + 16 * (WN * wn + j) + li;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + 16 * (WM * wm + i) + 4 * lg + r;
                if (m < M && n < N)
                    Y[static_cast<int64_t>(m) * N + n] = acc[i][j][r];
            }
        }
}

constexpr int NUM_CUS = 256;

template <int FMT, int WN, int WM, int BPS, int KS, int D = PF_DEPTH>
hipError_t launch_prefill_m16(const void* w, const void* x, float* y, int64_t m, int64_t n, int64_t k, hipStream_t s)
{
    const int64_t rb = row_bytes(FMT, k);
    const dim3 grid(static_cast<unsigned>((n + 32 * WN - 1) / (32 * WN)), static_cast<unsigned>((m + 32 * WM - 1) / (32 * WM)));
    hipLaunchKernelGGL((prefill_m16_kernel<FMT, WN, WM, BPS, D, KS>), grid, dim3(PF_THREADS * KS), 0, s,
                       static_cast<const uint8_t*>(w), static_cast<const __bf16*>(x), y, static_cast<int>(m),
                       static_cast<int>(n), static_cast<int>(k), rb);
    return hipGetLastError();
}

template <int FMT, int MW, int NT, int KS, bool COMPACT, int D = PF_DEPTH>
hipError_t launch_prefill_shape(const void* w, const void* x, float* y, int64_t m, int64_t n, int64_t k, hipStream_t s)
{
    const int64_t rb = row_bytes(FMT, k);
    const dim3 grid(static_cast<unsigned>((n + 32 * NT - 1) / (32 * NT)), static_cast<unsigned>((m + 4 * MW - 1) / (4 * MW)));
    hipLaunchKernelGGL((prefill_mfma_kernel<FMT, MW, NT, D, KS, COMPACT>), grid, dim3(PF_THREADS * KS), 0, s,
                       static_cast<const uint8_t*>(w), static_cast<const __bf16*>(x), y, static_cast<int>(m),
                       static_cast<int>(n), static_cast<int>(k), rb);
    return hipGetLastError();
}

// splits > 1 needs `part` for tiles x splits x the tile's FP32 sums
// (prefill_part_bytes) and runs the reduction as a second launch.
template <int MW, int NT>
constexpr int64_t prefill_tile_bytes() { return static_cast<int64_t>(PF_THREADS) * (MW / 32) * NT * 4 * 16; }

template <int FMT, int MW, int NT, int D = PF_DEPTH>
hipError_t launch_prefill_ws(const void* w, const void* x, float* y, int64_t m, int64_t n, int64_t k, hipStream_t s,
                             int splits = 1, float4* part = nullptr)
{
    const int64_t rb = row_bytes(FMT, k);
    const unsigned tn = static_cast<unsigned>((n + 32 * NT - 1) / (32 * NT)), tm = static_cast<unsigned>((m + 4 * MW - 1) / (4 * MW));
    hipLaunchKernelGGL((prefill_ws_kernel<FMT, MW, NT, D>), dim3(tn, tm, static_cast<unsigned>(splits)),
                       dim3(2 * PF_THREADS), 0, s, static_cast<const uint8_t*>(w), static_cast<const __bf16*>(x), y,
                       static_cast<int>(m), static_cast<int>(n), static_cast<int>(k), rb, splits, part);
    if (splits > 1) {
        constexpr int64_t TILE4 = prefill_tile_bytes<MW, NT>() / 16;
        const int64_t threads = static_cast<int64_t>(tn) * tm * TILE4;
        hipLaunchKernelGGL((prefill_reduce_kernel<MW, NT>), dim3(static_cast<unsigned>(threads / PF_THREADS)),
                           dim3(PF_THREADS), 0, s, part, y, static_cast<int>(m), static_cast<int>(n), splits,
                           static_cast<int>(tn));
    }
    return hipGetLastError();
}

// Split count for the warp-specialised kernel on a grid of `tiles` tiles
// and `steps` 64-column steps: about one workgroup per CU, at least
// `min_steps` steps a split, every split non-empty.
inline int prefill_splits(int64_t tiles, int64_t steps, int cus, int min_steps)
{
    int64_t want = std::min<int64_t>(cus / std::max<int64_t>(tiles, 1), steps / min_steps);
    if (want < 2)
        return 1;
    const int64_t per = (steps + want - 1) / want;
    return static_cast<int>((steps + per - 1) / per);
}

// Tile choice (measured on the Phi-4-mini projections at 512 tokens):
//   * grids of more than 256 workgroups of 256 tokens x 64 rows: the
//     warp-specialised kernel with 256 x 128 tiles (64 x 128 consumer wave
//     tiles; gate_up 76 -> 67 us);
//   * with a split buffer, K split over about one workgroup per CU of the
//     same 256 x 128 tiles (at least 16 steps a split) when the 256 x 64
//     grid has 128..256 workgroups or K >= 4096: qkv 42.0 -> 37.2 us (3
//     splits), down 65.5 -> 50.0 us (5 splits); o_proj (3072 columns, 96
//     workgroups of 256 x 64) stays on the 16 x 16 form (26.4 against 28.2);
//   * 256 tokens x 64 rows (64 x 64 wave tiles, each fragment used twice)
//     when that grid has at least 128 workgroups: up to one per
//     CU two step groups of 4 waves with compact tiles (160 KiB, two waves
//     per SIMD) when they divide the steps, else the padded tile (84 KiB);
//   * otherwise, when K is a multiple of 256 and 96-row x 64-token tiles
//     give 128..256 workgroups, the 16 x 16 block form with that tile, 128
//     columns per step and the steps split between two groups of 4 waves
//     (o_proj 28.4 -> 25.7 us, down 72.4 -> 61.0 us at 512 tokens);
//   * otherwise 128 tokens x 64 rows with the steps split between two
//     groups of 4 waves when they divide evenly (two waves per SIMD
//     overlap their phases).
template <int FMT>
hipError_t launch_prefill_fmt(const void* w, const void* x, float* y, int64_t m, int64_t n, int64_t k, hipStream_t s,
                              void* split)
{
    auto wgs = [&](int mt, int nt) { return ((n + nt - 1) / nt) * ((m + mt - 1) / mt); };
    const int64_t big = wgs(256, 64);
    const int64_t steps = (k / 32 + 1) / 2;
    if (big > NUM_CUS)
        return launch_prefill_ws<FMT, 64, 4>(w, x, y, m, n, k, s);
    // split K: the 256 x 128 warp-specialised tiles over about one workgroup
    // per CU, at least 16 steps a split, for grids whose alternatives leave
    // CUs idle (the 256 x 64 tiles at 128..256 workgroups) or whose K is
    // long (the partial sums cost M x N x 4 bytes per split twice)
    const int64_t tiles = wgs(256, 128);
    const int sp = prefill_splits(tiles, steps, NUM_CUS, 16);
    if (split && sp > 1 && (big >= NUM_CUS / 2 || k >= 4096) &&
        tiles * sp * prefill_tile_bytes<64, 4>() <= PREFILL_SPLIT_BYTES)
        return launch_prefill_ws<FMT, 64, 4>(w, x, y, m, n, k, s, sp, static_cast<float4*>(split));
    if (big >= NUM_CUS / 2)
        return steps % 2 == 0 ? launch_prefill_shape<FMT, 64, 2, 2, true>(w, x, y, m, n, k, s)
                              : launch_prefill_shape<FMT, 64, 2, 1, false>(w, x, y, m, n, k, s);
    const int64_t m16 = wgs(64, 96);
    if (k % 256 == 0 && m16 >= NUM_CUS / 2 && m16 <= NUM_CUS)
        return launch_prefill_m16<FMT, 3, 2, 4, 2>(w, x, y, m, n, k, s);
    if (steps % 2 == 0)
        return launch_prefill_shape<FMT, 32, 2, 2, false>(w, x, y, m, n, k, s);
    return launch_prefill_shape<FMT, 32, 2, 1, false>(w, x, y, m, n, k, s);
}

}  // namespace

hipError_t launch_prefill(int fmt, const void* w, const void* x_bf16, float* y, int64_t m, int64_t rows, int64_t cols,
                          hipStream_t stream, void* split)
{
    switch (fmt) {
    case FMT_Q8_0: return launch_prefill_fmt<FMT_Q8_0>(w, x_bf16, y, m, rows, cols, stream, split);
    case FMT_Q4_0: return launch_prefill_fmt<FMT_Q4_0>(w, x_bf16, y, m, rows, cols, stream, split);
    case FMT_Q4_K: return launch_prefill_fmt<FMT_Q4_K>(w, x_bf16, y, m, rows, cols, stream, split);
    case FMT_F16: return cols % 32 == 0 ? launch_prefill_fmt<FMT_F16>(w, x_bf16, y, m, rows, cols, stream, split)
                                        : hipErrorInvalidValue;
    case FMT_F32: return cols % 32 == 0 ? launch_prefill_fmt<FMT_F32>(w, x_bf16, y, m, rows, cols, stream, split)
                                        : hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
}

}  // namespace si
