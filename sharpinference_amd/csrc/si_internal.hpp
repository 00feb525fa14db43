// Internal declarations shared by the HIP translation units of
// libsharpinference_hip.  Nothing here is part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace si {

// GGUF tensor type ids (SharpInference.Gguf/GgufModelFile.cs:24-46).
enum Format : int {
    FMT_F32 = 0,
    FMT_F16 = 1,
    FMT_Q4_0 = 2,
    FMT_Q8_0 = 8,
    FMT_Q4_K = 12,
};

// Elements and bytes per block (an F16 / F32 "block" is one element); 0 for
// formats the matrix kernels do not take.
constexpr int block_elems(int fmt)
{
    return fmt == FMT_Q4_0 || fmt == FMT_Q8_0 ? 32 : fmt == FMT_Q4_K ? 256 : fmt == FMT_F16 || fmt == FMT_F32 ? 1 : 0;
}
constexpr int block_bytes(int fmt)
{
    return fmt == FMT_Q4_0 ? 18 : fmt == FMT_Q8_0 ? 34 : fmt == FMT_Q4_K ? 144 : fmt == FMT_F16 ? 2 : fmt == FMT_F32 ? 4 : 0;
}
constexpr bool is_block_quant(int fmt) { return fmt == FMT_Q4_0 || fmt == FMT_Q8_0 || fmt == FMT_Q4_K; }
// Weight formats of the matrix-vector kernels: the block-quantized ones and
// the dense F16 / F32 of the reference's own core.mat-vec
// (TierZeroOperationContracts.cs:161).
constexpr bool is_matrix_format(int fmt) { return is_block_quant(fmt) || fmt == FMT_F16 || fmt == FMT_F32; }

// Bytes of one row of `cols` elements, or -1 when cols is not a whole number
// of blocks (GgufModelFile.cs:323-329 rejects such tensors the same way).
inline int64_t row_bytes(int fmt, int64_t cols)
{
    const int be = block_elems(fmt);
    if (be == 0 || cols <= 0 || cols % be != 0)
        return -1;
    return cols / be * block_bytes(fmt);
}

// Transform applied to x while it is staged, before the product.
enum XformKind : int {
    XF_PLAIN = 0,
    XF_RMSNORM = 1,        // x_i * (1 / sqrt(sum(x^2) / cols + eps)) * weight_i
    XF_SWIGLU = 2,         // x holds [gate | up] (2 * cols values): gate / (1 + exp(-gate)) * up
    XF_LAYERNORM = 3,      // ((x - mean) * (1 / sqrt(var + eps))) * weight + bias
    XF_LAYERNORM_MIX = 4,  // ln = LAYERNORM(x); ln + (prev - ln) * mix
};

// Function applied to each output value (OUT_PLAIN also adds the residual).
enum OutKind : int {
    OUT_PLAIN = 0,
    OUT_SWIGLU_ROWS = 1,   // weight holds [gate rows; up rows]: y_r = g_r / (1 + exp(-g_r)) * u_r
    OUT_RELU_SQUARE = 2,   // max(v, 0)^2 (NaN stays NaN)
    OUT_TANH = 3,
    OUT_SIGMOID = 4,       // 1 / (1 + exp(-v))
};

// One quantized product y = out(W . in(x)) of a launch.  Several products
// without data dependences between them share one launch.
struct GemvOp {
    int fmt = 0;
    const void* w = nullptr;
    const float* x = nullptr;
    float* y = nullptr;
    int64_t rows = 0;                    // output rows (OUT_SWIGLU_ROWS reads 2 * rows weight rows)
    int64_t cols = 0;
    const float* residual = nullptr;     // OUT_PLAIN: y = W.x + residual (residual may be y)
    int in = XF_PLAIN;
    int out = OUT_PLAIN;
    const float* norm_weight = nullptr;
    const float* norm_bias = nullptr;
    const float* mix = nullptr;
    const float* prev = nullptr;
    float eps = 0.0f;
    float* norm_out = nullptr;           // XF_LAYERNORM*: the normalised x (before the mix), stored once
    const float* copy_src = nullptr;     // side job of the op's first workgroup:
    float* copy_dst = nullptr;           //   copy_dst[0..copy_n) = copy_src[0..copy_n)
    int64_t copy_n = 0;
    bool any_shape = false;              // plain products only: run the any-shape kernel (one wave per
                                         // row) whatever the shape, as a serial mat-vec is pinned
};

// Which kernel a launch used; reported to the caller for tests and profiles.
enum GemvPath : int { PATH_FAST = 1, PATH_GENERIC = 2, PATH_SHORT = 3 };

// Launches `count` independent products (no op reads what another writes).
// Consecutive ops that share a format and, for the tiled kernel, a column
// count go into one launch (up to 8 per launch).  Input transforms need the
// tiled kernel's column counts and alignment (hipErrorNotSupported
// otherwise).  paths[i] (optional) receives each op's kernel.
hipError_t launch_gemv_ops(const GemvOp* ops, int count, hipStream_t stream, int* paths);
// Plain product with an optional residual.
hipError_t launch_gemv(int fmt, const void* w, const float* x, float* y, int64_t rows, int64_t cols,
                       const float* residual, hipStream_t stream, int* path);
bool gemv_tiled_cols(int64_t cols);
// `split` (optional, PREFILL_SPLIT_BYTES, 16-byte aligned) holds the split-K
// partial sums of the grids that use it; without it those grids take the
// unsplit kernels.  Launches sharing one split buffer must be ordered.
constexpr int64_t PREFILL_SPLIT_BYTES = 32ll << 20;
hipError_t launch_prefill(int fmt, const void* w, const void* x_bf16, float* y, int64_t m, int64_t rows,
                          int64_t cols, hipStream_t stream, void* split = nullptr);
hipError_t launch_dequant(int fmt, const void* w, float* out, int64_t rows, int64_t cols,
                          hipStream_t stream);
hipError_t launch_fill_u32(void* dst, uint32_t value, uint64_t count, hipStream_t stream);
// parts: SI_HIP_CHECKSUM_PARTS (1024) words whose sum is the checksum.
hipError_t launch_checksum(const void* src, uint64_t bytes, uint32_t* parts, hipStream_t stream);

}  // namespace si
