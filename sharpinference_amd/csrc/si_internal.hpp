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

// Elements and bytes per block; 0 for formats the quantized path does not take.
constexpr int block_elems(int fmt)
{
    return fmt == FMT_Q4_0 || fmt == FMT_Q8_0 ? 32 : fmt == FMT_Q4_K ? 256 : 0;
}
constexpr int block_bytes(int fmt)
{
    return fmt == FMT_Q4_0 ? 18 : fmt == FMT_Q8_0 ? 34 : fmt == FMT_Q4_K ? 144 : 0;
}

// Bytes of one row of `cols` elements, or -1 when cols is not a whole number
// of blocks (GgufModelFile.cs:323-329 rejects such tensors the same way).
inline int64_t row_bytes(int fmt, int64_t cols)
{
    const int be = block_elems(fmt);
    if (be == 0 || cols <= 0 || cols % be != 0)
        return -1;
    return cols / be * block_bytes(fmt);
}

// Optional work fused around the product y = W . x.
struct GemvEpilogue {
    const float* residual = nullptr;   // y = W.x + residual when non-null
};

// Transform applied to x while it is staged, before the product.
enum XformKind : int {
    XF_PLAIN = 0,
    XF_RMSNORM = 1,   // x_i * (1 / sqrt(sum(x^2) / cols + eps)) * weight_i
    XF_SWIGLU = 2,    // x holds [gate | up] (2 * cols values): gate / (1 + exp(-gate)) * up
};
struct GemvXform {
    int kind = XF_PLAIN;
    const float* weight = nullptr;
    float eps = 0.0f;
};

// Which kernel a launch used; reported to the caller for tests and profiles.
enum GemvPath : int { PATH_FAST = 1, PATH_GENERIC = 2 };

hipError_t launch_gemv(int fmt, const void* w, const float* x, float* y, int64_t rows, int64_t cols,
                       const GemvEpilogue& epi, hipStream_t stream, int* path);
// Same product with a transform of x fused into the staging; only the tiled
// kernel's column counts take a transform (returns hipErrorNotSupported
// otherwise).
hipError_t launch_gemv_xform(int fmt, const void* w, const float* x, float* y, int64_t rows, int64_t cols,
                             const GemvEpilogue& epi, const GemvXform& xf, hipStream_t stream, int* path);
bool gemv_tiled_cols(int64_t cols);
hipError_t launch_prefill(int fmt, const void* w, const void* x_bf16, float* y, int64_t m, int64_t rows,
                          int64_t cols, hipStream_t stream);
hipError_t launch_dequant(int fmt, const void* w, float* out, int64_t rows, int64_t cols,
                          hipStream_t stream);
hipError_t launch_fill_u32(void* dst, uint32_t value, uint64_t count, hipStream_t stream);

}  // namespace si
