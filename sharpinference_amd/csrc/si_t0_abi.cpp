// C ABI of the T0 primitive and portable tensor operators (si_t0.hip) and
// of the pinned any-shape mat-vec.  Shape rules are the T0 contracts'
// (TierZeroOperationContracts.cs:55-119, PortableTensorOperationContracts.cs:
// 86-186); an output that overlaps an input is rejected, as the reference
// rejects in-place operator writes (GpuTierZeroInstruction.cs:461-463).
#include "si_context.hpp"
#include "si_t0.hpp"

#include <cmath>

using namespace si_abi;

namespace {

bool misaligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) != 0; }

// Largest element count of one operand (2^40 FP32 values = 4 TiB): byte
// counts and the kernels' 64-bit indices stay far from overflow.
constexpr int64_t MAX_ELEMENTS = int64_t{1} << 40;

// Dimensions of a rank 1..4 tensor, each >= 1; element count into *count.
bool dims_ok(int rank, const int64_t* dims, int64_t* count)
{
    if (rank < 1 || rank > si::T0_MAX_RANK || !dims)
        return false;
    int64_t n = 1;
    for (int a = 0; a < rank; a++) {
        if (dims[a] < 1 || dims[a] > MAX_ELEMENTS / n)
            return false;
        n *= dims[a];
    }
    *count = n;
    return true;
}

}  // namespace

extern "C" {

int si_hip_t0_elementwise(si_hip_context* ctx, int op, const float* left, const float* right, float* output,
                          int64_t count)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "t0_elementwise: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    if (op < 0 || op >= si::T0_OP_COUNT)
        return fail(ctx, SI_HIP_ERR_UNSUPPORTED, "t0_elementwise: unknown operator %d", op);
    const bool binary = si::t0_binary(op);
    if (!left || !output || (binary && !right) || count < 1 || count > MAX_ELEMENTS)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_elementwise: null operand, empty tensor or more than 2^40 elements");
    if (misaligned4(left) || misaligned4(output) || (binary && misaligned4(right)))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_elementwise: FP32 operands must be 4-byte aligned");
    const uint64_t bytes = static_cast<uint64_t>(count) * 4;
    if (overlaps(output, bytes, left, bytes) || (binary && overlaps(output, bytes, right, bytes)))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_elementwise: in-place operator writes are unsupported");
    const hipError_t e = si::launch_t0_elementwise(op, left, binary ? right : nullptr, output, count, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "t0_elementwise launch");
}

int si_hip_t0_cast_f16_f32(si_hip_context* ctx, const void* input, float* output, int64_t count)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "t0_cast: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    if (!input || !output || count < 1 || count > MAX_ELEMENTS)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_cast: null operand, empty tensor or more than 2^40 elements");
    if ((reinterpret_cast<uintptr_t>(input) & 1u) || misaligned4(output))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_cast: misaligned operand");
    if (overlaps(output, static_cast<uint64_t>(count) * 4, input, static_cast<uint64_t>(count) * 2))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_cast: in-place operator writes are unsupported");
    const hipError_t e = si::launch_t0_cast_f16(input, output, count, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "t0_cast launch");
}

int si_hip_t0_fill(si_hip_context* ctx, float value, float* output, int64_t count)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "t0_fill: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    if (!output || count < 1 || count > MAX_ELEMENTS || misaligned4(output))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_fill: null, empty, misaligned or larger than 2^40 elements output");
    // TensorFillValue: non-finite values are not supported (PortableTensorOperationContracts.cs:16-20)
    if (!std::isfinite(value))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_fill: the value must be finite");
    const hipError_t e = si::launch_t0_fill(output, value, count, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "t0_fill launch");
}

int si_hip_t0_reduce_last(si_hip_context* ctx, int mean, const float* input, float* output, int64_t rows,
                          int64_t cols)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "t0_reduce: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    if (!input || !output || rows < 1 || cols < 1 || rows > INT32_MAX || cols > INT32_MAX ||
        rows > MAX_ELEMENTS / cols)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_reduce: null operand or shape out of range");
    if (misaligned4(input) || misaligned4(output))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_reduce: FP32 operands must be 4-byte aligned");
    if (overlaps(output, static_cast<uint64_t>(rows) * 4, input, static_cast<uint64_t>(rows) * cols * 4))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_reduce: in-place operator writes are unsupported");
    const hipError_t e = si::launch_t0_reduce_last(mean != 0, input, output, rows, cols, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "t0_reduce launch");
}

int si_hip_t0_broadcast(si_hip_context* ctx, const float* input, int input_rank, const int64_t* input_dims,
                        float* output, int output_rank, const int64_t* output_dims)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "t0_broadcast: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    int64_t in_n = 0, out_n = 0;
    if (!input || !output || !dims_ok(input_rank, input_dims, &in_n) || !dims_ok(output_rank, output_dims, &out_n))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_broadcast: null operand or dimensions outside rank 1..4");
    if (misaligned4(input) || misaligned4(output))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_broadcast: FP32 operands must be 4-byte aligned");
    // trailing dimensions aligned; an input axis is 1 (repeated) or equal to the output's
    // (PortableTensorOperationContracts.cs:158-164)
    if (input_rank > output_rank)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_broadcast: incompatible dimensions");
    si::GatherShape s{};
    s.rank = output_rank;
    s.count = out_n;
    const int shift = output_rank - input_rank;
    int64_t stride = 1;
    for (int a = output_rank - 1; a >= 0; a--) {
        s.dims[a] = output_dims[a];
        if (a < shift) {
            s.strides[a] = 0;
            continue;
        }
        const int64_t d = input_dims[a - shift];
        if (d != 1 && d != output_dims[a])
            return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_broadcast: incompatible dimensions");
        s.strides[a] = d == 1 ? 0 : stride;
        stride *= d;
    }
    if (overlaps(output, static_cast<uint64_t>(out_n) * 4, input, static_cast<uint64_t>(in_n) * 4))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_broadcast: in-place operator writes are unsupported");
    const hipError_t e = si::launch_t0_gather(input, output, s, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "t0_broadcast launch");
}

int si_hip_t0_slice(si_hip_context* ctx, const float* input, int rank, const int64_t* input_dims, int axis,
                    int64_t start, int64_t length, float* output)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "t0_slice: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    int64_t in_n = 0;
    if (!input || !output || !dims_ok(rank, input_dims, &in_n))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_slice: null operand or dimensions outside rank 1..4");
    if (misaligned4(input) || misaligned4(output))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_slice: FP32 operands must be 4-byte aligned");
    // (PortableTensorOperationContracts.cs:138-149)
    if (axis < 0 || axis >= rank || length < 1 || start < 0 || start + length > input_dims[axis])
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_slice: incompatible dimensions");
    si::GatherShape s{};
    s.rank = rank;
    s.count = in_n / input_dims[axis] * length;
    int64_t stride = 1;
    for (int a = rank - 1; a >= 0; a--) {
        s.dims[a] = a == axis ? length : input_dims[a];
        s.strides[a] = stride;
        if (a == axis)
            s.base = start * stride;
        stride *= input_dims[a];
    }
    if (overlaps(output, static_cast<uint64_t>(s.count) * 4, input, static_cast<uint64_t>(in_n) * 4))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_slice: in-place operator writes are unsupported");
    const hipError_t e = si::launch_t0_gather(input, output, s, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "t0_slice launch");
}

int si_hip_t0_head_outer(si_hip_context* ctx, const float* left, const float* right, float* output, int64_t heads,
                         int64_t rows, int64_t cols)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "t0_head_outer: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    if (!left || !right || !output || heads < 1 || rows < 1 || cols < 1 || heads > INT32_MAX ||
        rows > INT32_MAX || cols > INT32_MAX || rows > MAX_ELEMENTS / cols || heads > MAX_ELEMENTS / (rows * cols))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_head_outer: null operand or shape out of range");
    if (misaligned4(left) || misaligned4(right) || misaligned4(output))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_head_outer: FP32 operands must be 4-byte aligned");
    const uint64_t ob = static_cast<uint64_t>(heads) * rows * cols * 4;
    if (overlaps(output, ob, left, static_cast<uint64_t>(heads) * rows * 4) ||
        overlaps(output, ob, right, static_cast<uint64_t>(heads) * cols * 4))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "t0_head_outer: in-place operator writes are unsupported");
    const hipError_t e = si::launch_t0_head_outer(left, right, output, heads, rows, cols, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "t0_head_outer launch");
}

int si_hip_gemv_any_shape(si_hip_context* ctx, int format, const void* w, const float* x, float* y, int64_t rows,
                          int64_t cols)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "gemv_any_shape: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    uint64_t wbytes = 0;
    if (const int rc = check_matrix(ctx, "gemv_any_shape", format, w, rows, cols, &wbytes))
        return rc;
    if (!x || !y)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_any_shape: null input or output");
    if (misaligned4(x) || misaligned4(y))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_any_shape: FP32 operands must be 4-byte aligned");
    const uint64_t ybytes = static_cast<uint64_t>(rows) * 4;
    if (overlaps(y, ybytes, w, wbytes) || overlaps(y, ybytes, x, static_cast<uint64_t>(cols) * 4))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_any_shape: output overlaps an input");
    si::GemvOp op;
    op.fmt = format;
    op.w = w;
    op.x = x;
    op.y = y;
    op.rows = rows;
    op.cols = cols;
    op.any_shape = true;
    const hipError_t e = si::launch_gemv_ops(&op, 1, ctx->stream, nullptr);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "gemv_any_shape launch");
}

}  // extern "C"
