// C ABI of libsharpinference_hip (declared in include/sharpinference_hip.h):
// contexts, device memory, the quantized matrix-vector entry points,
// recorded plans (HIP graphs) and event timing.
#include "si_context.hpp"
#include "si_decode.hpp"

#include <vector>

namespace si_abi {

namespace {
thread_local std::string g_thread_error;
}

const char* thread_error() { return g_thread_error.c_str(); }

int fail(si_hip_context* ctx, int code, const char* fmt, ...)
{
    char buf[768];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_thread_error = buf;
    if (ctx)
        ctx->error = buf;
    return code;
}

int hip_fail(si_hip_context* ctx, hipError_t e, const char* what)
{
    return fail(ctx, e == hipErrorOutOfMemory ? SI_HIP_ERR_OUT_OF_MEMORY : SI_HIP_ERR_DEVICE, "%s: %s (%d)",
                what, hipGetErrorString(e), static_cast<int>(e));
}

bool is_quant(int fmt) { return si::is_block_quant(fmt); }

const char* fmt_name(int fmt)
{
    switch (fmt) {
    case si::FMT_F32: return "F32";
    case si::FMT_F16: return "F16";
    case si::FMT_Q4_0: return "Q4_0";
    case si::FMT_Q8_0: return "Q8_0";
    case si::FMT_Q4_K: return "Q4_K";
    case SI_HIP_BF16: return "BF16";
    default: return "unknown";
    }
}

// Shared validation of a [rows, cols] weight operand (Q8_0, Q4_0, Q4_K, F16
// or F32); returns 0 or a status.
int check_matrix(si_hip_context* ctx, const char* op, int fmt, const void* w, int64_t rows, int64_t cols,
                 uint64_t* wbytes)
{
    if (!si::is_matrix_format(fmt))
        return fail(ctx, SI_HIP_ERR_UNSUPPORTED,
                    "%s: tensor type %s (%d) is not a weight format of the matrix kernels (Q8_0, Q4_0, Q4_K, F16, F32)",
                    op, fmt_name(fmt), fmt);
    if (rows <= 0 || rows > INT32_MAX)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: rows %lld out of range 1..%d", op, static_cast<long long>(rows),
                    INT32_MAX);
    if (cols > INT32_MAX)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: columns %lld out of range 1..%d", op, static_cast<long long>(cols),
                    INT32_MAX);
    const int64_t rb = si::row_bytes(fmt, cols);
    if (rb < 0)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: %lld columns is not a whole number of %d-element %s blocks", op,
                    static_cast<long long>(cols), si::block_elems(fmt), fmt_name(fmt));
    // (rows and columns below 2^31 keep the byte count below 2^64)
    if (!w)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: null weight pointer", op);
    *wbytes = static_cast<uint64_t>(rb) * static_cast<uint64_t>(rows);
    return SI_HIP_OK;
}

}  // namespace si_abi

using namespace si_abi;

extern "C" {

int si_hip_abi_version(void) { return SI_HIP_ABI_VERSION; }

int si_hip_device_count(int* count)
{
    if (!count)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "device_count: null output");
    int n = 0;
    const hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) {
        *count = 0;
        return hip_fail(nullptr, e, "hipGetDeviceCount");
    }
    *count = n;
    return SI_HIP_OK;
}

int si_hip_init(int device, si_hip_context** out)
{
    if (!out)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "init: null output");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess)
        return hip_fail(nullptr, e, "hipGetDeviceCount");
    if (device < 0 || device >= n)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "init: device %d out of range (%d visible)", device, n);
    if ((e = hipSetDevice(device)) != hipSuccess)
        return hip_fail(nullptr, e, "hipSetDevice");
    auto* ctx = new si_hip_context();
    ctx->device = device;
    // the device address of the library's attention scratch on this GPU
    // (looked up once per device, with the device current)
    if ((e = si::attention_scratch(device, &ctx->attention_scratch)) != hipSuccess) {
        delete ctx;
        return hip_fail(nullptr, e, "hipGetSymbolAddress (attention scratch)");
    }
    // the prefill's split-K partial sums (its small grids run unsplit without it)
    if (hipMalloc(&ctx->prefill_split, si::PREFILL_SPLIT_BYTES) != hipSuccess) {
        (void)hipGetLastError();
        ctx->prefill_split = nullptr;
    }
    if ((e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking)) != hipSuccess ||
        (e = hipEventCreate(&ctx->t0)) != hipSuccess || (e = hipEventCreate(&ctx->t1)) != hipSuccess) {
        hip_fail(nullptr, e, "init");
        if (ctx->t0) (void)hipEventDestroy(ctx->t0);
        if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
        if (ctx->prefill_split) (void)hipFree(ctx->prefill_split);
        delete ctx;
        return SI_HIP_ERR_DEVICE;
    }
    *out = ctx;
    return SI_HIP_OK;
}

int si_hip_destroy(si_hip_context* ctx)
{
    if (!ctx)
        return SI_HIP_OK;
    {
        Enter g(ctx);
        if (ctx->recording) {
            hipGraph_t graph = nullptr;
            (void)hipStreamEndCapture(ctx->stream, &graph);
            if (graph) (void)hipGraphDestroy(graph);
        }
        (void)hipStreamSynchronize(ctx->stream);
        (void)hipEventDestroy(ctx->t0);
        (void)hipEventDestroy(ctx->t1);
        (void)hipStreamDestroy(ctx->stream);
        if (ctx->prefill_split)
            (void)hipFree(ctx->prefill_split);
    }
    delete ctx;
    return SI_HIP_OK;
}

const char* si_hip_last_error(const si_hip_context* ctx)
{
    return ctx ? ctx->error.c_str() : si_abi::thread_error();
}

int si_hip_tensor_bytes(int format, int64_t rows, int64_t cols, uint64_t* bytes)
{
    if (!bytes)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "tensor_bytes: null output");
    int64_t rb;
    switch (format) {
    case si::FMT_F32: rb = cols > 0 ? cols * 4 : -1; break;
    case si::FMT_F16:
    case SI_HIP_BF16: rb = cols > 0 ? cols * 2 : -1; break;
    case si::FMT_Q4_0:
    case si::FMT_Q8_0:
    case si::FMT_Q4_K: rb = si::row_bytes(format, cols); break;
    default:
        return fail(nullptr, SI_HIP_ERR_UNSUPPORTED, "tensor_bytes: GGUF tensor type %d is not supported", format);
    }
    if (rb < 0 || rows <= 0)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "tensor_bytes: shape [%lld, %lld] is not valid for %s",
                    static_cast<long long>(rows), static_cast<long long>(cols), fmt_name(format));
    *bytes = static_cast<uint64_t>(rb) * static_cast<uint64_t>(rows);
    return SI_HIP_OK;
}

int si_hip_alloc(si_hip_context* ctx, uint64_t bytes, void** device_ptr)
{
    if (!ctx || !device_ptr)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "alloc: null argument");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    *device_ptr = nullptr;
    if (ctx->recording)
        return fail(ctx, SI_HIP_ERR_STATE, "alloc: not allowed while recording a plan");
    if (bytes == 0)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "alloc: zero bytes");
    const hipError_t e = hipMalloc(device_ptr, bytes);
    if (e != hipSuccess) {
        *device_ptr = nullptr;
        return hip_fail(ctx, e, "hipMalloc");
    }
    return SI_HIP_OK;
}

int si_hip_free(si_hip_context* ctx, void* device_ptr)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "free: null context");
    Enter g(ctx);
    if (ctx->recording)
        return fail(ctx, SI_HIP_ERR_STATE, "free: not allowed while recording a plan");
    if (!device_ptr)
        return SI_HIP_OK;
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess)
        e = hipFree(device_ptr);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "hipFree");
}

static int copy_sync(si_hip_context* ctx, void* dst, const void* src, uint64_t bytes, hipMemcpyKind kind,
                     const char* op)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "%s: null context", op);
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    if (ctx->recording)
        return fail(ctx, SI_HIP_ERR_STATE, "%s: not allowed while recording a plan", op);
    if (bytes == 0)
        return SI_HIP_OK;
    if (!dst || !src)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: null pointer", op);
    hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, ctx->stream);
    if (e == hipSuccess)
        e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, op);
}

int si_hip_upload(si_hip_context* ctx, void* device_dst, const void* host_src, uint64_t bytes)
{
    return copy_sync(ctx, device_dst, host_src, bytes, hipMemcpyHostToDevice, "upload");
}

int si_hip_readback(si_hip_context* ctx, void* host_dst, const void* device_src, uint64_t bytes)
{
    return copy_sync(ctx, host_dst, device_src, bytes, hipMemcpyDeviceToHost, "readback");
}

int si_hip_copy(si_hip_context* ctx, void* device_dst, const void* device_src, uint64_t bytes)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "copy: null context");
    Enter g(ctx);
    if (bytes == 0)
        return SI_HIP_OK;
    if (!device_dst || !device_src)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "copy: null pointer");
    if (overlaps(device_dst, bytes, device_src, bytes))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "copy: source and destination overlap");
    const hipError_t e = hipMemcpyAsync(device_dst, device_src, bytes, hipMemcpyDeviceToDevice, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "copy");
}

int si_hip_fill_u32(si_hip_context* ctx, void* device_dst, uint32_t value, uint64_t count)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "fill: null context");
    Enter g(ctx);
    if (count == 0)
        return SI_HIP_OK;
    if (!device_dst || (reinterpret_cast<uintptr_t>(device_dst) & 3u))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "fill: destination must be a non-null 4-byte aligned pointer");
    const hipError_t e = si::launch_fill_u32(device_dst, value, count, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "fill");
}

int si_hip_checksum(si_hip_context* ctx, const void* device_src, uint64_t bytes, uint32_t* parts)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "checksum: null context");
    Enter g(ctx);
    if (!device_src || !parts || !aligned(device_src, 16) || !aligned(parts, 4) || bytes % 4 != 0 || bytes == 0)
        return fail(ctx, SI_HIP_ERR_ARGUMENT,
                    "checksum: src must be 16-byte aligned with a non-zero multiple of 4 bytes, parts 4-byte aligned");
    if (overlaps(parts, 4 * SI_HIP_CHECKSUM_PARTS, device_src, bytes))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "checksum: parts overlap src");
    const hipError_t e = si::launch_checksum(device_src, bytes, parts, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "checksum");
}

int si_hip_sync(si_hip_context* ctx)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "sync: null context");
    Enter g(ctx);
    if (ctx->recording)
        return fail(ctx, SI_HIP_ERR_STATE, "sync: not allowed while recording a plan");
    const hipError_t e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "hipStreamSynchronize");
}

int si_hip_gemv(si_hip_context* ctx, int format, const void* w, const float* x, float* y, int64_t rows,
                int64_t cols, const float* residual, int* path)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "gemv: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    uint64_t wbytes = 0;
    if (const int rc = check_matrix(ctx, "gemv", format, w, rows, cols, &wbytes))
        return rc;
    if (!x || !y)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv: null input or output");
    if ((reinterpret_cast<uintptr_t>(x) & 3u) || (reinterpret_cast<uintptr_t>(y) & 3u) ||
        (reinterpret_cast<uintptr_t>(residual) & 3u))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv: FP32 operands must be 4-byte aligned");
    const uint64_t ybytes = static_cast<uint64_t>(rows) * 4, xbytes = static_cast<uint64_t>(cols) * 4;
    // Writable aliasing is rejected (D3D12VmSchedule.cs:88-96); an exact
    // residual == y is an in-place accumulate and is allowed.
    if (overlaps(y, ybytes, w, wbytes) || overlaps(y, ybytes, x, xbytes) ||
        (residual && residual != y && overlaps(y, ybytes, residual, ybytes)))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv: output overlaps an input");
    const hipError_t e = si::launch_gemv(format, w, x, y, rows, cols, residual, ctx->stream, path);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "gemv launch");
}

int si_hip_gemm_prefill(si_hip_context* ctx, int format, const void* w, const void* x_bf16, float* y, int64_t m,
                        int64_t rows, int64_t cols)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "gemm_prefill: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    uint64_t wbytes = 0;
    if (const int rc = check_matrix(ctx, "gemm_prefill", format, w, rows, cols, &wbytes))
        return rc;
    if (m <= 0 || m > INT32_MAX)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemm_prefill: token count %lld out of range", static_cast<long long>(m));
    if (!is_quant(format) && cols % 32 != 0)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemm_prefill: %s weights need a multiple of 32 columns, got %lld",
                    fmt_name(format), static_cast<long long>(cols));
    if (!x_bf16 || !y)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemm_prefill: null input or output");
    if ((reinterpret_cast<uintptr_t>(x_bf16) & 15u) || (reinterpret_cast<uintptr_t>(y) & 3u))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemm_prefill: X must be 16-byte aligned and Y 4-byte aligned");
    const uint64_t ybytes = static_cast<uint64_t>(m) * static_cast<uint64_t>(rows) * 4;
    const uint64_t xbytes = static_cast<uint64_t>(m) * static_cast<uint64_t>(cols) * 2;
    if (overlaps(y, ybytes, w, wbytes) || overlaps(y, ybytes, x_bf16, xbytes))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemm_prefill: output overlaps an input");
    if (wbytes > UINT32_MAX || xbytes > UINT32_MAX)
        return fail(ctx, SI_HIP_ERR_UNSUPPORTED, "gemm_prefill: W and X must each be smaller than 4 GiB");
    const hipError_t e = si::launch_prefill(format, w, x_bf16, y, m, rows, cols, ctx->stream, ctx->prefill_split);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "gemm_prefill launch");
}

int si_hip_dequant(si_hip_context* ctx, int format, const void* w, float* out, int64_t rows, int64_t cols)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "dequant: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    uint64_t wbytes = 0;
    if (const int rc = check_matrix(ctx, "dequant", format, w, rows, cols, &wbytes))
        return rc;
    if (!out || (reinterpret_cast<uintptr_t>(out) & 3u))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "dequant: output must be a non-null 4-byte aligned pointer");
    if (overlaps(out, static_cast<uint64_t>(rows) * static_cast<uint64_t>(cols) * 4, w, wbytes))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "dequant: output overlaps the weights");
    const hipError_t e = si::launch_dequant(format, w, out, rows, cols, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "dequant launch");
}

int si_hip_plan_begin(si_hip_context* ctx)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "plan_begin: null context");
    Enter g(ctx);
    if (ctx->recording)
        return fail(ctx, SI_HIP_ERR_STATE, "plan_begin: already recording");
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess)
        e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed);
    if (e != hipSuccess)
        return hip_fail(ctx, e, "hipStreamBeginCapture");
    ctx->recording = true;
    return SI_HIP_OK;
}

int si_hip_plan_end(si_hip_context* ctx, si_hip_plan** out)
{
    if (!ctx || !out)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "plan_end: null argument");
    Enter g(ctx);
    *out = nullptr;
    if (!ctx->recording)
        return fail(ctx, SI_HIP_ERR_STATE, "plan_end: not recording");
    ctx->recording = false;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
    if (e != hipSuccess) {
        if (graph) (void)hipGraphDestroy(graph);
        return hip_fail(ctx, e, "hipStreamEndCapture");
    }
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return hip_fail(ctx, e, "hipGraphInstantiate");
    }
    // Upload the executable graph now, on the plan's stream, so that its first
    // launch (a session's first token, a bench's first timed step) does not
    // pay for it.
    e = hipGraphUpload(exec, ctx->stream);
    if (e != hipSuccess) {
        (void)hipGraphExecDestroy(exec);
        (void)hipGraphDestroy(graph);
        return hip_fail(ctx, e, "hipGraphUpload");
    }
    auto* plan = new si_hip_plan();
    plan->ctx = ctx;
    plan->graph = graph;
    plan->exec = exec;
    *out = plan;
    return SI_HIP_OK;
}

int si_hip_plan_destroy(si_hip_plan* plan)
{
    if (!plan)
        return SI_HIP_OK;
    {
        Enter g(plan->ctx);
        (void)hipStreamSynchronize(plan->ctx->stream);
        (void)hipGraphExecDestroy(plan->exec);
        (void)hipGraphDestroy(plan->graph);
    }
    delete plan;
    return SI_HIP_OK;
}

int si_hip_plan_launch(si_hip_plan* plan)
{
    if (!plan)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "plan_launch: null plan");
    si_hip_context* ctx = plan->ctx;
    Enter g(ctx);
    if (ctx->recording)
        return fail(ctx, SI_HIP_ERR_STATE, "plan_launch: not allowed while recording a plan");
    const hipError_t e = hipGraphLaunch(plan->exec, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "hipGraphLaunch");
}

int si_hip_plan_launch_sequence(si_hip_plan* const* plans, int nplans, int64_t steps)
{
    if (!plans || nplans <= 0 || steps < 0)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "plan_launch_sequence: bad arguments");
    si_hip_context* ctx = plans[0] ? plans[0]->ctx : nullptr;
    for (int i = 0; i < nplans; i++)
        if (!plans[i] || plans[i]->ctx != ctx)
            return fail(ctx, SI_HIP_ERR_ARGUMENT, "plan_launch_sequence: plans must be non-null and share a context");
    Enter g(ctx);
    if (ctx->recording)
        return fail(ctx, SI_HIP_ERR_STATE, "plan_launch_sequence: not allowed while recording a plan");
    for (int64_t i = 0; i < steps; i++) {
        const hipError_t e = hipGraphLaunch(plans[i % nplans]->exec, ctx->stream);
        if (e != hipSuccess)
            return hip_fail(ctx, e, "hipGraphLaunch");
    }
    return SI_HIP_OK;
}

int si_hip_plan_measure_us(si_hip_plan* plan, int repetitions, double* microseconds)
{
    if (!plan || !microseconds)
        return fail(plan ? plan->ctx : nullptr, SI_HIP_ERR_ARGUMENT, "plan_measure: null argument");
    si_hip_context* ctx = plan->ctx;
    Enter g(ctx);
    if (repetitions < 1 || repetitions > 1024)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "plan_measure: repetitions %d outside 1..1024", repetitions);
    if (ctx->recording)
        return fail(ctx, SI_HIP_ERR_STATE, "plan_measure: not allowed while recording a plan");
    // the measurement records the context's timer events: an open
    // timer_begin would lose its start
    if (ctx->timer_open)
        return fail(ctx, SI_HIP_ERR_STATE, "plan_measure: not allowed while a timer_begin is open");
    hipError_t e = hipEventRecord(ctx->t0, ctx->stream);
    for (int i = 0; e == hipSuccess && i < repetitions; i++)
        e = hipGraphLaunch(plan->exec, ctx->stream);
    if (e == hipSuccess) e = hipEventRecord(ctx->t1, ctx->stream);
    if (e == hipSuccess) e = hipEventSynchronize(ctx->t1);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, ctx->t0, ctx->t1);
    if (e != hipSuccess)
        return hip_fail(ctx, e, "plan_measure");
    if (!(ms > 0.0f))
        return fail(ctx, SI_HIP_ERR_DEVICE, "plan_measure: GPU timestamps did not advance");
    *microseconds = 1000.0 * static_cast<double>(ms) / repetitions;
    return SI_HIP_OK;
}

int si_hip_timer_begin(si_hip_context* ctx)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "timer_begin: null context");
    Enter g(ctx);
    if (ctx->recording)
        return fail(ctx, SI_HIP_ERR_STATE, "timer_begin: not allowed while recording a plan");
    const hipError_t e = hipEventRecord(ctx->t0, ctx->stream);
    if (e != hipSuccess)
        return hip_fail(ctx, e, "hipEventRecord");
    ctx->timer_open = true;
    return SI_HIP_OK;
}

int si_hip_timer_end(si_hip_context* ctx, double* milliseconds)
{
    if (!ctx || !milliseconds)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "timer_end: null argument");
    Enter g(ctx);
    if (!ctx->timer_open)
        return fail(ctx, SI_HIP_ERR_STATE, "timer_end: no timer_begin on this context");
    ctx->timer_open = false;
    hipError_t e = hipEventRecord(ctx->t1, ctx->stream);
    if (e == hipSuccess) e = hipEventSynchronize(ctx->t1);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, ctx->t0, ctx->t1);
    if (e != hipSuccess)
        return hip_fail(ctx, e, "timer_end");
    *milliseconds = static_cast<double>(ms);
    return SI_HIP_OK;
}

}  // extern "C"
