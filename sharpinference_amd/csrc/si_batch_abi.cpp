// C ABI of the batched (prefill) transformer launches (si_batch.hip):
// argument checks, then the launch(es) on the context stream.
#include "si_batch.hpp"
#include "si_context.hpp"
#include "si_internal.hpp"

#include <cmath>

using namespace si_abi;

namespace {

int check_ptr(si_hip_context* ctx, const char* op, const void* p, const char* name, uintptr_t align = 4)
{
    if (!p || !aligned(p, align))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: %s must be a non-null %u-byte aligned device pointer", op, name,
                    static_cast<unsigned>(align));
    return SI_HIP_OK;
}

int check_batch(si_hip_context* ctx, const char* op, int batch)
{
    if (batch < 1 || batch > si::BATCH_MAX)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: batch %d outside 1..%d", op, batch, si::BATCH_MAX);
    return SI_HIP_OK;
}

int check_width(si_hip_context* ctx, const char* op, int64_t width, int64_t max = 1 << 20)
{
    if (width < 1 || width > max)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: width %lld outside 1..%lld", op, static_cast<long long>(width),
                    static_cast<long long>(max));
    return SI_HIP_OK;
}

int cache_bytes(int fmt) { return fmt == SI_HIP_F32 ? 4 : fmt == SI_HIP_F16 ? 2 : 0; }

struct Span {
    const void* p;
    uint64_t n;
};

// Fails when any written span overlaps a read span or another written one.
int check_disjoint(si_hip_context* ctx, const char* op, std::initializer_list<Span> writes,
                   std::initializer_list<Span> reads)
{
    for (auto w = writes.begin(); w != writes.end(); ++w) {
        for (const auto& r : reads)
            if (overlaps(w->p, w->n, r.p, r.n))
                return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: an output overlaps an input", op);
        for (auto v = w + 1; v != writes.end(); ++v)
            if (overlaps(w->p, w->n, v->p, v->n))
                return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: outputs overlap", op);
    }
    return SI_HIP_OK;
}

int launched(si_hip_context* ctx, hipError_t e, const char* op)
{
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, op);
}

// The attention launches' shape checks.
int check_attention_shape(si_hip_context* ctx, const char* op, const si_hip_batch_attention_args* a)
{
    if (!a)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: null arguments", op);
    const int cb = cache_bytes(a->cache_format);
    if (cb == 0)
        return fail(ctx, SI_HIP_ERR_UNSUPPORTED, "%s: cache format %d is not F32 or F16", op, a->cache_format);
    if (a->head_size != si::BATCH_HEAD)
        return fail(ctx, SI_HIP_ERR_UNSUPPORTED, "%s: head size %d (128 is built)", op, a->head_size);
    if (const int rc = check_batch(ctx, op, a->batch))
        return rc;
    if (a->kv_heads < 1 || a->query_heads < 1 || a->query_heads % a->kv_heads != 0 ||
        a->query_heads / a->kv_heads > si::BATCH_GROUP_MAX)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: query heads %d must be 1..%d times KV heads %d", op,
                    a->query_heads, si::BATCH_GROUP_MAX, a->kv_heads);
    if (a->context < 1 || a->context > 16384)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: context %d outside 1..16384", op, a->context);
    return SI_HIP_OK;
}

// The attention launches' shared checks; `values` selects the values form.
int check_attention(si_hip_context* ctx, const char* op, const si_hip_batch_attention_args* a, bool values)
{
    if (const int rc = check_attention_shape(ctx, op, a))
        return rc;
    const int cb = cache_bytes(a->cache_format);
    const uint64_t q_b = static_cast<uint64_t>(a->batch) * a->query_heads * si::BATCH_HEAD * 4;
    const uint64_t s_b = static_cast<uint64_t>(a->batch) * a->query_heads * a->context * 4;
    const uint64_t c_b = static_cast<uint64_t>(a->context) * a->kv_heads * si::BATCH_HEAD * cb;
    if (check_ptr(ctx, op, a->cache, "cache", 16) || check_ptr(ctx, op, a->control, "control") ||
        check_ptr(ctx, op, a->output, "output", values ? 8 : 4))
        return SI_HIP_ERR_ARGUMENT;
    if (!values) {
        if (check_ptr(ctx, op, a->query, "query", 16))
            return SI_HIP_ERR_ARGUMENT;
        return check_disjoint(ctx, op, {{a->output, s_b}}, {{a->query, q_b}, {a->cache, c_b}, {a->control, 8}});
    }
    if (check_ptr(ctx, op, a->probabilities, "probabilities") || check_ptr(ctx, op, a->workspace, "workspace", 8))
        return SI_HIP_ERR_ARGUMENT;
    const uint64_t ws_b = static_cast<uint64_t>(si::batch_values_workspace_floats(a->batch, a->query_heads, a->context)) * 4;
    return check_disjoint(ctx, op, {{a->output, q_b}, {a->workspace, ws_b}},
                          {{a->probabilities, s_b}, {a->cache, c_b}, {a->control, 8}});
}

si::BatchAttentionArgs attention(const si_hip_batch_attention_args* a)
{
    si::BatchAttentionArgs r;
    r.query = a->query;
    r.probabilities = a->probabilities;
    r.cache = a->cache;
    r.control = a->control;
    r.out = a->output;
    r.workspace = a->workspace;
    r.cache_fp16 = a->cache_format == SI_HIP_F16;
    r.batch = a->batch;
    r.query_heads = a->query_heads;
    r.kv_heads = a->kv_heads;
    r.context = a->context;
    return r;
}

}  // namespace

extern "C" {

int si_hip_batch_gather_rows(si_hip_context* ctx, const float* table, int64_t table_rows, int64_t width,
                             const int32_t* control, float* output, int batch)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "batch_gather_rows: null context");
    Enter g(ctx);
    const char* op = "batch_gather_rows";
    if (check_batch(ctx, op, batch) || check_width(ctx, op, width))
        return SI_HIP_ERR_ARGUMENT;
    if (table_rows < 1 || table_rows > INT32_MAX)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: table rows %lld out of range", op, static_cast<long long>(table_rows));
    if (check_ptr(ctx, op, table, "table") || check_ptr(ctx, op, control, "control") ||
        check_ptr(ctx, op, output, "output"))
        return SI_HIP_ERR_ARGUMENT;
    const uint64_t o_b = static_cast<uint64_t>(batch) * width * 4;
    if (check_disjoint(ctx, op, {{output, o_b}}, {{table, static_cast<uint64_t>(table_rows) * width * 4}, {control, 8}}))
        return SI_HIP_ERR_ARGUMENT;
    return launched(ctx, si::launch_batch_gather_rows(table, table_rows, static_cast<int>(width), control, output, batch,
                                                      ctx->stream),
                    op);
}

int si_hip_batch_rms_norm(si_hip_context* ctx, const float* input, const float* weight, const int32_t* control,
                          float* output, int batch, int64_t width, float eps)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "batch_rms_norm: null context");
    Enter g(ctx);
    const char* op = "batch_rms_norm";
    if (check_batch(ctx, op, batch) || check_width(ctx, op, width))
        return SI_HIP_ERR_ARGUMENT;
    if (!std::isfinite(eps) || eps < 0.0f)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: epsilon must be finite and non-negative", op);
    if (check_ptr(ctx, op, input, "input") || check_ptr(ctx, op, weight, "weight") ||
        check_ptr(ctx, op, control, "control") || check_ptr(ctx, op, output, "output"))
        return SI_HIP_ERR_ARGUMENT;
    const uint64_t m = static_cast<uint64_t>(batch) * width * 4;
    if (check_disjoint(ctx, op, {{output, m}}, {{input, m}, {weight, static_cast<uint64_t>(width) * 4}, {control, 8}}))
        return SI_HIP_ERR_ARGUMENT;
    return launched(ctx, si::launch_batch_rms_norm(input, nullptr, weight, nullptr, output, batch,
                                                   static_cast<int>(width), eps, control, ctx->stream),
                    op);
}

int si_hip_batch_residual_rms_norm(si_hip_context* ctx, const float* hidden, const float* residual,
                                   const float* weight, const int32_t* control, float* updated, float* output,
                                   int batch, int64_t width, float eps)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "batch_residual_rms_norm: null context");
    Enter g(ctx);
    const char* op = "batch_residual_rms_norm";
    if (check_batch(ctx, op, batch) || check_width(ctx, op, width))
        return SI_HIP_ERR_ARGUMENT;
    if (!std::isfinite(eps) || eps < 0.0f)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: epsilon must be finite and non-negative", op);
    if (check_ptr(ctx, op, hidden, "hidden") || check_ptr(ctx, op, residual, "residual") ||
        check_ptr(ctx, op, weight, "weight") || check_ptr(ctx, op, control, "control") ||
        check_ptr(ctx, op, updated, "updated") || check_ptr(ctx, op, output, "output"))
        return SI_HIP_ERR_ARGUMENT;
    const uint64_t m = static_cast<uint64_t>(batch) * width * 4;
    if (check_disjoint(ctx, op, {{updated, m}, {output, m}},
                       {{hidden, m}, {residual, m}, {weight, static_cast<uint64_t>(width) * 4}, {control, 8}}))
        return SI_HIP_ERR_ARGUMENT;
    return launched(ctx, si::launch_batch_rms_norm(hidden, residual, weight, updated, output, batch,
                                                   static_cast<int>(width), eps, control, ctx->stream),
                    op);
}

int si_hip_batch_matvec(si_hip_context* ctx, int format, const void* weight, const float* input,
                        const int32_t* control, float* output, int batch, int64_t rows, int64_t columns)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "batch_matvec: null context");
    Enter g(ctx);
    const char* op = "batch_matvec";
    uint64_t wbytes = 0;
    if (const int rc = check_matrix(ctx, op, format, weight, rows, columns, &wbytes))
        return rc;
    if (check_batch(ctx, op, batch))
        return SI_HIP_ERR_ARGUMENT;
    if (columns % 32 != 0 || columns > (1 << 20))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: %lld columns is not a multiple of 32 up to 1048576", op,
                    static_cast<long long>(columns));
    if (check_ptr(ctx, op, weight, "weight", 16) || check_ptr(ctx, op, input, "input", 16) ||
        check_ptr(ctx, op, control, "control") || check_ptr(ctx, op, output, "output"))
        return SI_HIP_ERR_ARGUMENT;
    const uint64_t x_b = static_cast<uint64_t>(batch) * columns * 4, y_b = static_cast<uint64_t>(batch) * rows * 4;
    if (check_disjoint(ctx, op, {{output, y_b}}, {{weight, wbytes}, {input, x_b}, {control, 8}}))
        return SI_HIP_ERR_ARGUMENT;
    return launched(ctx, si::launch_batch_matvec(format, weight, input, output, batch, rows, columns, control,
                                                 ctx->stream),
                    op);
}

int si_hip_batch_swiglu(si_hip_context* ctx, const float* gate_up, const int32_t* control, float* output, int batch,
                        int64_t width)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "batch_swiglu: null context");
    Enter g(ctx);
    const char* op = "batch_swiglu";
    if (check_batch(ctx, op, batch) || check_width(ctx, op, width))
        return SI_HIP_ERR_ARGUMENT;
    if (check_ptr(ctx, op, gate_up, "gate_up") || check_ptr(ctx, op, control, "control") ||
        check_ptr(ctx, op, output, "output"))
        return SI_HIP_ERR_ARGUMENT;
    const uint64_t m = static_cast<uint64_t>(batch) * width * 4;
    if (check_disjoint(ctx, op, {{output, m}}, {{gate_up, 2 * m}, {control, 8}}))
        return SI_HIP_ERR_ARGUMENT;
    return launched(ctx, si::launch_batch_swiglu(gate_up, output, batch, static_cast<int>(width), control, ctx->stream),
                    op);
}

int si_hip_batch_rope_kv_write(si_hip_context* ctx, const si_hip_batch_rope_args* a)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "batch_rope_kv_write: null context");
    Enter g(ctx);
    const char* op = "batch_rope_kv_write";
    if (!a)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: null arguments", op);
    const int cb = cache_bytes(a->cache_format);
    if (cb == 0)
        return fail(ctx, SI_HIP_ERR_UNSUPPORTED, "%s: cache format %d is not F32 or F16", op, a->cache_format);
    if (check_batch(ctx, op, a->batch))
        return SI_HIP_ERR_ARGUMENT;
    if (a->head_size < 1 || a->query_size < 1 || a->kv_size < 1 || a->query_size % a->head_size != 0 ||
        a->kv_size % a->head_size != 0 || a->rotary_size < 0 || a->rotary_size > a->head_size ||
        (a->rotary_size & 1) || a->context < 1 ||
        static_cast<int64_t>(a->query_size) + 2 * static_cast<int64_t>(a->kv_size) > (1 << 20))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: invalid query, cache, head or rotary dimensions", op);
    if (!std::isfinite(a->rope_scale))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: rope_scale must be finite", op);
    if (check_ptr(ctx, op, a->qkv, "qkv") || check_ptr(ctx, op, a->control, "control") ||
        (a->rotary_size > 0 && check_ptr(ctx, op, a->frequencies, "frequencies")) ||
        check_ptr(ctx, op, a->query, "query") || check_ptr(ctx, op, a->key_cache, "key_cache", cb) ||
        check_ptr(ctx, op, a->value_cache, "value_cache", cb))
        return SI_HIP_ERR_ARGUMENT;
    const uint64_t qkv_b = static_cast<uint64_t>(a->batch) * (a->query_size + 2ull * a->kv_size) * 4;
    const uint64_t q_b = static_cast<uint64_t>(a->batch) * a->query_size * 4;
    const uint64_t c_b = static_cast<uint64_t>(a->context) * a->kv_size * cb;
    const uint64_t f_b = static_cast<uint64_t>(a->rotary_size / 2) * 4;
    if (check_disjoint(ctx, op, {{a->query, q_b}, {a->key_cache, c_b}, {a->value_cache, c_b}},
                       {{a->qkv, qkv_b}, {a->frequencies, f_b}, {a->control, 8}}))
        return SI_HIP_ERR_ARGUMENT;
    si::BatchRopeArgs r;
    r.qkv = a->qkv;
    r.control = a->control;
    r.frequencies = a->frequencies;
    r.query = a->query;
    r.key_cache = a->key_cache;
    r.value_cache = a->value_cache;
    r.cache_fp16 = a->cache_format == SI_HIP_F16;
    r.batch = a->batch;
    r.query_size = a->query_size;
    r.kv_size = a->kv_size;
    r.head_size = a->head_size;
    r.rotary_size = a->rotary_size;
    r.context = a->context;
    r.rope_scale = a->rope_scale;
    return launched(ctx, si::launch_batch_rope_kv_write(r, ctx->stream), op);
}

int si_hip_batch_gqa_scores(si_hip_context* ctx, const si_hip_batch_attention_args* a)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "batch_gqa_scores: null context");
    Enter g(ctx);
    if (const int rc = check_attention(ctx, "batch_gqa_scores", a, false))
        return rc;
    return launched(ctx, si::launch_batch_gqa_scores(attention(a), ctx->stream), "batch_gqa_scores");
}

int si_hip_batch_causal_softmax(si_hip_context* ctx, const float* scores, const int32_t* control,
                                float* probabilities, int batch, int heads, int64_t context)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "batch_causal_softmax: null context");
    Enter g(ctx);
    const char* op = "batch_causal_softmax";
    if (check_batch(ctx, op, batch))
        return SI_HIP_ERR_ARGUMENT;
    if (heads < 1 || heads > 4096 || context < 1 || context > 16384)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: heads %d or context %lld out of range", op, heads,
                    static_cast<long long>(context));
    if (check_ptr(ctx, op, scores, "scores") || check_ptr(ctx, op, control, "control") ||
        check_ptr(ctx, op, probabilities, "probabilities"))
        return SI_HIP_ERR_ARGUMENT;
    const uint64_t m = static_cast<uint64_t>(batch) * heads * context * 4;
    if (check_disjoint(ctx, op, {{probabilities, m}}, {{scores, m}, {control, 8}}))
        return SI_HIP_ERR_ARGUMENT;
    return launched(ctx, si::launch_batch_causal_softmax(scores, probabilities, batch, heads, static_cast<int>(context),
                                                         control, ctx->stream),
                    op);
}

int si_hip_batch_gqa_values(si_hip_context* ctx, const si_hip_batch_attention_args* a)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "batch_gqa_values: null context");
    Enter g(ctx);
    if (const int rc = check_attention(ctx, "batch_gqa_values", a, true))
        return rc;
    return launched(ctx, si::launch_batch_gqa_values(attention(a), ctx->stream), "batch_gqa_values");
}

int si_hip_batch_gqa_attention(si_hip_context* ctx, const si_hip_batch_attention_args* a, const void* value_cache)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "batch_gqa_attention: null context");
    Enter g(ctx);
    const char* op = "batch_gqa_attention";
    if (const int rc = check_attention_shape(ctx, op, a))
        return rc;
    const uint64_t q_b = static_cast<uint64_t>(a->batch) * a->query_heads * si::BATCH_HEAD * 4;
    const uint64_t c_b = static_cast<uint64_t>(a->context) * a->kv_heads * si::BATCH_HEAD * cache_bytes(a->cache_format);
    const uint64_t ws_b = static_cast<uint64_t>(si::batch_values_workspace_floats(a->batch, a->query_heads, a->context)) * 4;
    if (check_ptr(ctx, op, a->query, "query", 16) || check_ptr(ctx, op, a->cache, "cache", 16) ||
        check_ptr(ctx, op, value_cache, "value_cache", 16) || check_ptr(ctx, op, a->control, "control") ||
        check_ptr(ctx, op, a->output, "output", 8) || check_ptr(ctx, op, a->workspace, "workspace", 8))
        return SI_HIP_ERR_ARGUMENT;
    if (check_disjoint(ctx, op, {{a->output, q_b}, {a->workspace, ws_b}},
                       {{a->query, q_b}, {a->cache, c_b}, {value_cache, c_b}, {a->control, 8}}))
        return SI_HIP_ERR_ARGUMENT;
    return launched(ctx, si::launch_batch_gqa_attention(attention(a), value_cache, ctx->stream), op);
}

int si_hip_batch_values_workspace_bytes(int batch, int query_heads, int context, uint64_t* bytes)
{
    if (!bytes || batch < 1 || query_heads < 1 || context < 1)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "batch_values_workspace_bytes: bad arguments");
    *bytes = static_cast<uint64_t>(si::batch_values_workspace_floats(batch, query_heads, context)) * 4;
    return SI_HIP_OK;
}

int si_hip_batch_select_last(si_hip_context* ctx, const float* input, const int32_t* control, float* output,
                             int batch, int64_t width)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "batch_select_last: null context");
    Enter g(ctx);
    const char* op = "batch_select_last";
    if (check_batch(ctx, op, batch) || check_width(ctx, op, width))
        return SI_HIP_ERR_ARGUMENT;
    if (check_ptr(ctx, op, input, "input") || check_ptr(ctx, op, control, "control") ||
        check_ptr(ctx, op, output, "output"))
        return SI_HIP_ERR_ARGUMENT;
    if (check_disjoint(ctx, op, {{output, static_cast<uint64_t>(width) * 4}},
                       {{input, static_cast<uint64_t>(batch) * width * 4}, {control, 8}}))
        return SI_HIP_ERR_ARGUMENT;
    return launched(ctx, si::launch_batch_select_last(input, output, batch, static_cast<int>(width), control, ctx->stream),
                    op);
}

}  // extern "C"
