// C ABI of the op-by-op transformer launches (si_transformer.hip): argument
// checks, then one launch on the context stream.
#include "si_context.hpp"
#include "si_transformer.hpp"

#include <cmath>

using namespace si_abi;

namespace {

int check_vec(si_hip_context* ctx, const char* op, const void* p, const char* name, uintptr_t align = 4)
{
    if (!p || !aligned(p, align))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: %s must be a non-null %u-byte aligned device pointer", op, name,
                    static_cast<unsigned>(align));
    return SI_HIP_OK;
}

int check_eps(si_hip_context* ctx, const char* op, int64_t n, float eps)
{
    if (n < 1 || n > (1 << 20))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: %lld values outside 1..1048576", op, static_cast<long long>(n));
    if (!std::isfinite(eps) || eps < 0.0f)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: epsilon must be finite and non-negative", op);
    return SI_HIP_OK;
}

int cache_bytes(int fmt) { return fmt == SI_HIP_F32 ? 4 : fmt == SI_HIP_F16 ? 2 : 0; }

}  // namespace

extern "C" {

int si_hip_rms_norm(si_hip_context* ctx, const float* input, const float* weight, float* output, int64_t n, float eps)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "rms_norm: null context");
    Enter g(ctx);
    if (const int rc = check_eps(ctx, "rms_norm", n, eps))
        return rc;
    if (check_vec(ctx, "rms_norm", input, "input") || check_vec(ctx, "rms_norm", weight, "weight") ||
        check_vec(ctx, "rms_norm", output, "output"))
        return SI_HIP_ERR_ARGUMENT;
    const uint64_t b = static_cast<uint64_t>(n) * 4;
    if (overlaps(output, b, input, b) || overlaps(output, b, weight, b))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "rms_norm: output overlaps an input");
    const hipError_t e = si::launch_rms_norm(input, weight, output, static_cast<int>(n), eps, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "rms_norm launch");
}

int si_hip_residual_rms_norm(si_hip_context* ctx, const float* hidden, const float* residual, const float* weight,
                             float* updated, float* output, int64_t n, float eps)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "residual_rms_norm: null context");
    Enter g(ctx);
    const char* op = "residual_rms_norm";
    if (const int rc = check_eps(ctx, op, n, eps))
        return rc;
    if (check_vec(ctx, op, hidden, "hidden") || check_vec(ctx, op, residual, "residual") ||
        check_vec(ctx, op, weight, "weight") || check_vec(ctx, op, updated, "updated") ||
        check_vec(ctx, op, output, "output"))
        return SI_HIP_ERR_ARGUMENT;
    const uint64_t b = static_cast<uint64_t>(n) * 4;
    for (const void* w : {static_cast<const void*>(updated), static_cast<const void*>(output)})
        for (const void* r : {static_cast<const void*>(hidden), static_cast<const void*>(residual),
                              static_cast<const void*>(weight)})
            if (overlaps(w, b, r, b))
                return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: an output overlaps an input", op);
    if (overlaps(updated, b, output, b))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: updated and output overlap", op);
    const hipError_t e =
        si::launch_residual_rms_norm(hidden, residual, weight, updated, output, static_cast<int>(n), eps, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "residual_rms_norm launch");
}

int si_hip_swiglu(si_hip_context* ctx, const float* gate_up, float* output, int64_t n)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "swiglu: null context");
    Enter g(ctx);
    if (n < 1 || n > INT32_MAX)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "swiglu: %lld values out of range", static_cast<long long>(n));
    if (check_vec(ctx, "swiglu", gate_up, "gate_up") || check_vec(ctx, "swiglu", output, "output"))
        return SI_HIP_ERR_ARGUMENT;
    if (overlaps(output, static_cast<uint64_t>(n) * 4, gate_up, static_cast<uint64_t>(n) * 8))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "swiglu: output overlaps gate_up");
    const hipError_t e = si::launch_swiglu(gate_up, output, n, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "swiglu launch");
}

int si_hip_rope_kv_write(si_hip_context* ctx, const si_hip_rope_kv_write_args* a)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "rope_kv_write: null context");
    Enter g(ctx);
    const char* op = "rope_kv_write";
    if (!a)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: null arguments", op);
    const int cb = cache_bytes(a->cache_format);
    if (cb == 0)
        return fail(ctx, SI_HIP_ERR_UNSUPPORTED, "%s: cache format %d is not F32 or F16", op, a->cache_format);
    if (a->head_size < 1 || a->query_size < 1 || a->kv_size < 1 || a->query_size % a->head_size != 0 ||
        a->kv_size % a->head_size != 0 || a->rotary_size < 0 || a->rotary_size > a->head_size ||
        (a->rotary_size & 1) || a->context < 1 ||
        static_cast<int64_t>(a->query_size) + 2 * static_cast<int64_t>(a->kv_size) > INT32_MAX)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: invalid query, cache, head or rotary dimensions", op);
    if (!std::isfinite(a->rope_scale))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: rope_scale must be finite", op);
    if (check_vec(ctx, op, a->qkv, "qkv") || check_vec(ctx, op, a->position, "position") ||
        (a->rotary_size > 0 && check_vec(ctx, op, a->frequencies, "frequencies")) ||
        check_vec(ctx, op, a->query, "query") || check_vec(ctx, op, a->key_cache, "key_cache", cb) ||
        check_vec(ctx, op, a->value_cache, "value_cache", cb))
        return SI_HIP_ERR_ARGUMENT;
    const uint64_t qkv_b = (static_cast<uint64_t>(a->query_size) + 2ull * a->kv_size) * 4;
    const uint64_t q_b = static_cast<uint64_t>(a->query_size) * 4;
    const uint64_t c_b = static_cast<uint64_t>(a->context) * a->kv_size * cb;
    const uint64_t f_b = static_cast<uint64_t>(a->rotary_size / 2) * 4;
    const void* writes[3] = {a->query, a->key_cache, a->value_cache};
    const uint64_t wb[3] = {q_b, c_b, c_b};
    for (int i = 0; i < 3; i++) {
        if (overlaps(writes[i], wb[i], a->qkv, qkv_b) || overlaps(writes[i], wb[i], a->frequencies, f_b) ||
            overlaps(writes[i], wb[i], a->position, 4))
            return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: an output overlaps an input", op);
        for (int j = i + 1; j < 3; j++)
            if (overlaps(writes[i], wb[i], writes[j], wb[j]))
                return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: query and caches overlap", op);
    }
    si::RopeKvWriteArgs r;
    r.qkv = a->qkv;
    r.position = a->position;
    r.frequencies = a->frequencies;
    r.query = a->query;
    r.key_cache = a->key_cache;
    r.value_cache = a->value_cache;
    r.cache_fp16 = a->cache_format == SI_HIP_F16;
    r.query_size = a->query_size;
    r.kv_size = a->kv_size;
    r.head_size = a->head_size;
    r.rotary_size = a->rotary_size;
    r.context = a->context;
    r.rope_scale = a->rope_scale;
    const hipError_t e = si::launch_rope_kv_write(r, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "rope_kv_write launch");
}

int si_hip_grouped_query_attention(si_hip_context* ctx, const si_hip_gqa_args* a)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "grouped_query_attention: null context");
    Enter g(ctx);
    const char* op = "grouped_query_attention";
    if (!a)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: null arguments", op);
    const int cb = cache_bytes(a->cache_format);
    if (cb == 0)
        return fail(ctx, SI_HIP_ERR_UNSUPPORTED, "%s: cache format %d is not F32 or F16", op, a->cache_format);
    if (a->head_size != 64 && a->head_size != 128 && a->head_size != 256)
        return fail(ctx, SI_HIP_ERR_UNSUPPORTED, "%s: head size %d (64, 128 and 256 are built)", op, a->head_size);
    if (a->kv_heads < 1 || a->query_heads < 1 || a->query_heads % a->kv_heads != 0)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: query heads %d must be a multiple of KV heads %d", op,
                    a->query_heads, a->kv_heads);
    if (a->context < 1 || a->context > 16384)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: context %d outside 1..16384", op, a->context);
    if (check_vec(ctx, op, a->query, "query", 16) || check_vec(ctx, op, a->key_cache, "key_cache", 16) ||
        check_vec(ctx, op, a->value_cache, "value_cache", 16) || check_vec(ctx, op, a->position, "position") ||
        check_vec(ctx, op, a->output, "output") || check_vec(ctx, op, a->workspace, "workspace"))
        return SI_HIP_ERR_ARGUMENT;
    const uint64_t o_b = static_cast<uint64_t>(a->query_heads) * a->head_size * 4;
    const uint64_t c_b = static_cast<uint64_t>(a->context) * a->kv_heads * a->head_size * cb;
    const uint64_t ws_b = static_cast<uint64_t>(si::gqa_workspace_floats(a->query_heads, a->head_size, a->context)) * 4;
    const struct {
        const void* p;
        uint64_t n;
    } reads[] = {{a->query, o_b}, {a->key_cache, c_b}, {a->value_cache, c_b}, {a->position, 4}};
    for (const auto& r : reads)
        if (overlaps(a->output, o_b, r.p, r.n) || overlaps(a->workspace, ws_b, r.p, r.n))
            return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: output or workspace overlaps an input", op);
    if (overlaps(a->output, o_b, a->workspace, ws_b))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: output overlaps the workspace", op);
    si::GqaArgs r;
    r.query = a->query;
    r.key_cache = a->key_cache;
    r.value_cache = a->value_cache;
    r.position = a->position;
    r.output = a->output;
    r.cache_fp16 = a->cache_format == SI_HIP_F16;
    r.query_heads = a->query_heads;
    r.kv_heads = a->kv_heads;
    r.head_size = a->head_size;
    r.context = a->context;
    r.chunks = (a->context + 63) / 64;
    r.workspace = a->workspace;
    const hipError_t e = si::launch_gqa(r, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "grouped_query_attention launch");
}

int si_hip_gqa_workspace_bytes(int query_heads, int head_size, int context, uint64_t* bytes)
{
    if (!bytes || query_heads < 1 || head_size < 1 || context < 1)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "gqa_workspace_bytes: bad arguments");
    *bytes = static_cast<uint64_t>(si::gqa_workspace_floats(query_heads, head_size, context)) * 4;
    return SI_HIP_OK;
}

}  // extern "C"
