// C ABI of the decode-step operators (fused-norm GEMV, row gather,
// attention, argmax) and the Phi-4 decode program recorder.
//
// The recorder is the HIP counterpart of the reference's hand-built Phi-4
// decode program (SharpInference.Architectures.Phi4.D3D12/
// Phi4D3D12TextSession.cs:866-919): embedding gather, 32 x (RMSNorm + qkv,
// rotary + KV append + attention, o_proj + residual, RMSNorm + gate_up,
// SwiGLU + down + residual), final RMSNorm + vocabulary projection, argmax,
// recorded once into one plan and replayed per token with a single
// submission (the ExecuteWithTransfers pattern, D3D12VmExecutor.cs:298).
// The token and position come from a device control buffer [token, position]
// written by the caller before each replay (Phi4D3D12TextSession.cs:212-226).
#include "si_context.hpp"
#include "si_decode.hpp"

#include <vector>

using namespace si_abi;

namespace {

int check_fp32(si_hip_context* ctx, const char* op, const void* p, const char* what)
{
    if (!p || !aligned(p, 4))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "%s: %s must be a non-null 4-byte aligned pointer", op, what);
    return SI_HIP_OK;
}

int attention_check(si_hip_context* ctx, const si_hip_attention* a)
{
    if (!a)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "attention: null arguments");
    if (a->head_dim != 128)
        return fail(ctx, SI_HIP_ERR_UNSUPPORTED, "attention: head_dim %d (only 128 is built)", a->head_dim);
    if (a->kv_heads <= 0 || a->heads <= 0 || a->heads % a->kv_heads != 0 || a->heads / a->kv_heads > 4)
        return fail(ctx, SI_HIP_ERR_UNSUPPORTED, "attention: %d query heads over %d KV heads (group of 1..4 is built)",
                    a->heads, a->kv_heads);
    if (a->rotary_dim < 0 || a->rotary_dim > a->head_dim || (a->rotary_dim & 1))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "attention: rotary_dim %d must be even and <= head_dim", a->rotary_dim);
    if (a->capacity <= 0 || a->capacity > 16384)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "attention: capacity %d outside 1..16384", a->capacity);
    if (!a->qkv || !a->position || !a->k_cache || !a->v_cache || !a->out || !a->workspace)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "attention: null pointer");
    if (!aligned(a->qkv, 4) || !aligned(a->position, 4) || !aligned(a->k_cache, 16) || !aligned(a->v_cache, 16) ||
        !aligned(a->out, 4) || !aligned(a->workspace, 4))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "attention: misaligned pointer");
    return SI_HIP_OK;
}

si::AttentionArgs attention_args(const si_hip_attention* a)
{
    si::AttentionArgs r;
    r.qkv = a->qkv;
    r.position = a->position;
    r.k_cache = static_cast<__half*>(a->k_cache);
    r.v_cache = static_cast<__half*>(a->v_cache);
    r.out = a->out;
    r.workspace = a->workspace;
    r.heads = a->heads;
    r.kv_heads = a->kv_heads;
    r.head_dim = a->head_dim;
    r.rotary_dim = a->rotary_dim;
    r.capacity = a->capacity;
    r.max_chunks = (a->capacity + 63) / 64;
    r.rope_base = a->rope_base;
    r.rope_scale = a->rope_scale;
    return r;
}

// Device scratch of one decode program: attention partials, then argmax.
uint64_t phi4_workspace_bytes(const si_hip_phi4_model* m)
{
    const uint64_t att = static_cast<uint64_t>(si::attention_workspace_floats(m->heads, m->capacity)) * 4;
    return ((att + 255) & ~uint64_t(255)) + static_cast<uint64_t>(si::argmax_workspace_bytes());
}

int phi4_check(si_hip_context* ctx, const si_hip_phi4_model* m)
{
    if (!m)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "phi4: null model");
    if (m->layers <= 0 || !m->layer)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "phi4: no layers");
    if (m->heads * m->head_dim != m->hidden)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "phi4: heads * head_dim (%d * %d) != hidden %d", m->heads, m->head_dim,
                    m->hidden);
    if (!si::gemv_tiled_cols(m->hidden) || !si::gemv_tiled_cols(m->ffn))
        return fail(ctx, SI_HIP_ERR_UNSUPPORTED,
                    "phi4: hidden %d and ffn %d must be tiled column counts (1024/2048/3072/4096/6144/8192) "
                    "for the fused norms", m->hidden, m->ffn);
    for (int fmt : {m->weight_format, m->embed_format, m->head_format})
        if (!si::is_matrix_format(fmt))
            return fail(ctx, SI_HIP_ERR_UNSUPPORTED,
                        "phi4: tensor type %d is not a weight format of the matrix kernels (Q8_0, Q4_0, Q4_K, F16, F32)",
                        fmt);
    if (si::row_bytes(m->weight_format, m->hidden) < 0 || si::row_bytes(m->weight_format, m->ffn) < 0 ||
        si::row_bytes(m->embed_format, m->hidden) < 0 || si::row_bytes(m->head_format, m->hidden) < 0)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "phi4: hidden/ffn are not whole blocks of the weight formats");
    if (!m->embed || !m->lm_head || !m->output_norm || !m->control || !m->hidden_state || !m->qkv || !m->attn ||
        !m->gate_up || !m->logits || !m->workspace || !m->next_token)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "phi4: null buffer");
    for (int l = 0; l < m->layers; l++) {
        const si_hip_phi4_layer& L = m->layer[l];
        if (!L.attn_norm || !L.qkv || !L.o || !L.ffn_norm || !L.up || !L.down || !L.k_cache || !L.v_cache)
            return fail(ctx, SI_HIP_ERR_ARGUMENT, "phi4: layer %d has a null tensor", l);
    }
    si_hip_attention a{};
    a.head_dim = m->head_dim;
    a.heads = m->heads;
    a.kv_heads = m->kv_heads;
    a.rotary_dim = m->rotary_dim;
    a.capacity = m->capacity;
    a.qkv = m->qkv;
    a.position = m->control + 1;
    a.k_cache = m->layer[0].k_cache;
    a.v_cache = m->layer[0].v_cache;
    a.out = m->attn;
    a.workspace = static_cast<float*>(m->workspace);
    return attention_check(ctx, &a);
}

// Launches one decode step on the context stream (recorded when capturing).
// chunk_bound > 0: the attention grids cover the first chunk_bound
// 128-position chunks only (a step recorded for a range of positions).
hipError_t phi4_step(si_hip_context* ctx, const si_hip_phi4_model* m, int chunk_bound)
{
    hipStream_t s = ctx->stream;
    const int H = m->hidden;
    const int qkv_rows = H + 2 * m->kv_heads * m->head_dim;
    float* att_ws = static_cast<float*>(m->workspace);
    const uint64_t att_bytes = (static_cast<uint64_t>(si::attention_workspace_floats(m->heads, m->capacity)) * 4 + 255) &
                               ~uint64_t(255);
    void* am_ws = static_cast<uint8_t*>(m->workspace) + att_bytes;
    // the embedding row, and (every layer attends at the same position)
    // one rotary table per step, in one launch
    si_hip_attention a{};
    a.qkv = m->qkv;
    a.position = m->control + 1;
    a.out = m->attn;
    a.workspace = att_ws;
    a.heads = m->heads;
    a.kv_heads = m->kv_heads;
    a.head_dim = m->head_dim;
    a.rotary_dim = m->rotary_dim;
    a.capacity = m->capacity;
    a.rope_base = m->rope_base;
    a.rope_scale = m->rope_scale;
    hipError_t e =
        si::launch_step_start(m->embed_format, m->embed, m->vocab, H, m->control, m->hidden_state, attention_args(&a), s);
    for (int l = 0; e == hipSuccess && l < m->layers; l++) {
        const si_hip_phi4_layer& L = m->layer[l];
        si::GemvOp qkv;
        qkv.fmt = m->weight_format;
        qkv.w = L.qkv;
        qkv.x = m->hidden_state;
        qkv.y = m->qkv;
        qkv.rows = qkv_rows;
        qkv.cols = H;
        qkv.in = si::XF_RMSNORM;
        qkv.norm_weight = L.attn_norm;
        qkv.eps = m->rms_eps;
        e = si::launch_gemv_ops(&qkv, 1, s, nullptr);
        if (e != hipSuccess) break;
        a.k_cache = L.k_cache;
        a.v_cache = L.v_cache;
        si::AttentionArgs aa = attention_args(&a);
        aa.chunk_bound = chunk_bound;
        e = si::launch_attention(aa, s, false);
        if (e != hipSuccess) break;
        // hidden += W_o . attn
        e = si::launch_gemv(m->weight_format, L.o, m->attn, m->hidden_state, H, H, m->hidden_state, s, nullptr);
        if (e != hipSuccess) break;
        // act = silu(gate) * up, gate and up rows of W_up on RMSNorm(hidden)
        si::GemvOp up;
        up.fmt = m->weight_format;
        up.w = L.up;
        up.x = m->hidden_state;
        up.y = m->gate_up;
        up.rows = m->ffn;
        up.cols = H;
        up.in = si::XF_RMSNORM;
        up.out = si::OUT_SWIGLU_ROWS;
        up.norm_weight = L.ffn_norm;
        up.eps = m->rms_eps;
        e = si::launch_gemv_ops(&up, 1, s, nullptr);
        if (e != hipSuccess) break;
        // hidden += W_down . act
        e = si::launch_gemv(m->weight_format, L.down, m->gate_up, m->hidden_state, H, m->ffn, m->hidden_state, s,
                            nullptr);
    }
    if (e == hipSuccess) {
        si::GemvOp head;
        head.fmt = m->head_format;
        head.w = m->lm_head;
        head.x = m->hidden_state;
        head.y = m->logits;
        head.rows = m->vocab;
        head.cols = H;
        head.in = si::XF_RMSNORM;
        head.norm_weight = m->output_norm;
        head.eps = m->rms_eps;
        e = si::launch_gemv_ops(&head, 1, s, nullptr);
    }
    if (e == hipSuccess)
        e = si::launch_argmax(m->logits, m->vocab, am_ws, m->next_token, s);
    return e;
}

}  // namespace

extern "C" {

int si_hip_gemv_fused(si_hip_context* ctx, int format, const void* w, const float* x, float* y, int64_t rows,
                      int64_t cols, const float* residual, int xform, const float* norm_weight, float eps, int* path)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "gemv_fused: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    uint64_t wbytes = 0;
    if (const int rc = check_matrix(ctx, "gemv_fused", format, w, rows, cols, &wbytes))
        return rc;
    if (xform != SI_HIP_X_PLAIN && xform != SI_HIP_X_RMSNORM && xform != SI_HIP_X_SWIGLU)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_fused: unknown transform %d", xform);
    if (xform != SI_HIP_X_PLAIN && !si::gemv_tiled_cols(cols))
        return fail(ctx, SI_HIP_ERR_UNSUPPORTED,
                    "gemv_fused: a fused transform needs cols in {1024, 2048, 3072, 4096, 6144, 8192}, got %lld",
                    static_cast<long long>(cols));
    if (!x || !y || !aligned(y, 4) || (residual && !aligned(residual, 4)))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_fused: null or misaligned FP32 operand");
    if (xform != SI_HIP_X_PLAIN && (!aligned(x, 16) || !aligned(w, 4)))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_fused: a fused transform needs x 16-byte and W 4-byte aligned");
    if (xform == SI_HIP_X_RMSNORM && (!norm_weight || !aligned(norm_weight, 16)))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_fused: RMSNorm weight must be a 16-byte aligned pointer");
    const uint64_t ybytes = static_cast<uint64_t>(rows) * 4;
    const uint64_t xbytes = static_cast<uint64_t>(cols) * 4 * (xform == SI_HIP_X_SWIGLU ? 2 : 1);
    if (overlaps(y, ybytes, w, wbytes) || overlaps(y, ybytes, x, xbytes) ||
        (residual && residual != y && overlaps(y, ybytes, residual, ybytes)))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_fused: output overlaps an input");
    si::GemvOp op;
    op.fmt = format;
    op.w = w;
    op.x = x;
    op.y = y;
    op.rows = rows;
    op.cols = cols;
    op.residual = residual;
    op.in = xform;
    op.norm_weight = norm_weight;
    op.eps = eps;
    const hipError_t e = si::launch_gemv_ops(&op, 1, ctx->stream, path);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "gemv_fused launch");
}

int si_hip_gemv_batch(si_hip_context* ctx, const si_hip_gemv_op* ops, int count, int* paths)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "gemv_batch: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    if (!ops || count < 1 || count > 64)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_batch: need 1..64 ops, got %d", count);
    struct Range {
        const void* p;
        uint64_t n;
    };
    std::vector<std::vector<Range>> reads(count), writes(count);
    std::vector<si::GemvOp> launch(count);
    for (int i = 0; i < count; i++) {
        const si_hip_gemv_op& o = ops[i];
        if (o.reserved != 0 || o.reserved2 != 0)
            return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_batch: op %d: reserved fields must be 0", i);
        if (o.output < SI_HIP_OUT_PLAIN || o.output > SI_HIP_OUT_SIGMOID)
            return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_batch: op %d: unknown output function %d", i, o.output);
        if (o.input_xform < SI_HIP_X_PLAIN || o.input_xform > SI_HIP_X_LAYERNORM_MIX)
            return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_batch: op %d: unknown transform %d", i, o.input_xform);
        const bool swiglu_rows = o.output == SI_HIP_OUT_SWIGLU_ROWS;
        const bool ln = o.input_xform == SI_HIP_X_LAYERNORM || o.input_xform == SI_HIP_X_LAYERNORM_MIX;
        uint64_t wbytes = 0;
        if (const int rc = check_matrix(ctx, "gemv_batch", o.format, o.weight, swiglu_rows ? 2 * o.rows : o.rows,
                                        o.cols, &wbytes))
            return rc;
        if (!o.x || !o.y || !aligned(o.y, 4) || !aligned(o.x, 4) || (o.residual && !aligned(o.residual, 4)))
            return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_batch: op %d: null or misaligned FP32 operand", i);
        if (o.residual && o.output != SI_HIP_OUT_PLAIN)
            return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_batch: op %d: a residual needs the plain output", i);
        if (o.input_xform != SI_HIP_X_PLAIN) {
            if (!si::gemv_tiled_cols(o.cols))
                return fail(ctx, SI_HIP_ERR_UNSUPPORTED,
                            "gemv_batch: op %d: a fused transform needs cols in {1024, 2048, 3072, 4096, 6144, 8192}, "
                            "got %lld", i, static_cast<long long>(o.cols));
            if (!aligned(o.x, 16) || !aligned(o.weight, 4))
                return fail(ctx, SI_HIP_ERR_ARGUMENT,
                            "gemv_batch: op %d: a fused transform needs x 16-byte and W 4-byte aligned", i);
        }
        const bool need_w = o.input_xform == SI_HIP_X_RMSNORM || ln;
        if (need_w && (!o.norm_weight || !aligned(o.norm_weight, 16)))
            return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_batch: op %d: norm weight must be a 16-byte aligned pointer", i);
        if (ln && (!o.norm_bias || !aligned(o.norm_bias, 16)))
            return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_batch: op %d: norm bias must be a 16-byte aligned pointer", i);
        if (o.input_xform == SI_HIP_X_LAYERNORM_MIX &&
            (!o.mix || !o.prev || !aligned(o.mix, 16) || !aligned(o.prev, 16)))
            return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_batch: op %d: mix and prev must be 16-byte aligned pointers", i);
        if (o.norm_out && (!ln || !aligned(o.norm_out, 16)))
            return fail(ctx, SI_HIP_ERR_ARGUMENT,
                        "gemv_batch: op %d: norm_out needs a layer-norm transform and 16-byte alignment", i);
        const uint64_t cb = static_cast<uint64_t>(o.cols) * 4, yb = static_cast<uint64_t>(o.rows) * 4;
        reads[i] = {{o.weight, wbytes}, {o.x, o.input_xform == SI_HIP_X_SWIGLU ? 2 * cb : cb}};
        if (need_w) reads[i].push_back({o.norm_weight, cb});
        if (ln) reads[i].push_back({o.norm_bias, cb});
        if (o.input_xform == SI_HIP_X_LAYERNORM_MIX) {
            reads[i].push_back({o.mix, cb});
            reads[i].push_back({o.prev, cb});
        }
        writes[i] = {{o.y, yb}};
        if (o.norm_out) writes[i].push_back({o.norm_out, cb});
        // the residual may be y itself (an in-place accumulate); any other
        // overlap with a write is rejected below
        if (o.residual && o.residual != o.y) reads[i].push_back({o.residual, yb});

        si::GemvOp& op = launch[i];
        op.fmt = o.format;
        op.w = o.weight;
        op.x = o.x;
        op.y = o.y;
        op.rows = o.rows;
        op.cols = o.cols;
        op.residual = o.residual;
        op.in = o.input_xform;
        op.out = o.output;
        op.norm_weight = o.norm_weight;
        op.norm_bias = o.norm_bias;
        op.mix = o.mix;
        op.prev = o.prev;
        op.norm_out = o.norm_out;
        op.eps = o.eps;
    }
    // Pending-write rule of one barrier interval (D3D12VmSchedule.cs:74-99):
    // nothing an op writes may be read or written by any op of the batch,
    // the op itself included (except its own residual == y).
    for (int i = 0; i < count; i++)
        for (const Range& wr : writes[i])
            for (int j = 0; j < count; j++) {
                for (const Range& rd : reads[j])
                    if (overlaps(wr.p, wr.n, rd.p, rd.n))
                        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_batch: op %d writes what op %d reads", i, j);
                for (const Range& w2 : writes[j])
                    if (&w2 != &wr && overlaps(wr.p, wr.n, w2.p, w2.n))
                        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gemv_batch: ops %d and %d write overlapping memory", i, j);
            }
    const hipError_t e = si::launch_gemv_ops(launch.data(), count, ctx->stream, paths);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "gemv_batch launch");
}

int si_hip_gather_row(si_hip_context* ctx, int format, const void* table, int64_t rows, int64_t cols,
                      const int32_t* index, float* out)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "gather_row: null context");
    Enter g(ctx);
    uint64_t tbytes = 0;
    if (const int rc = check_matrix(ctx, "gather_row", format, table, rows, cols, &tbytes))
        return rc;
    if (!index || !aligned(index, 4))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gather_row: index must be a 4-byte aligned device pointer");
    if (const int rc = check_fp32(ctx, "gather_row", out, "out"))
        return rc;
    if (overlaps(out, static_cast<uint64_t>(cols) * 4, table, tbytes) ||
        overlaps(out, static_cast<uint64_t>(cols) * 4, index, 4))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "gather_row: output overlaps an input");
    const hipError_t e = si::launch_gather_row(format, table, rows, cols, index, out, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "gather_row launch");
}

int si_hip_attention_workspace_bytes(int heads, int capacity, uint64_t* bytes)
{
    if (!bytes || heads <= 0 || capacity <= 0)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "attention_workspace_bytes: bad arguments");
    *bytes = static_cast<uint64_t>(si::attention_workspace_floats(heads, capacity)) * 4;
    return SI_HIP_OK;
}

int si_hip_attention_decode(si_hip_context* ctx, const si_hip_attention* args)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "attention: null context");
    Enter g(ctx);
    if (const int rc = attention_check(ctx, args))
        return rc;
    const hipError_t e = si::launch_attention(attention_args(args), ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "attention launch");
}

int si_hip_attention_decode_noalloc(si_hip_context* ctx, const si_hip_attention* args)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "attention_noalloc: null context");
    Enter g(ctx);
    if (!args)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "attention_noalloc: null arguments");
    if (args->workspace)
        return fail(ctx, SI_HIP_ERR_ARGUMENT,
                    "attention_noalloc: workspace must be NULL (the library's device scratch is used)");
    if (args->heads > 0 && args->capacity > 0 &&
        si::attention_workspace_floats(args->heads, args->capacity) > si::ATTENTION_SCRATCH_FLOATS)
        return fail(ctx, SI_HIP_ERR_UNSUPPORTED,
                    "attention_noalloc: %d heads at capacity %d need %lld workspace bytes; the library's scratch "
                    "holds %lld (use si_hip_attention_decode with a workspace)",
                    args->heads, args->capacity,
                    static_cast<long long>(si::attention_workspace_floats(args->heads, args->capacity) * 4),
                    static_cast<long long>(si::ATTENTION_SCRATCH_FLOATS * 4));
    si_hip_attention a = *args;
    a.workspace = ctx->attention_scratch;
    if (const int rc = attention_check(ctx, &a))
        return rc;
    const hipError_t e = si::launch_attention(attention_args(&a), ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "attention_noalloc launch");
}

int si_hip_argmax_workspace_bytes(uint64_t* bytes)
{
    if (!bytes)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "argmax_workspace_bytes: null output");
    *bytes = static_cast<uint64_t>(si::argmax_workspace_bytes());
    return SI_HIP_OK;
}

int si_hip_argmax(si_hip_context* ctx, const float* values, int64_t n, void* workspace, int32_t* index)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "argmax: null context");
    Enter g(ctx);
    if (n <= 0 || n > INT32_MAX)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "argmax: count %lld out of range", static_cast<long long>(n));
    if (check_fp32(ctx, "argmax", values, "values") || check_fp32(ctx, "argmax", workspace, "workspace") ||
        check_fp32(ctx, "argmax", index, "index"))
        return SI_HIP_ERR_ARGUMENT;
    const hipError_t e = si::launch_argmax(values, n, workspace, index, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "argmax launch");
}

int si_hip_phi4_workspace_bytes(const si_hip_phi4_model* model, uint64_t* bytes)
{
    if (!model || !bytes || model->heads <= 0 || model->capacity <= 0)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "phi4_workspace_bytes: bad arguments");
    *bytes = phi4_workspace_bytes(model);
    return SI_HIP_OK;
}

int si_hip_phi4_decode(si_hip_context* ctx, const si_hip_phi4_model* model)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "phi4_decode: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    if (const int rc = phi4_check(ctx, model))
        return rc;
    const hipError_t e = phi4_step(ctx, model, 0);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "phi4 decode step");
}

int si_hip_phi4_decode_bounded(si_hip_context* ctx, const si_hip_phi4_model* model, int position_bound)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "phi4_decode_bounded: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    if (const int rc = phi4_check(ctx, model))
        return rc;
    if (position_bound < 0 || position_bound >= model->capacity)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "phi4_decode_bounded: position bound %d outside the cache (capacity %d)",
                    position_bound, model->capacity);
    if (model->rotary_dim % 16 != 0)
        return fail(ctx, SI_HIP_ERR_UNSUPPORTED,
                    "phi4_decode_bounded: rotary_dim %d (the bounded attention grid needs a multiple of 16)",
                    model->rotary_dim);
    const hipError_t e = phi4_step(ctx, model, position_bound / 128 + 1);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "phi4 decode step (bounded)");
}

}  // extern "C"
