// C ABI of the RWKV-7 operators and the RWKV-7 token-step recorder.
//
// The recorder is the HIP form of the portable RWKV-7 forward-token graph
// (SharpInference.Architectures.Rwkv7/PortableRwkv7GraphProvider.cs:190-292),
// which the reference runs as ~90 unfused tensor nodes per layer.  Here a
// layer is six launches:
//   1. r, k, v and the w1/a1/g1/v1 LoRA inputs in one launch; each op stages
//      LayerNorm(x) mixed with att_prev by its own mix row (:202-210), w1
//      applies tanh and g1 sigmoid to their outputs (:214-224);
//   2. the w2/a2/g2/v2 LoRA outputs in one launch;
//   3. the time-mix core (decay, adaptation, key normalisation, state update,
//      readout, GroupNorm, bonus, gate; :224-276), which also stores
//      LayerNorm(x) into att_prev (:278) once every reader of att_prev ran;
//   4. x += output . att (:277);
//   5. relu(ffn_key . mix(LayerNorm(x), ffn_prev))^2 (:280-287);
//   6. x += ffn_value . hidden, storing LayerNorm(x) into ffn_prev (:288).
#include "si_context.hpp"
#include "si_decode.hpp"
#include "si_rwkv.hpp"

using namespace si_abi;

namespace {

constexpr float LN_EPS = 1e-5f;   // Normalize(x, 1e-5f), PortableRwkv7GraphProvider.cs:193,202,280,290

// Float offsets of the step's scratch vectors inside the workspace, each
// rounded up to 64 floats (256 bytes).
struct RwkvScratch {
    int64_t r, k, v, hw, ha, hg, hv, wl, al, g, vl, att, ln1, ln2, hid, v_first, emb, argmax, total_bytes;
};

RwkvScratch rwkv_scratch(const si_hip_rwkv7_model* m)
{
    RwkvScratch s{};
    int64_t at = 0;
    auto take = [&](int64_t n) {
        const int64_t o = at;
        at += (n + 63) / 64 * 64;
        return o;
    };
    const int64_t D = m->hidden;
    s.r = take(D);
    s.k = take(D);
    s.v = take(D);
    s.hw = take(m->rank_w);
    s.ha = take(m->rank_a);
    s.hg = take(m->rank_g);
    s.hv = take(m->rank_v);
    s.wl = take(D);
    s.al = take(D);
    s.g = take(D);
    s.vl = take(D);
    s.att = take(D);
    s.ln1 = take(D);
    s.ln2 = take(D);
    s.hid = take(m->ffn);
    s.v_first = take(D);
    s.emb = take(D);
    s.argmax = at;
    s.total_bytes = at * 4 + si::argmax_workspace_bytes();
    return s;
}

bool a16(const void* p) { return p && aligned(p, 16); }

int rwkv7_check(si_hip_context* ctx, const si_hip_rwkv7_model* m)
{
    if (!m)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "rwkv7: null model");
    if (m->layers < 1 || m->heads < 1 || m->hidden != m->heads * si::RWKV_HEAD || m->vocab < 1 || m->ffn < 1)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "rwkv7: need layers, heads, ffn, vocab >= 1 and hidden = heads * 64");
    if (!si::gemv_tiled_cols(m->hidden) || !si::gemv_tiled_cols(m->ffn))
        return fail(ctx, SI_HIP_ERR_UNSUPPORTED,
                    "rwkv7: hidden %d and ffn %d must be tiled column counts (1024/2048/3072/4096/6144/8192) for the "
                    "fused LayerNorm", m->hidden, m->ffn);
    if (!si::is_matrix_format(m->weight_format) || !si::is_matrix_format(m->embed_format) ||
        !si::is_matrix_format(m->head_format))
        return fail(ctx, SI_HIP_ERR_UNSUPPORTED, "rwkv7: formats must be Q8_0, Q4_0, Q4_K, F16 or F32");
    const int be = si::block_elems(m->weight_format);
    for (int rank : {m->rank_w, m->rank_a, m->rank_g, m->rank_v})
        if (rank < 1 || rank % be != 0)
            return fail(ctx, SI_HIP_ERR_ARGUMENT, "rwkv7: LoRA rank %d is not a positive multiple of %d", rank, be);
    if (si::row_bytes(m->weight_format, m->hidden) < 0 || si::row_bytes(m->weight_format, m->ffn) < 0 ||
        si::row_bytes(m->embed_format, m->hidden) < 0 || si::row_bytes(m->head_format, m->hidden) < 0)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "rwkv7: hidden/ffn are not whole blocks of the formats");
    if (!m->embed || !m->head || !m->layer || !m->control || !m->next_token || !m->logits ||
        !aligned(m->embed, 4) || !aligned(m->head, 4))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "rwkv7: null or misaligned model tensor");
    if (!a16(m->ln0_weight) || !a16(m->ln0_bias) || !a16(m->ln_out_weight) || !a16(m->ln_out_bias) ||
        !a16(m->hidden_state) || !m->workspace || !aligned(m->workspace, 256))
        return fail(ctx, SI_HIP_ERR_ARGUMENT,
                    "rwkv7: norms and hidden_state need 16-byte alignment, the workspace 256-byte alignment");
    for (int l = 0; l < m->layers; l++) {
        const si_hip_rwkv7_layer& L = m->layer[l];
        const float* vec[] = {L.ln1_weight, L.ln1_bias, L.ln2_weight, L.ln2_bias, L.mix, L.w0, L.a0, L.k_k, L.k_a,
                              L.r_k, L.lnx_weight, L.lnx_bias, L.ffn_mix, L.att_prev, L.ffn_prev, L.wkv};
        for (const float* p : vec)
            if (!a16(p))
                return fail(ctx, SI_HIP_ERR_ARGUMENT, "rwkv7: layer %d: null or misaligned FP32 vector", l);
        const void* mats[] = {L.receptance, L.key, L.value, L.output, L.w1, L.w2, L.a1, L.a2, L.g1, L.g2,
                              L.ffn_key, L.ffn_value};
        for (const void* p : mats)
            if (!p || !aligned(p, 4))
                return fail(ctx, SI_HIP_ERR_ARGUMENT, "rwkv7: layer %d: null or misaligned matrix", l);
        if (l > 0 && (!L.v1 || !L.v2 || !L.v0 || !aligned(L.v1, 4) || !aligned(L.v2, 4)))
            return fail(ctx, SI_HIP_ERR_ARGUMENT, "rwkv7: layer %d needs the value LoRA (v0, v1, v2)", l);
    }
    return 0;
}

si::GemvOp mat(int fmt, const void* w, const float* x, float* y, int64_t rows, int64_t cols)
{
    si::GemvOp op;
    op.fmt = fmt;
    op.w = w;
    op.x = x;
    op.y = y;
    op.rows = rows;
    op.cols = cols;
    return op;
}

// Launches one token step on the context stream (recorded when capturing).
hipError_t rwkv7_step(si_hip_context* ctx, const si_hip_rwkv7_model* m)
{
    hipStream_t s = ctx->stream;
    const int D = m->hidden, F = m->ffn, fmt = m->weight_format;
    const RwkvScratch o = rwkv_scratch(m);
    float* ws = static_cast<float*>(m->workspace);
    float* x = m->hidden_state;
    // x = ln0(emb[token]) (:191-193), the gather inside the LayerNorm launch
    hipError_t e = si::launch_gather_layernorm(m->embed_format, m->embed, m->vocab, D, m->control, m->ln0_weight,
                                               m->ln0_bias, LN_EPS, x, s);
    for (int l = 0; e == hipSuccess && l < m->layers; l++) {
        const si_hip_rwkv7_layer& L = m->layer[l];
        // 1. time-mix projections on mix(LayerNorm(x), att_prev, x_rwkvag row t)
        si::GemvOp a[7];
        int na = 0;
        auto tm = [&](const void* w, int row, float* y, int64_t rows, int out) {
            si::GemvOp op = mat(fmt, w, x, y, rows, D);
            op.in = si::XF_LAYERNORM_MIX;
            op.out = out;
            op.norm_weight = L.ln1_weight;
            op.norm_bias = L.ln1_bias;
            op.mix = L.mix + static_cast<int64_t>(row) * D;
            op.prev = L.att_prev;
            op.eps = LN_EPS;
            a[na++] = op;
        };
        tm(L.receptance, 0, ws + o.r, D, si::OUT_PLAIN);
        a[0].norm_out = ws + o.ln1;
        tm(L.w1, 1, ws + o.hw, m->rank_w, si::OUT_TANH);
        tm(L.key, 2, ws + o.k, D, si::OUT_PLAIN);
        tm(L.value, 3, ws + o.v, D, si::OUT_PLAIN);
        tm(L.a1, 4, ws + o.ha, m->rank_a, si::OUT_PLAIN);
        tm(L.g1, 5, ws + o.hg, m->rank_g, si::OUT_SIGMOID);
        if (l > 0)
            tm(L.v1, 3, ws + o.hv, m->rank_v, si::OUT_PLAIN);
        e = si::launch_gemv_ops(a, na, s, nullptr);
        if (e != hipSuccess) break;
        // 2. LoRA outputs: formed inside the time-mix core's kernel where it
        //    takes them (Q8_0 / Q4_0 up matrices within its LDS staging),
        //    else one launch of the four short-row products
        si::WkvArgs w{};
        w.heads = m->heads;
        w.first_layer = l == 0;
        w.lora_fmt = fmt;
        w.up[0] = L.w2;
        w.up[1] = L.a2;
        w.up[2] = L.g2;
        w.up[3] = l > 0 ? L.v2 : nullptr;
        w.hid[0] = ws + o.hw;
        w.hid[1] = ws + o.ha;
        w.hid[2] = ws + o.hg;
        w.hid[3] = l > 0 ? ws + o.hv : nullptr;
        w.rank[0] = m->rank_w;
        w.rank[1] = m->rank_a;
        w.rank[2] = m->rank_g;
        w.rank[3] = l > 0 ? m->rank_v : 0;
        if (!si::wkv_lora_supported(w)) {
            w.lora_fmt = 0;
            si::GemvOp b[4] = {mat(fmt, L.w2, ws + o.hw, ws + o.wl, D, m->rank_w),
                               mat(fmt, L.a2, ws + o.ha, ws + o.al, D, m->rank_a),
                               mat(fmt, L.g2, ws + o.hg, ws + o.g, D, m->rank_g),
                               mat(fmt, L.v2, ws + o.hv, ws + o.vl, D, m->rank_v)};
            e = si::launch_gemv_ops(b, l > 0 ? 4 : 3, s, nullptr);
            if (e != hipSuccess) break;
        }
        // 3. time-mix core; att_prev = LayerNorm(x) now that its readers ran
        w.r = ws + o.r;
        w.k = ws + o.k;
        w.v = ws + o.v;
        w.w_lora = ws + o.wl;
        w.a_lora = ws + o.al;
        w.gate = ws + o.g;
        w.v_lora = ws + o.vl;
        w.w0 = L.w0;
        w.a0 = L.a0;
        w.v0 = L.v0;
        w.k_k = L.k_k;
        w.k_a = L.k_a;
        w.r_k = L.r_k;
        w.lnx_weight = L.lnx_weight;
        w.lnx_bias = L.lnx_bias;
        w.v_first = ws + o.v_first;
        w.state = L.wkv;
        w.out = ws + o.att;
        w.copy_src = ws + o.ln1;
        w.copy_dst = L.att_prev;
        // the previous layer's ffn_prev = its LayerNorm(x) of step 5, now
        // that its FFN key product (the reader) has run; the value product
        // then carries no side copy (the last layer's store rides on the head)
        if (l > 0) {
            w.copy2_src = ws + o.ln2;
            w.copy2_dst = m->layer[l - 1].ffn_prev;
        }
        e = si::launch_rwkv_wkv(w, s);
        if (e != hipSuccess) break;
        // 4. x += output . att
        e = si::launch_gemv(fmt, L.output, ws + o.att, x, D, D, x, s, nullptr);
        if (e != hipSuccess) break;
        // 5. hidden = relu(ffn_key . mix(LayerNorm(x), ffn_prev, x_k))^2
        si::GemvOp key = mat(fmt, L.ffn_key, x, ws + o.hid, F, D);
        key.in = si::XF_LAYERNORM_MIX;
        key.out = si::OUT_RELU_SQUARE;
        key.norm_weight = L.ln2_weight;
        key.norm_bias = L.ln2_bias;
        key.mix = L.ffn_mix;
        key.prev = L.ffn_prev;
        key.eps = LN_EPS;
        key.norm_out = ws + o.ln2;
        e = si::launch_gemv_ops(&key, 1, s, nullptr);
        if (e != hipSuccess) break;
        // 6. x += ffn_value . hidden (ffn_prev = LayerNorm(x) of step 5 is
        //    stored by the next layer's time-mix core or by the head)
        si::GemvOp val = mat(fmt, L.ffn_value, ws + o.hid, x, D, F);
        val.residual = x;
        e = si::launch_gemv_ops(&val, 1, s, nullptr);
    }
    if (e == hipSuccess) {   // logits = head . ln_out(x) (:290-291)
        si::GemvOp head = mat(m->head_format, m->head, x, m->logits, m->vocab, D);
        head.in = si::XF_LAYERNORM;
        head.norm_weight = m->ln_out_weight;
        head.norm_bias = m->ln_out_bias;
        head.eps = LN_EPS;
        head.copy_src = ws + o.ln2;   // the last layer's ffn_prev
        head.copy_dst = m->layer[m->layers - 1].ffn_prev;
        head.copy_n = D;
        e = si::launch_gemv_ops(&head, 1, s, nullptr);
    }
    if (e == hipSuccess)
        e = si::launch_argmax(m->logits, m->vocab, ws + o.argmax, m->next_token, s);
    return e;
}

}  // namespace

extern "C" {

int si_hip_batched_matvec(si_hip_context* ctx, const float* matrix, const float* vector, float* out, int batch,
                          int rows, int cols)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "batched_matvec: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    if (!matrix || !vector || !out || batch < 1 || rows < 1 || cols < 1)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "batched_matvec: null operand or empty shape");
    const uint64_t ob = static_cast<uint64_t>(batch) * rows * 4;
    if (overlaps(out, ob, matrix, ob * cols) || overlaps(out, ob, vector, static_cast<uint64_t>(batch) * cols * 4))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "batched_matvec: output overlaps an input");
    const hipError_t e = si::launch_batched_matvec(matrix, vector, out, batch, rows, cols, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "batched_matvec launch");
}

int si_hip_layernorm(si_hip_context* ctx, const float* x, const float* weight, const float* bias, int n, float eps,
                     float* out)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "layernorm: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    if (!x || !weight || !bias || !out || n < 1 || n > 8192)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "layernorm: null operand or n %d outside 1..8192", n);
    const uint64_t nb = static_cast<uint64_t>(n) * 4;
    if ((out != x && overlaps(out, nb, x, nb)) || overlaps(out, nb, weight, nb) || overlaps(out, nb, bias, nb))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "layernorm: output overlaps an input (other than out == x)");
    const hipError_t e = si::launch_layernorm(x, weight, bias, n, eps, out, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "layernorm launch");
}

int si_hip_rwkv7_wkv(si_hip_context* ctx, const si_hip_rwkv7_wkv_args* a)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "rwkv7_wkv: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    if (!a || a->heads < 1)
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "rwkv7_wkv: null arguments or heads < 1");
    const float* in[] = {a->r, a->k, a->v, a->w_lora, a->a_lora, a->gate, a->w0, a->a0, a->k_k, a->k_a, a->r_k,
                         a->lnx_weight, a->lnx_bias};
    for (const float* p : in)
        if (!p || !aligned(p, 4))
            return fail(ctx, SI_HIP_ERR_ARGUMENT, "rwkv7_wkv: null or misaligned input vector");
    if (!a->first_layer && (!a->v_lora || !a->v0))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "rwkv7_wkv: a later layer needs v_lora and v0");
    if (!a->v_first || !a->out || !aligned(a->out, 4) || !a16(a->state))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "rwkv7_wkv: null output, v_first, or state not 16-byte aligned");
    const uint64_t vb = static_cast<uint64_t>(a->heads) * si::RWKV_HEAD * 4, sb = vb * si::RWKV_HEAD;
    for (const float* p : in)
        if (overlaps(a->out, vb, p, vb) || overlaps(a->state, sb, p, vb) || overlaps(a->v_first, vb, p, vb))
            return fail(ctx, SI_HIP_ERR_ARGUMENT, "rwkv7_wkv: an output overlaps an input");
    if (overlaps(a->out, vb, a->state, sb) || overlaps(a->out, vb, a->v_first, vb) ||
        overlaps(a->state, sb, a->v_first, vb))
        return fail(ctx, SI_HIP_ERR_ARGUMENT, "rwkv7_wkv: out, state and v_first overlap");
    si::WkvArgs w{};
    w.heads = a->heads;
    w.first_layer = a->first_layer ? 1 : 0;
    w.r = a->r;
    w.k = a->k;
    w.v = a->v;
    w.w_lora = a->w_lora;
    w.a_lora = a->a_lora;
    w.gate = a->gate;
    w.v_lora = a->v_lora;
    w.w0 = a->w0;
    w.a0 = a->a0;
    w.v0 = a->v0;
    w.k_k = a->k_k;
    w.k_a = a->k_a;
    w.r_k = a->r_k;
    w.lnx_weight = a->lnx_weight;
    w.lnx_bias = a->lnx_bias;
    w.v_first = a->v_first;
    w.state = a->state;
    w.out = a->out;
    const hipError_t e = si::launch_rwkv_wkv(w, ctx->stream);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "rwkv7_wkv launch");
}

int si_hip_rwkv7_workspace_bytes(const si_hip_rwkv7_model* model, uint64_t* bytes)
{
    if (!model || !bytes || model->hidden < 1 || model->ffn < 1 || model->rank_w < 1 || model->rank_a < 1 ||
        model->rank_g < 1 || model->rank_v < 1)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "rwkv7_workspace_bytes: null or incomplete model");
    *bytes = static_cast<uint64_t>(rwkv_scratch(model).total_bytes);
    return SI_HIP_OK;
}

int si_hip_rwkv7_decode(si_hip_context* ctx, const si_hip_rwkv7_model* model)
{
    if (!ctx)
        return fail(nullptr, SI_HIP_ERR_ARGUMENT, "rwkv7_decode: null context");
    Enter g(ctx);
    if (g.err != hipSuccess)
        return hip_fail(ctx, g.err, "hipSetDevice");
    if (const int rc = rwkv7_check(ctx, model))
        return rc;
    const hipError_t e = rwkv7_step(ctx, model);
    return e == hipSuccess ? SI_HIP_OK : hip_fail(ctx, e, "rwkv7 decode step");
}

}  // extern "C"
