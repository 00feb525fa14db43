// Batched (prefill) transformer launches (si_batch.hip) shared by the C ABI.
// Every launch takes control = device int32[2] {start, valid}: rows
// 0..valid-1 of the batch are live, row r is the token at position
// start + r; rows at or past valid are left untouched.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace si {

constexpr int BATCH_MAX = 16;            // rows of a batch (the reference's prefill batch)
constexpr int BATCH_HEAD = 128;          // head size of the batched attention launches
constexpr int BATCH_GROUP_MAX = 8;       // query heads per KV head
constexpr int BATCH_CHUNK = 64;          // cache positions per attention workgroup

struct BatchRopeArgs {
    const float* qkv;          // [batch][query_size + 2 * kv_size]
    const int32_t* control;
    const float* frequencies;  // [rotary_size / 2]
    float* query;              // [batch][query_size]
    void* key_cache;           // [context][kv_size], FP32 or fp16
    void* value_cache;
    bool cache_fp16;
    int batch;
    int query_size;
    int kv_size;
    int head_size;
    int rotary_size;
    int context;
    float rope_scale;
};

struct BatchAttentionArgs {
    const float* query;          // scores: [batch][query_heads * 128]
    const float* probabilities;  // values: [batch][query_heads][context]
    const void* cache;           // key cache (scores) or value cache (values): [context][kv_heads][128]
    const int32_t* control;
    float* out;                  // scores [batch][query_heads][context] or values [batch][query_heads * 128]
    float* workspace;            // values: batch_values_workspace_floats
    bool cache_fp16;
    int batch;
    int query_heads;
    int kv_heads;
    int context;
};

int64_t batch_values_workspace_floats(int batch, int query_heads, int context);

hipError_t launch_batch_gather_rows(const float* table, int64_t table_rows, int width, const int32_t* control,
                                    float* out, int batch, hipStream_t s);
hipError_t launch_batch_rms_norm(const float* hidden, const float* residual, const float* weight, float* updated,
                                 float* out, int batch, int width, float eps, const int32_t* control, hipStream_t s);
hipError_t launch_batch_swiglu(const float* gate_up, float* out, int batch, int width, const int32_t* control,
                               hipStream_t s);
hipError_t launch_batch_rope_kv_write(const BatchRopeArgs& a, hipStream_t s);
hipError_t launch_batch_gqa_scores(const BatchAttentionArgs& a, hipStream_t s);
hipError_t launch_batch_causal_softmax(const float* scores, float* probabilities, int batch, int heads, int context,
                                       const int32_t* control, hipStream_t s);
hipError_t launch_batch_gqa_values(const BatchAttentionArgs& a, hipStream_t s);
// scores, causal softmax and values in two launches: a.cache is the key cache,
// a.query the queries, a.out the values' output, a.workspace the values'
// workspace; a.probabilities is not used.
hipError_t launch_batch_gqa_attention(const BatchAttentionArgs& a, const void* value_cache, hipStream_t s);
hipError_t launch_batch_select_last(const float* input, float* out, int batch, int width, const int32_t* control,
                                    hipStream_t s);
// y[t][o] = sum_k x[t][k] W[o][k] for t < min(batch, valid), FP32 products
// and sums (v_mfma_f32_16x16x4_f32), W in any matrix format, columns % 32 == 0
// (Q4_K: % 256).
hipError_t launch_batch_matvec(int fmt, const void* w, const float* x, float* y, int batch, int64_t rows,
                               int64_t cols, const int32_t* control, hipStream_t s);

}  // namespace si
