// Op-by-op transformer launches (si_transformer.hip) shared by the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace si {

struct RopeKvWriteArgs {
    const float* qkv;          // [query_size + 2 * kv_size]
    const int32_t* position;   // device scalar: the token's row
    const float* frequencies;  // [rotary_size / 2]
    float* query;              // [query_size]
    void* key_cache;           // [context][kv_size], FP32 or fp16
    void* value_cache;
    bool cache_fp16;
    int query_size;
    int kv_size;               // kv_heads * head_size
    int head_size;
    int rotary_size;
    int context;
    float rope_scale;
};

struct GqaArgs {
    const float* query;        // [query_heads * head_size]
    const void* key_cache;     // [context][kv_heads][head_size]
    const void* value_cache;
    const int32_t* position;
    float* output;             // [query_heads * head_size]
    bool cache_fp16;
    int query_heads;
    int kv_heads;
    int head_size;             // 64, 128 or 256
    int context;
    int chunks;                // ceil(context / 64)
    float* workspace;          // gqa_workspace_floats: per head and chunk (max, sum, weighted values)
};

int64_t gqa_workspace_floats(int query_heads, int head_size, int context);

hipError_t launch_rms_norm(const float* x, const float* w, float* out, int n, float eps, hipStream_t s);
hipError_t launch_residual_rms_norm(const float* hidden, const float* residual, const float* w, float* updated,
                                    float* out, int n, float eps, hipStream_t s);
hipError_t launch_swiglu(const float* gate_up, float* out, int64_t n, hipStream_t s);
hipError_t launch_rope_kv_write(const RopeKvWriteArgs& a, hipStream_t s);
hipError_t launch_gqa(const GqaArgs& a, hipStream_t s);

}  // namespace si
