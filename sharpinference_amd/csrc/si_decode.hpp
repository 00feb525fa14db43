// Decode-step operators shared by the C ABI and the Phi-4 program builder.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace si {

// Grouped-query attention for one new token over an fp16 KV cache laid out
// [kv_heads][capacity][head_dim].  qkv = [q (heads*128) | k (kv_heads*128) |
// v (kv_heads*128)] before the rotary embedding; `position` is a device
// scalar (the new token's index, also its cache slot).
struct AttentionArgs {
    const float* qkv;
    const int32_t* position;
    __half* k_cache;
    __half* v_cache;
    float* out;            // [heads * 128]
    float* workspace;      // attention_workspace_floats(heads, capacity)
    int heads;
    int kv_heads;
    int head_dim;          // 128
    int rotary_dim;        // even, <= head_dim
    int capacity;
    int max_chunks;        // ceil(capacity / 64)
    float rope_base;
    float rope_scale;
};

int64_t attention_workspace_floats(int heads, int capacity);
int64_t argmax_workspace_bytes();
hipError_t launch_gather_row(int fmt, const void* table, int64_t rows, int64_t cols, const int32_t* index, float* out,
                             hipStream_t s);
// The per-step preparation (rotary table of the position) runs first when
// `prep`; a program that attends several layers at one position prepares
// once and passes prep = false afterwards.
hipError_t launch_attention_prep(const AttentionArgs& a, hipStream_t s);
hipError_t launch_attention(const AttentionArgs& a, hipStream_t s, bool prep = true);
hipError_t launch_argmax(const float* values, int64_t n, void* workspace, int32_t* out, hipStream_t s);

}  // namespace si
