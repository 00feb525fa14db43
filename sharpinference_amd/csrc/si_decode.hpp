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
    // > 0: the chunk grid covers only the first chunk_bound 128-position
    // chunks, whose K / V rows are requested before the position returns;
    // a position at or past chunk_bound * 128 yields NaN outputs and no
    // cache append.  0: the grid covers the whole cache.
    int chunk_bound = 0;
};

int64_t attention_workspace_floats(int heads, int capacity);

// Largest attention workspace the library's own device scratch holds (the
// allocation-free entry point): 524288 floats = 2 MiB per GPU, enough for
// heads * ceil(capacity / 64) <= 4032 (e.g. 24 heads up to 10752 cached
// positions, 32 heads up to 8064).
constexpr int64_t ATTENTION_SCRATCH_FLOATS = 524288;
// Device address of that scratch on `device` (looked up once per device,
// with the device current; the caller makes it current).
hipError_t attention_scratch(int device, float** out);
int64_t argmax_workspace_bytes();
hipError_t launch_gather_row(int fmt, const void* table, int64_t rows, int64_t cols, const int32_t* index, float* out,
                             hipStream_t s);
// The per-step preparation (rotary table of the position) runs first when
// `prep`; a program that attends several layers at one position prepares
// once and passes prep = false afterwards.
hipError_t launch_attention_prep(const AttentionArgs& a, hipStream_t s);
// One launch of the decode step's start: launch_gather_row's embedding row
// and launch_attention_prep's rotary table.
hipError_t launch_step_start(int fmt, const void* table, int64_t rows, int64_t cols, const int32_t* index, float* out,
                             const AttentionArgs& a, hipStream_t s);
hipError_t launch_attention(const AttentionArgs& a, hipStream_t s, bool prep = true);
hipError_t launch_argmax(const float* values, int64_t n, void* workspace, int32_t* out, hipStream_t s);

}  // namespace si
