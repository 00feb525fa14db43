// RWKV-7 decode-step operators shared by the C ABI and the RWKV-7 program
// builder.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace si {

constexpr int RWKV_HEAD = 64;   // head size the WKV kernel takes

// Time-mix core of one layer (PortableRwkv7GraphProvider.cs:224-276), all
// vectors [heads * 64].
struct WkvArgs {
    int heads;
    int first_layer;            // 1: value = v and v_first = v; 0: value gated toward v_first
    const float* r;
    const float* k;
    const float* v;
    const float* w_lora;        // w2 . tanh(w1 . xw)
    const float* a_lora;        // a2 . (a1 . xa)
    const float* gate;          // g2 . sigmoid(g1 . xg)
    const float* v_lora;        // v2 . (v1 . xv), read when !first_layer
    const float* w0;
    const float* a0;
    const float* v0;
    const float* k_k;
    const float* k_a;
    const float* r_k;
    const float* lnx_weight;
    const float* lnx_bias;
    float* v_first;
    float* state;               // [heads][64][64], updated in place
    float* out;
    const float* copy_src;      // optional: copy_dst = copy_src ([heads * 64]), a state store
    float* copy_dst;
};

hipError_t launch_rwkv_wkv(const WkvArgs& a, hipStream_t s);
// out = ((x - mean) * (1 / sqrt(var + eps))) * w + b over n <= 8192 values,
// one workgroup.
hipError_t launch_layernorm(const float* x, const float* w, const float* b, int n, float eps, float* out,
                            hipStream_t s);
// out[b][r] = sum_c m[b][r][c] * v[b][c] in FP32 (core.tensor.batched-mat-vec).
hipError_t launch_batched_matvec(const float* m, const float* v, float* out, int batch, int rows, int cols,
                                 hipStream_t s);

}  // namespace si
