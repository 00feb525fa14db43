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
    const float* copy2_src = nullptr;   // optional: a second such store
    float* copy2_dst = nullptr;
    // In-kernel LoRA outputs.  lora_fmt 0: w_lora, a_lora, gate and v_lora
    // are read as given.  lora_fmt Q8_0 / Q4_0: they are not read; each
    // head's workgroup forms its 64 elements of up[m] . hid[m] itself, for
    // the up matrices m = w2, a2, g2, v2 ([heads * 64, rank[m]] in that
    // format, 16-byte aligned) and their FP32 hidden vectors hid[m] (the
    // outputs of w1 with tanh, a1, g1 with sigmoid, v1; 16-byte aligned);
    // rank[3] = 0 on the first layer.  Each element is its row's block
    // products (the hidden vectors as digit planes, as the matrix-vector
    // kernels stage x) summed in order.
    int lora_fmt = 0;
    const void* up[4] = {};
    const float* hid[4] = {};
    int rank[4] = {};
};

// Limits of the in-kernel LoRA outputs: the head's rows of the four up
// matrices are staged in LDS, and a head forms at most 1536 block products
// (the sum of the ranks at most 24 blocks of 32).
constexpr int WKV_LORA_LDS_BYTES = 48 * 1024;
constexpr int WKV_LORA_MAX_ITEMS = 1536;
// Whether the in-kernel LoRA outputs take these arguments (format, ranks,
// 16-byte aligned up matrices and hidden vectors, the limits above).
bool wkv_lora_supported(const WkvArgs& a);

hipError_t launch_rwkv_wkv(const WkvArgs& a, hipStream_t s);
// out = ((x - mean) * (1 / sqrt(var + eps))) * w + b over n <= 8192 values,
// one workgroup.
hipError_t launch_layernorm(const float* x, const float* w, const float* b, int n, float eps, float* out,
                            hipStream_t s);
// The same LayerNorm over row *index of a GGUF table [rows, cols] (the
// embedding gather fused in; an index outside the table gives NaN).
hipError_t launch_gather_layernorm(int fmt, const void* table, int64_t rows, int64_t cols, const int32_t* index,
                                   const float* w, const float* b, float eps, float* out, hipStream_t s);
// out[b][r] = sum_c m[b][r][c] * v[b][c] in FP32 (core.tensor.batched-mat-vec).
hipError_t launch_batched_matvec(const float* m, const float* v, float* out, int batch, int rows, int cols,
                                 hipStream_t s);

}  // namespace si
