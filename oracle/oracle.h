/*
 * CPU oracle for the quantized matrix-vector hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library links, loads or
 * calls this code; only tests/, the smoke check and the CPU-baseline leg of
 * bench.py use it, and only as the checker / the timed CPU baseline.
 *
 * What it restates:
 *   - GGUF tensor byte sizes: SharpInference.Gguf/GgufModelFile.cs:301-331
 *     (Q4_0 = 18 B / 32, Q8_0 = 34 B / 32).  Q4_K (144 B / 256) is rejected
 *     by the reference (GgufModelFile.cs:320); its size comes from the GGUF v3
 *     block definition.
 *   - Block decoding (dequantisation) of Q8_0, Q4_0, Q4_K: the reference has
 *     no decoder (it only mirrors the type ids, GgufModelFile.cs:24-46).  The
 *     algorithm is the public GGML block format of GGUF version 3 (the only
 *     version the reference reader accepts, GgufModelFile.cs:51,85), as
 *     implemented by ggml's dequantize_row_q8_0 / _q4_0 / _q4_K.  ggml is not
 *     a dependency of the reference and is absent from this image.
 *   - The CpuVm matrix-vector product with FP16 weights:
 *     SharpInference.Backends.Cpu/CpuHalfMatrixOperators.cs:11-43,123-137
 *     (dequantised row -> FP32 scratch -> FP32 dot), emitted for core.mat-vec
 *     by SharpInference.Instructions.Cpu/CpuTierZeroInstruction.cs:47-55.
 *   - An fp64 recomputation from the exactly dequantised FP32 weights, the
 *     same kind of truth the reference tests use
 *     (SharpInference.Tests/GpuMatVecTests.cs:33-34).
 */
#ifndef SI_ORACLE_H
#define SI_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type ids (GgufModelFile.cs:24-46). */
enum {
    ORC_F32 = 0,
    ORC_F16 = 1,
    ORC_Q4_0 = 2,
    ORC_Q8_0 = 8,
    ORC_Q4_K = 12,
};

/* ---- scalar conversions ---------------------------------------------- */
float orc_half_to_float(uint16_t h);
uint16_t orc_float_to_half(float f);      /* round to nearest even */
float orc_bf16_to_float(uint16_t b);
uint16_t orc_float_to_bf16(float f);      /* round to nearest even */

/* ---- sizes ------------------------------------------------------------ */
/* Bytes of a [rows, cols] tensor of `format`; -1 if cols is not a multiple of
 * the block size or the format is unknown. */
int64_t orc_tensor_bytes(int format, int64_t rows, int64_t cols);
int64_t orc_row_bytes(int format, int64_t cols);
int orc_block_elems(int format);
int orc_block_bytes(int format);

/* ---- seeded synthetic generators -------------------------------------- */
/* Q8_0: q ~ U{-127..127}, d = fp16(|N(0, sigma)| / 127). */
void orc_gen_q8_0(uint64_t seed, int64_t rows, int64_t cols, double sigma, uint8_t* out);
/* Q4_0: nibble ~ U{0..15}, d = fp16(|N(0, sigma)| / 8). */
void orc_gen_q4_0(uint64_t seed, int64_t rows, int64_t cols, double sigma, uint8_t* out);
/* Q4_K: q ~ U{0..15}, 6-bit sc/m ~ U{0..63},
 * d = fp16(|N(0, sigma)| / 504), dmin = fp16(|N(0, sigma)| / 63). */
void orc_gen_q4_k(uint64_t seed, int64_t rows, int64_t cols, double sigma, uint8_t* out);
void orc_gen_quant(int format, uint64_t seed, int64_t rows, int64_t cols, double sigma, uint8_t* out);
/* n values ~ N(mean, sigma) as fp32 / fp16 / bf16 bit patterns. */
void orc_gen_normal_f32(uint64_t seed, int64_t n, double mean, double sigma, float* out);
void orc_gen_normal_f16(uint64_t seed, int64_t n, double mean, double sigma, uint16_t* out);
void orc_gen_normal_bf16(uint64_t seed, int64_t n, double mean, double sigma, uint16_t* out);

/* ---- block decoding ----------------------------------------------------- */
void orc_dequant_row(int format, const uint8_t* row, int64_t cols, float* out);
int orc_dequant(int format, const uint8_t* w, int64_t rows, int64_t cols, float* out);
/* Q4_K 6-bit (scale, min) of sub-block j (0..7) from the 12 packed bytes. */
void orc_q4_k_scale_min(int j, const uint8_t* scales, int* sc, int* m);

/* ---- matrix-vector products -------------------------------------------- */
/* CpuVm order: per row, dequantise into an FP32 scratch and take the FP32
 * dot with x; small problems run serially over 1024-element chunks, large
 * ones run rows in parallel on `threads` threads (<=0: all cores). */
int orc_gemv_cpuvm(int format, const uint8_t* w, const float* x, float* y,
                   int64_t rows, int64_t cols, int threads);
/* fp64 truth over the exactly dequantised weights. */
int orc_gemv_f64(int format, const uint8_t* w, const float* x, double* y,
                 int64_t rows, int64_t cols);
/* FP32 dot in the oracle's fixed order: 8 interleaved fused multiply-add lane accumulators
 * (element i feeds lane i % 8), then ((l0+l4)+(l2+l6))+((l1+l5)+(l3+l7)). */
float orc_dot_f32(const float* a, const float* b, int64_t n);

/* ---- batched prefill product ------------------------------------------- */
/* Y[m, r] = sum_c X[m, c] * W[r, c] with X bf16, following the
 * transpose_right branch of CpuInstructionNumerics.MatrixMultiply
 * (CpuInstructionNumerics.cs:66-77): one CpuVm matvec per token row. */
int orc_gemm_prefill_cpuvm(int format, const uint8_t* w, const uint16_t* x_bf16, float* y,
                           int64_t m, int64_t rows, int64_t cols, int threads);
int orc_gemm_prefill_f64(int format, const uint8_t* w, const uint16_t* x_bf16, double* y,
                         int64_t m, int64_t rows, int64_t cols);

/* ---- Phi-4 decode step (Phi4TextModel.cs) ------------------------------- */
/* RmsNorm (:107-128): sum of squares in order, scale = 1/sqrt(sum/n + eps),
 * out = x * scale * w. */
void orc_rmsnorm(const float* x, const float* w, int n, float eps, float* out);
/* ApplyRotary (:212-229) over `heads` heads of head_dim values in place. */
void orc_rope(float* values, int heads, int head_dim, int rotary_dim, int position, float base, float scale);
/* ComputeAttention (:231-273) for one token over `length` cached rows of an
 * fp16 cache laid out [kv_heads][capacity][head_dim]. */
void orc_attention(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, int heads, int kv_heads,
                   int head_dim, int capacity, int length, float* out);
/* First index of the maximum (transformer.argmax). */
int orc_argmax(const float* v, int64_t n);

typedef struct orc_phi4_model {
    int layers, hidden, heads, kv_heads, head_dim, rotary_dim, ffn, vocab, capacity;
    int weight_format, embed_format, head_format;
    float rms_eps, rope_base, rope_scale;
    const uint8_t* embed;
    const uint8_t* lm_head;
    const float* output_norm;
    const float* const* attn_norm;   /* per layer */
    const uint8_t* const* qkv;
    const uint8_t* const* o;
    const float* const* ffn_norm;
    const uint8_t* const* up;
    const uint8_t* const* down;
    uint16_t* const* k_cache;        /* fp16 [kv_heads][capacity][head_dim] per layer */
    uint16_t* const* v_cache;
} orc_phi4_model;

/* One decode step (Phi4TextSession.ForwardToken, :329-344 with ForwardLayer
 * :59-93 and GetLogits :95-105, untied Q8_0 head): writes logits[vocab],
 * appends this token's fp16 K/V at `position`, returns the argmax. */
int orc_phi4_decode_step(const orc_phi4_model* m, int token, int position, float* logits, int threads);

/* ---- RWKV-7 decode step (PortableRwkv7GraphProvider.cs:199-290) -------- */
/* Sum of n floats: 8 lanes in order, fixed merge (the SIMD shape of
 * TensorPrimitives.Sum, whose exact order the reference does not fix). */
float orc_sum_f32(const float* a, int64_t n);
/* Normalize + Affine (:163-170, :180-182): mean = sum/n, c = x - mean,
 * var = sum(c*c)/n, out = (c * (1/sqrt(var + eps))) * w + b.  w and b may
 * be NULL (no affine). */
void orc_layernorm(const float* x, const float* w, const float* b, int n, float eps, float* out);

/* WKV state update of `heads` heads of size n (:255-269), state
 * [heads][n][n] updated in place:
 *   proj[i] = sum_l S[i][l] kn[l]
 *   S'[i][j] = (S[i][j] * decay[j] + value[i] * key[j]) + (-proj[i]) * (kn[j] * adapt[j])
 *   out[i] = sum_j S'[i][j] r[j]            (BatchedMatVec, :270) */
void orc_rwkv7_wkv_update(int heads, int n, float* state, const float* r, const float* decay, const float* key,
                          const float* value, const float* kn, const float* adapt, float* out);

/* The whole time-mix core of one layer after its projections (:224-275):
 * decay, adaptation, key normalisation, key/value adjustment, the state
 * update above, GroupNorm (eps 64e-5) + ln_x affine, the r_k bonus and the
 * gate.  Vectors are [heads * n]; v_first is written when first_layer and
 * read otherwise. */
typedef struct orc_rwkv7_wkv_args {
    int heads, head_size, first_layer;
    const float* r, *k, *v;
    const float* w_lora, *a_lora, *gate, *v_lora;     /* w2.tanh(w1.xw), a2.(a1.xa), g2.sigmoid(g1.xg), v2.(v1.xv) */
    const float* w0, *a0, *v0, *k_k, *k_a, *r_k, *lnx_weight, *lnx_bias;
    float* v_first;
    float* state;
    float* out;
} orc_rwkv7_wkv_args;
void orc_rwkv7_wkv(const orc_rwkv7_wkv_args* a);

typedef struct orc_rwkv7_layer {
    const float* ln1_weight, *ln1_bias, *ln2_weight, *ln2_bias;
    const float* mix;                                   /* x_rwkvag [6][hidden]: r, w, k, v, a, g */
    const uint8_t* receptance, *key, *value, *output;   /* [hidden, hidden] */
    const uint8_t* w1, *w2, *a1, *a2, *g1, *g2, *v1, *v2;   /* [rank, hidden] / [hidden, rank] */
    const float* w0, *a0, *v0, *k_k, *k_a, *r_k, *lnx_weight, *lnx_bias;
    const float* ffn_mix;                               /* ffn.x_k [hidden] */
    const uint8_t* ffn_key, *ffn_value;                 /* [ffn, hidden], [hidden, ffn] */
    float* att_prev, *ffn_prev;                         /* state [hidden] */
    float* wkv;                                         /* state [heads][head_size][head_size] */
} orc_rwkv7_layer;

typedef struct orc_rwkv7_model {
    int layers, hidden, heads, head_size, ffn, vocab;
    int rank_w, rank_a, rank_v, rank_g;
    int weight_format, embed_format, head_format;
    const uint8_t* embed;                               /* [vocab, hidden] */
    const float* ln0_weight, *ln0_bias;
    const orc_rwkv7_layer* layer;
    const float* ln_out_weight, *ln_out_bias;
    const uint8_t* head;                                /* [vocab, hidden] */
} orc_rwkv7_model;

/* One token through the graph (:190-290): writes logits[vocab], updates
 * every layer's state, returns the argmax, or -1 for a token outside the
 * vocabulary. */
int orc_rwkv7_decode_step(const orc_rwkv7_model* m, int token, float* logits, int threads);

/* ---- timing helper for the CPU baseline -------------------------------- */
double orc_now_seconds(void);
int orc_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
