/*
 * CPU oracle for the quantized matrix-vector hot path (see oracle.h).
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/, the smoke check and the CPU
 * baseline leg of bench.py as the checker.  The product library never links
 * or loads it.
 *
 * Built with -ffp-contract=off so that every FP32 multiply and subtract below
 * rounds on its own; the Q4_K decode depends on that order.
 */
#include "oracle.h"

#include <math.h>
#if defined(__F16C__)
#include <immintrin.h>
#endif
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------ */
/* scalar conversions                                                        */
/* ------------------------------------------------------------------------ */

static float bits_to_float(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t float_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* IEEE binary16 -> binary32, exact (every half is a float). */
float orc_half_to_float(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        /* zero or subnormal: man * 2^-24, exact in binary32 */
        float v = (float)man * 0x1.0p-24f;
        return bits_to_float(float_to_bits(v) | sign);
    }
    if (exp == 31)
        return bits_to_float(sign | 0x7f800000u | (man << 13) | (man ? 0x00400000u : 0u));
    return bits_to_float(sign | ((exp + 112u) << 23) | (man << 13));
}

/* binary32 -> binary16 with round-to-nearest-even. */
/* The same exact conversion through the F16C instruction (x86-64-v3). */
static inline float half_to_float_fast(uint16_t h)
{
#if defined(__F16C__)
    return _cvtsh_ss(h);
#else
    return orc_half_to_float(h);
#endif
}

uint16_t orc_float_to_half(float f)
{
    uint32_t x = float_to_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u)
        return sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u);
    if (ax >= 0x477ff000u)          /* >= 65520: rounds to infinity */
        return sign | 0x7c00u;
    if (ax < 0x38800000u) {         /* below 2^-14: half subnormal (or zero) */
        float a = bits_to_float(ax) * 16777216.0f;   /* exact: scale by 2^24 */
        uint32_t m = (uint32_t)nearbyintf(a);        /* default mode: nearest even */
        return sign | (uint16_t)m;
    }
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u)))
        h++;
    return sign | (uint16_t)h;
}

float orc_bf16_to_float(uint16_t b) { return bits_to_float((uint32_t)b << 16); }

uint16_t orc_float_to_bf16(float f)
{
    uint32_t x = float_to_bits(f);
    if ((x & 0x7fffffffu) > 0x7f800000u)
        return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

/* ------------------------------------------------------------------------ */
/* sizes (GgufModelFile.cs:301-331, plus the GGUF v3 Q4_K super-block)        */
/* ------------------------------------------------------------------------ */

int orc_block_elems(int format)
{
    switch (format) {
    case ORC_F32: case ORC_F16: return 1;
    case ORC_Q4_0: case ORC_Q8_0: return 32;
    case ORC_Q4_K: return 256;
    default: return 0;
    }
}

int orc_block_bytes(int format)
{
    switch (format) {
    case ORC_F32: return 4;
    case ORC_F16: return 2;
    case ORC_Q4_0: return 18;
    case ORC_Q8_0: return 34;
    case ORC_Q4_K: return 144;
    default: return 0;
    }
}

int64_t orc_row_bytes(int format, int64_t cols)
{
    int be = orc_block_elems(format);
    if (be == 0 || cols <= 0 || cols % be != 0)
        return -1;
    return cols / be * orc_block_bytes(format);
}

int64_t orc_tensor_bytes(int format, int64_t rows, int64_t cols)
{
    int64_t rb = orc_row_bytes(format, cols);
    if (rb < 0 || rows <= 0)
        return -1;
    return rb * rows;
}

/* ------------------------------------------------------------------------ */
/* seeded generators (splitmix64 stream + Box-Muller)                        */
/* ------------------------------------------------------------------------ */

static uint64_t sm64(uint64_t* s)
{
    uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

static double u01_open(uint64_t* s) { return (double)((sm64(s) >> 11) + 1) * 0x1.0p-53; }

static double normal(uint64_t* s)
{
    double u1 = u01_open(s), u2 = u01_open(s);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

static int uniform_int(uint64_t* s, int lo, int hi)
{
    return lo + (int)(sm64(s) % (uint64_t)(hi - lo + 1));
}

void orc_gen_q8_0(uint64_t seed, int64_t rows, int64_t cols, double sigma, uint8_t* out)
{
    uint64_t s = seed;
    int64_t nblocks = rows * (cols / 32);
    for (int64_t b = 0; b < nblocks; b++) {
        uint8_t* blk = out + b * 34;
        uint16_t d = orc_float_to_half((float)(fabs(normal(&s) * sigma) / 127.0));
        memcpy(blk, &d, 2);
        for (int i = 0; i < 32; i++)
            blk[2 + i] = (uint8_t)(int8_t)uniform_int(&s, -127, 127);
    }
}

void orc_gen_q4_0(uint64_t seed, int64_t rows, int64_t cols, double sigma, uint8_t* out)
{
    uint64_t s = seed;
    int64_t nblocks = rows * (cols / 32);
    for (int64_t b = 0; b < nblocks; b++) {
        uint8_t* blk = out + b * 18;
        uint16_t d = orc_float_to_half((float)(fabs(normal(&s) * sigma) / 8.0));
        memcpy(blk, &d, 2);
        for (int i = 0; i < 16; i++) {
            int lo = uniform_int(&s, 0, 15), hi = uniform_int(&s, 0, 15);
            blk[2 + i] = (uint8_t)(lo | (hi << 4));
        }
    }
}

/* Packs eight 6-bit (scale, min) pairs into the 12 GGUF Q4_K scale bytes:
 * bytes 0-3 hold sc[0..3] in bits 0-5 and sc[4..7] bits 4-5 in bits 6-7;
 * bytes 4-7 hold m[0..3] in bits 0-5 and m[4..7] bits 4-5 in bits 6-7;
 * bytes 8-11 hold sc[4..7] bits 0-3 (low nibble) and m[4..7] bits 0-3
 * (high nibble). */
static void pack_q4_k_scales(const int* sc, const int* m, uint8_t* q)
{
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((m[j + 4] & 15) << 4));
    }
}

void orc_gen_q4_k(uint64_t seed, int64_t rows, int64_t cols, double sigma, uint8_t* out)
{
    uint64_t s = seed;
    int64_t nblocks = rows * (cols / 256);
    for (int64_t b = 0; b < nblocks; b++) {
        uint8_t* blk = out + b * 144;
        uint16_t d = orc_float_to_half((float)(fabs(normal(&s) * sigma) / 504.0));
        uint16_t dmin = orc_float_to_half((float)(fabs(normal(&s) * sigma) / 63.0));
        memcpy(blk, &d, 2);
        memcpy(blk + 2, &dmin, 2);
        int sc[8], m[8];
        for (int j = 0; j < 8; j++) {
            sc[j] = uniform_int(&s, 0, 63);
            m[j] = uniform_int(&s, 0, 63);
        }
        pack_q4_k_scales(sc, m, blk + 4);
        for (int i = 0; i < 128; i++)
            blk[16 + i] = (uint8_t)uniform_int(&s, 0, 255);
    }
}

void orc_gen_quant(int format, uint64_t seed, int64_t rows, int64_t cols, double sigma, uint8_t* out)
{
    switch (format) {
    case ORC_Q8_0: orc_gen_q8_0(seed, rows, cols, sigma, out); break;
    case ORC_Q4_0: orc_gen_q4_0(seed, rows, cols, sigma, out); break;
    case ORC_Q4_K: orc_gen_q4_k(seed, rows, cols, sigma, out); break;
    default: break;
    }
}

void orc_gen_normal_f32(uint64_t seed, int64_t n, double mean, double sigma, float* out)
{
    uint64_t s = seed;
    for (int64_t i = 0; i < n; i++)
        out[i] = (float)(mean + sigma * normal(&s));
}

void orc_gen_normal_f16(uint64_t seed, int64_t n, double mean, double sigma, uint16_t* out)
{
    uint64_t s = seed;
    for (int64_t i = 0; i < n; i++)
        out[i] = orc_float_to_half((float)(mean + sigma * normal(&s)));
}

void orc_gen_normal_bf16(uint64_t seed, int64_t n, double mean, double sigma, uint16_t* out)
{
    uint64_t s = seed;
    for (int64_t i = 0; i < n; i++)
        out[i] = orc_float_to_bf16((float)(mean + sigma * normal(&s)));
}

/* ------------------------------------------------------------------------ */
/* block decoding (GGML dequantize_row_q8_0 / _q4_0 / _q4_K)                 */
/* ------------------------------------------------------------------------ */

static uint16_t load_u16(const uint8_t* p) { uint16_t v; memcpy(&v, p, 2); return v; }

void orc_q4_k_scale_min(int j, const uint8_t* q, int* sc, int* m)
{
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

static void dequant_q8_0_block(const uint8_t* blk, float* out)
{
    float d = orc_half_to_float(load_u16(blk));
    for (int i = 0; i < 32; i++)
        out[i] = d * (float)(int8_t)blk[2 + i];
}

static void dequant_q4_0_block(const uint8_t* blk, float* out)
{
    float d = orc_half_to_float(load_u16(blk));
    for (int i = 0; i < 16; i++) {
        out[i] = d * (float)((blk[2 + i] & 0xF) - 8);
        out[i + 16] = d * (float)((blk[2 + i] >> 4) - 8);
    }
}

static void dequant_q4_k_block(const uint8_t* blk, float* out)
{
    float d = orc_half_to_float(load_u16(blk));
    float dmin = orc_half_to_float(load_u16(blk + 2));
    const uint8_t* scales = blk + 4;
    const uint8_t* q = blk + 16;
    for (int c = 0; c < 4; c++) {
        int sc, m;
        orc_q4_k_scale_min(2 * c, scales, &sc, &m);
        float d1 = d * (float)sc, m1 = dmin * (float)m;
        orc_q4_k_scale_min(2 * c + 1, scales, &sc, &m);
        float d2 = d * (float)sc, m2 = dmin * (float)m;
        for (int l = 0; l < 32; l++) {
            float p = d1 * (float)(q[32 * c + l] & 0xF);
            out[64 * c + l] = p - m1;
        }
        for (int l = 0; l < 32; l++) {
            float p = d2 * (float)(q[32 * c + l] >> 4);
            out[64 * c + 32 + l] = p - m2;
        }
    }
}

void orc_dequant_row(int format, const uint8_t* row, int64_t cols, float* out)
{
    switch (format) {
    case ORC_Q8_0:
        for (int64_t b = 0; b < cols / 32; b++) dequant_q8_0_block(row + b * 34, out + b * 32);
        break;
    case ORC_Q4_0:
        for (int64_t b = 0; b < cols / 32; b++) dequant_q4_0_block(row + b * 18, out + b * 32);
        break;
    case ORC_Q4_K:
        for (int64_t b = 0; b < cols / 256; b++) dequant_q4_k_block(row + b * 144, out + b * 256);
        break;
    case ORC_F16:
        for (int64_t i = 0; i < cols; i++) out[i] = orc_half_to_float(load_u16(row + 2 * i));
        break;
    case ORC_F32:
        memcpy(out, row, (size_t)cols * 4);
        break;
    default:
        break;
    }
}

int orc_dequant(int format, const uint8_t* w, int64_t rows, int64_t cols, float* out)
{
    int64_t rb = orc_row_bytes(format, cols);
    if (rb < 0 || rows <= 0)
        return -1;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++)
        orc_dequant_row(format, w + r * rb, cols, out + r * cols);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* matrix-vector products                                                    */
/* ------------------------------------------------------------------------ */

float orc_dot_f32(const float* a, const float* b, int64_t n)
{
    float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int k = 0; k < 8; k++)
            lane[k] = fmaf(a[i + k], b[i + k], lane[k]);
    for (int k = 0; i < n; i++, k++)
        lane[k] = fmaf(a[i], b[i], lane[k]);
    return ((lane[0] + lane[4]) + (lane[2] + lane[6])) + ((lane[1] + lane[5]) + (lane[3] + lane[7]));
}

/* Thresholds of CpuHalfMatrixOperators.cs:8-9. */
#define PARALLEL_ROW_THRESHOLD 64
#define PARALLEL_ELEMENT_THRESHOLD 65536
#define SERIAL_CHUNK 1024

int orc_gemv_cpuvm(int format, const uint8_t* w, const float* x, float* y,
                   int64_t rows, int64_t cols, int threads)
{
    int64_t rb = orc_row_bytes(format, cols);
    if (rb < 0 || rows <= 0)
        return -1;
    int be = orc_block_elems(format);
    if (rows < PARALLEL_ROW_THRESHOLD || rows * cols < PARALLEL_ELEMENT_THRESHOLD) {
        /* serial: bounded conversion chunks summed in FP32 (:15-22, :123-137) */
        float scratch[SERIAL_CHUNK];
        for (int64_t r = 0; r < rows; r++) {
            float sum = 0.0f;
            for (int64_t c0 = 0; c0 < cols; c0 += SERIAL_CHUNK) {
                int64_t len = cols - c0 < SERIAL_CHUNK ? cols - c0 : SERIAL_CHUNK;
                orc_dequant_row(format, w + r * rb + (c0 / be) * orc_block_bytes(format), len, scratch);
                sum += orc_dot_f32(scratch, x + c0, len);
            }
            y[r] = sum;
        }
        return 0;
    }
    /* parallel rows: dequantise the row into FP32 scratch, then dot (:24-41) */
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel num_threads(nt)
#endif
    {
        float* scratch = (float*)malloc((size_t)cols * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int64_t r = 0; r < rows; r++) {
            orc_dequant_row(format, w + r * rb, cols, scratch);
            y[r] = orc_dot_f32(scratch, x, cols);
        }
        free(scratch);
    }
    (void)threads;
    return 0;
}

int orc_gemv_f64(int format, const uint8_t* w, const float* x, double* y,
                 int64_t rows, int64_t cols)
{
    int64_t rb = orc_row_bytes(format, cols);
    if (rb < 0 || rows <= 0)
        return -1;
#pragma omp parallel
    {
        float* scratch = (float*)malloc((size_t)cols * sizeof(float));
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; r++) {
            orc_dequant_row(format, w + r * rb, cols, scratch);
            double s = 0.0;
            for (int64_t c = 0; c < cols; c++)
                s += (double)scratch[c] * (double)x[c];
            y[r] = s;
        }
        free(scratch);
    }
    return 0;
}

int orc_gemm_prefill_cpuvm(int format, const uint8_t* w, const uint16_t* x_bf16, float* y,
                           int64_t m, int64_t rows, int64_t cols, int threads)
{
    if (orc_row_bytes(format, cols) < 0 || rows <= 0 || m <= 0)
        return -1;
    float* xf = (float*)malloc((size_t)cols * sizeof(float));
    int rc = 0;
    for (int64_t t = 0; t < m && rc == 0; t++) {
        for (int64_t c = 0; c < cols; c++)
            xf[c] = orc_bf16_to_float(x_bf16[t * cols + c]);
        rc = orc_gemv_cpuvm(format, w, xf, y + t * rows, rows, cols, threads);
    }
    free(xf);
    return rc;
}

int orc_gemm_prefill_f64(int format, const uint8_t* w, const uint16_t* x_bf16, double* y,
                         int64_t m, int64_t rows, int64_t cols)
{
    int64_t rb = orc_row_bytes(format, cols);
    if (rb < 0 || rows <= 0 || m <= 0)
        return -1;
    float* wf = (float*)malloc((size_t)(rows * cols) * sizeof(float));
    double* xd = (double*)malloc((size_t)(m * cols) * sizeof(double));
    orc_dequant(format, w, rows, cols, wf);
    for (int64_t i = 0; i < m * cols; i++)
        xd[i] = (double)orc_bf16_to_float(x_bf16[i]);
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t t = 0; t < m; t++)
        for (int64_t r = 0; r < rows; r++) {
            const float* wr = wf + r * cols;
            const double* xr = xd + t * cols;
            double s = 0.0;
            for (int64_t c = 0; c < cols; c++)
                s += (double)wr[c] * xr[c];
            y[t * rows + r] = s;
        }
    free(wf);
    free(xd);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Phi-4 decode step                                                          */
/* ------------------------------------------------------------------------ */

void orc_rmsnorm(const float* x, const float* w, int n, float eps, float* out)
{
    float sum = 0.0f;
    for (int i = 0; i < n; i++)
        sum += x[i] * x[i];
    float scale = 1.0f / sqrtf(sum / (float)n + eps);
    for (int i = 0; i < n; i++)
        out[i] = x[i] * scale * w[i];
}

void orc_rope(float* values, int heads, int head_dim, int rotary_dim, int position, float base, float scale)
{
    int half = rotary_dim / 2;
    for (int h = 0; h < heads; h++) {
        float* hv = values + (int64_t)h * head_dim;
        for (int i = 0; i < half; i++) {
            float frequency = 1.0f / powf(base, 2.0f * (float)i / (float)rotary_dim);
            float angle = (float)position * frequency;
            float c = cosf(angle) * scale;
            float sn = sinf(angle) * scale;
            float left = hv[i], right = hv[i + half];
            hv[i] = left * c - right * sn;
            hv[i + half] = right * c + left * sn;
        }
    }
}

void orc_attention(const float* q, const uint16_t* k_cache, const uint16_t* v_cache, int heads, int kv_heads,
                   int head_dim, int capacity, int length, float* out)
{
    int group = heads / kv_heads;
    /* heads are independent: one thread per head, each with the sequential
       per-head order of ComputeAttention */
#pragma omp parallel for schedule(static)
    for (int h = 0; h < heads; h++) {
        int g = h / group;
        const uint16_t* kc = k_cache + (int64_t)g * capacity * head_dim;
        const uint16_t* vc = v_cache + (int64_t)g * capacity * head_dim;
        float* scores = (float*)malloc((size_t)length * sizeof(float));
        float* o = out + (int64_t)h * head_dim;
        for (int d = 0; d < head_dim; d++)
            o[d] = 0.0f;
        float maximum = -INFINITY;
        for (int t = 0; t < length; t++) {
            float score = 0.0f;
            for (int d = 0; d < head_dim; d++)
                score += q[h * head_dim + d] * half_to_float_fast(kc[(int64_t)t * head_dim + d]);
            score /= sqrtf((float)head_dim);
            scores[t] = score;
            maximum = fmaxf(maximum, score);
        }
        float denominator = 0.0f;
        for (int t = 0; t < length; t++) {
            scores[t] = expf(scores[t] - maximum);
            denominator += scores[t];
        }
        for (int t = 0; t < length; t++) {
            float p = scores[t] / denominator;
            for (int d = 0; d < head_dim; d++)
                o[d] += p * half_to_float_fast(vc[(int64_t)t * head_dim + d]);
        }
        free(scores);
    }
}

int orc_argmax(const float* v, int64_t n)
{
    /* first index of the maximum; NaN never wins; all-NaN gives 0 */
    int64_t best = -1;
    float bv = -INFINITY;
    for (int64_t i = 0; i < n; i++)
        if (v[i] > bv || (v[i] == bv && best < 0)) {
            bv = v[i];
            best = i;
        }
    return best < 0 ? 0 : (int)best;
}

int orc_phi4_decode_step(const orc_phi4_model* m, int token, int position, float* logits, int threads)
{
    int H = m->hidden, D = m->head_dim, KVH = m->kv_heads;
    int qkv_rows = H + 2 * KVH * D;
    if (token < 0 || token >= m->vocab || position < 0 || position >= m->capacity)
        return -1;
    float* hidden = (float*)malloc((size_t)H * sizeof(float));
    float* normed = (float*)malloc((size_t)H * sizeof(float));
    float* qkv = (float*)malloc((size_t)qkv_rows * sizeof(float));
    float* attn = (float*)malloc((size_t)H * sizeof(float));
    float* proj = (float*)malloc((size_t)H * sizeof(float));
    float* gate_up = (float*)malloc((size_t)2 * m->ffn * sizeof(float));
    /* Embed (:44-53): the token's row of the embedding table */
    orc_dequant_row(m->embed_format, m->embed + (int64_t)token * orc_row_bytes(m->embed_format, H), H, hidden);
    for (int l = 0; l < m->layers; l++) {
        orc_rmsnorm(hidden, m->attn_norm[l], H, m->rms_eps, normed);
        orc_gemv_cpuvm(m->weight_format, m->qkv[l], normed, qkv, qkv_rows, H, threads);
        orc_rope(qkv, m->heads, D, m->rotary_dim, position, m->rope_base, m->rope_scale);
        orc_rope(qkv + H, KVH, D, m->rotary_dim, position, m->rope_base, m->rope_scale);
        /* Phi4KeyValueCache.Append with fp16 storage */
        for (int g = 0; g < KVH; g++)
            for (int d = 0; d < D; d++) {
                int64_t slot = ((int64_t)g * m->capacity + position) * D + d;
                m->k_cache[l][slot] = orc_float_to_half(qkv[H + g * D + d]);
                m->v_cache[l][slot] = orc_float_to_half(qkv[H + KVH * D + g * D + d]);
            }
        orc_attention(qkv, m->k_cache[l], m->v_cache[l], m->heads, KVH, D, m->capacity, position + 1, attn);
        orc_gemv_cpuvm(m->weight_format, m->o[l], attn, proj, H, H, threads);
        for (int i = 0; i < H; i++)
            hidden[i] += proj[i];
        orc_rmsnorm(hidden, m->ffn_norm[l], H, m->rms_eps, normed);
        orc_gemv_cpuvm(m->weight_format, m->up[l], normed, gate_up, 2 * m->ffn, H, threads);
        for (int i = 0; i < m->ffn; i++) {
            float gate = gate_up[i];
            gate_up[i] = gate / (1.0f + expf(-gate)) * gate_up[m->ffn + i];
        }
        orc_gemv_cpuvm(m->weight_format, m->down[l], gate_up, proj, H, m->ffn, threads);
        for (int i = 0; i < H; i++)
            hidden[i] += proj[i];
    }
    orc_rmsnorm(hidden, m->output_norm, H, m->rms_eps, normed);
    orc_gemv_cpuvm(m->head_format, m->lm_head, normed, logits, m->vocab, H, threads);
    free(hidden); free(normed); free(qkv); free(attn); free(proj); free(gate_up);
    return orc_argmax(logits, m->vocab);
}

/* ------------------------------------------------------------------------ */
/* RWKV-7 decode step (PortableRwkv7GraphProvider.cs)                        */
/* ------------------------------------------------------------------------ */

float orc_sum_f32(const float* a, int64_t n)
{
    float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int k = 0; k < 8; k++)
            lane[k] += a[i + k];
    for (int k = 0; i < n; i++, k++)
        lane[k] += a[i];
    return ((lane[0] + lane[4]) + (lane[2] + lane[6])) + ((lane[1] + lane[5]) + (lane[3] + lane[7]));
}

void orc_layernorm(const float* x, const float* w, const float* b, int n, float eps, float* out)
{
    float* c = (float*)malloc((size_t)n * sizeof(float));
    float mean = orc_sum_f32(x, n) / (float)n;                     /* ReduceMean :129 */
    for (int i = 0; i < n; i++)
        c[i] = x[i] - mean;                                        /* centered */
    for (int i = 0; i < n; i++)
        out[i] = c[i] * c[i];                                      /* Square */
    float var = orc_sum_f32(out, n) / (float)n;
    float inv = 1.0f / sqrtf(var + eps);                           /* ReciprocalSquareRoot(var + eps) */
    for (int i = 0; i < n; i++) {
        float v = c[i] * inv;
        if (w) v = v * w[i];                                       /* Affine :180-182 */
        if (b) v = v + b[i];
        out[i] = v;
    }
    free(c);
}

static float sigmoidf_(float v) { return 1.0f / (1.0f + expf(-v)); }

void orc_rwkv7_wkv_update(int heads, int n, float* state, const float* r, const float* decay, const float* key,
                          const float* value, const float* kn, const float* adapt, float* out)
{
    float* proj = (float*)malloc((size_t)n * sizeof(float));
    float* ak = (float*)malloc((size_t)n * sizeof(float));
    for (int h = 0; h < heads; h++) {
        float* S = state + (int64_t)h * n * n;
        const int o = h * n;
        for (int j = 0; j < n; j++)
            ak[j] = kn[o + j] * adapt[o + j];                      /* adaptedKey :254 */
        for (int i = 0; i < n; i++)
            proj[i] = orc_dot_f32(S + (int64_t)i * n, kn + o, n);  /* BatchedMatVec(state, kn) :256 */
        for (int i = 0; i < n; i++)
            for (int j = 0; j < n; j++) {
                float* s = S + (int64_t)i * n + j;
                float negp = 0.0f - proj[i];
                *s = (*s * decay[o + j] + value[o + i] * key[o + j]) + negp * ak[j];
            }
        for (int i = 0; i < n; i++)
            out[o + i] = orc_dot_f32(S + (int64_t)i * n, r + o, n); /* BatchedMatVec(updated, r) :270 */
    }
    free(proj);
    free(ak);
}

void orc_rwkv7_wkv(const orc_rwkv7_wkv_args* a)
{
    const int H = a->heads, N = a->head_size, D = H * N;
    float* decay = (float*)calloc((size_t)D, sizeof(float));
    float* adapt = (float*)calloc((size_t)D, sizeof(float));
    float* kn = (float*)calloc((size_t)D, sizeof(float));
    float* key = (float*)calloc((size_t)D, sizeof(float));
    float* value = (float*)calloc((size_t)D, sizeof(float));
    float* tmp = (float*)calloc((size_t)D, sizeof(float));
    float* y = (float*)calloc((size_t)D, sizeof(float));
    for (int i = 0; i < D; i++) {
        decay[i] = expf(-0.606531f * sigmoidf_(a->w_lora[i] + a->w0[i]));   /* :232-234 */
        adapt[i] = sigmoidf_(a->a_lora[i] + a->a0[i]);                      /* :235-237 */
    }
    for (int h = 0; h < H; h++) {                                           /* :241-246 */
        const int o = h * N;
        for (int j = 0; j < N; j++) {
            float sk = a->k[o + j] * a->k_k[o + j];
            tmp[o + j] = sk * sk;
        }
        float squares = orc_sum_f32(tmp + o, N);
        float inv = 1.0f / sqrtf(squares > 1e-24f ? squares : 1e-24f);
        for (int j = 0; j < N; j++)
            kn[o + j] = (a->k[o + j] * a->k_k[o + j]) * inv;
    }
    for (int i = 0; i < D; i++) {
        float ka = a->k[i] * a->k_a[i];                                     /* :247-248 */
        key[i] = (a->k[i] + adapt[i] * ka) - ka;
        if (a->first_layer) {                                               /* :249-257 */
            value[i] = a->v[i];
            a->v_first[i] = a->v[i];
        } else {
            float vg = sigmoidf_(a->v_lora[i] + a->v0[i]);
            value[i] = a->v[i] + (a->v_first[i] - a->v[i]) * vg;
        }
    }
    orc_rwkv7_wkv_update(H, N, a->state, a->r, decay, key, value, kn, adapt, y);
    for (int h = 0; h < H; h++) {
        const int o = h * N;
        orc_layernorm(y + o, a->lnx_weight + o, a->lnx_bias + o, N, 64e-5f, tmp + o);   /* :272-273, :171-178 */
        for (int j = 0; j < N; j++)
            y[o + j] = (key[o + j] * a->r[o + j]) * a->r_k[o + j];         /* bonus factors :274 */
        float bonus = orc_sum_f32(y + o, N);
        for (int j = 0; j < N; j++)
            a->out[o + j] = (tmp[o + j] + value[o + j] * bonus) * a->gate[o + j];   /* :276 */
    }
    free(decay); free(adapt); free(kn); free(key); free(value); free(tmp); free(y);
}

static void mix_(const float* x, const float* prev, const float* mix, int n, float* out)
{
    for (int i = 0; i < n; i++)
        out[i] = x[i] + (prev[i] - x[i]) * mix[i];                      /* Mix :183-184 */
}

int orc_rwkv7_decode_step(const orc_rwkv7_model* m, int token, float* logits, int threads)
{
    const int D = m->hidden, F = m->ffn, fmt = m->weight_format;
    if (token < 0 || token >= m->vocab)
        return -1;
    const int rmax = m->rank_g > m->rank_w ? m->rank_g : m->rank_w;
    float* x = (float*)malloc((size_t)D * sizeof(float));
    float* row = (float*)malloc((size_t)D * sizeof(float));
    float* normed = (float*)malloc((size_t)D * sizeof(float));
    float* xm = (float*)malloc((size_t)6 * D * sizeof(float));
    float* r = (float*)malloc((size_t)D * sizeof(float));
    float* k = (float*)malloc((size_t)D * sizeof(float));
    float* v = (float*)malloc((size_t)D * sizeof(float));
    float* wl = (float*)malloc((size_t)D * sizeof(float));
    float* al = (float*)malloc((size_t)D * sizeof(float));
    float* g = (float*)malloc((size_t)D * sizeof(float));
    float* vl = (float*)malloc((size_t)D * sizeof(float));
    float* h1 = (float*)malloc((size_t)(rmax > m->rank_v ? rmax : m->rank_v) * sizeof(float) + 4 * (size_t)m->rank_a);
    float* att = (float*)malloc((size_t)D * sizeof(float));
    float* proj = (float*)malloc((size_t)D * sizeof(float));
    float* v_first = (float*)malloc((size_t)D * sizeof(float));
    float* hid = (float*)malloc((size_t)F * sizeof(float));
    /* x = ln0(emb[token]) (:191-193) */
    orc_dequant_row(m->embed_format, m->embed + (int64_t)token * orc_row_bytes(m->embed_format, D), D, row);
    orc_layernorm(row, m->ln0_weight, m->ln0_bias, D, 1e-5f, x);
    for (int l = 0; l < m->layers; l++) {
        const orc_rwkv7_layer* L = &m->layer[l];
        orc_layernorm(x, L->ln1_weight, L->ln1_bias, D, 1e-5f, normed);   /* :202-203 */
        for (int t = 0; t < 6; t++)                                     /* xr, xw, xk, xv, xa, xg :205-210 */
            mix_(normed, L->att_prev, L->mix + (int64_t)t * D, D, xm + (int64_t)t * D);
        const float* xr = xm, *xw = xm + D, *xk = xm + 2 * D, *xv = xm + 3 * D, *xa = xm + 4 * D, *xg = xm + 5 * D;
        orc_gemv_cpuvm(fmt, L->receptance, xr, r, D, D, threads);
        orc_gemv_cpuvm(fmt, L->key, xk, k, D, D, threads);
        orc_gemv_cpuvm(fmt, L->value, xv, v, D, D, threads);
        orc_gemv_cpuvm(fmt, L->w1, xw, h1, m->rank_w, D, threads);          /* decay LoRA :214-216 */
        for (int i = 0; i < m->rank_w; i++)
            h1[i] = tanhf(h1[i]);
        orc_gemv_cpuvm(fmt, L->w2, h1, wl, D, m->rank_w, threads);
        orc_gemv_cpuvm(fmt, L->a1, xa, h1, m->rank_a, D, threads);          /* adaptation LoRA :220-222 */
        orc_gemv_cpuvm(fmt, L->a2, h1, al, D, m->rank_a, threads);
        orc_gemv_cpuvm(fmt, L->g1, xg, h1, m->rank_g, D, threads);          /* gate LoRA :223-224 */
        for (int i = 0; i < m->rank_g; i++)
            h1[i] = sigmoidf_(h1[i]);
        orc_gemv_cpuvm(fmt, L->g2, h1, g, D, m->rank_g, threads);
        if (l > 0) {                                                        /* value LoRA :252-254 */
            orc_gemv_cpuvm(fmt, L->v1, xv, h1, m->rank_v, D, threads);
            orc_gemv_cpuvm(fmt, L->v2, h1, vl, D, m->rank_v, threads);
        }
        orc_rwkv7_wkv_args wa = {m->heads, m->head_size, l == 0, r, k, v, wl, al, g, vl, L->w0, L->a0, L->v0,
                                 L->k_k, L->k_a, L->r_k, L->lnx_weight, L->lnx_bias, v_first, L->wkv, att};
        orc_rwkv7_wkv(&wa);
        orc_gemv_cpuvm(fmt, L->output, att, proj, D, D, threads);           /* :277 */
        for (int i = 0; i < D; i++)
            x[i] += proj[i];
        memcpy(L->att_prev, normed, (size_t)D * sizeof(float));             /* Store :278 */
        orc_layernorm(x, L->ln2_weight, L->ln2_bias, D, 1e-5f, normed);     /* :280-281 */
        mix_(normed, L->ffn_prev, L->ffn_mix, D, row);                      /* :282-283 */
        orc_gemv_cpuvm(fmt, L->ffn_key, row, hid, F, D, threads);
        for (int i = 0; i < F; i++) {
            float h = hid[i] > 0.0f ? hid[i] : (hid[i] != hid[i] ? hid[i] : 0.0f);   /* Relu :284-285 */
            hid[i] = h * h;                                                 /* Square :287 */
        }
        orc_gemv_cpuvm(fmt, L->ffn_value, hid, proj, D, F, threads);
        for (int i = 0; i < D; i++)
            x[i] += proj[i];
        memcpy(L->ffn_prev, normed, (size_t)D * sizeof(float));             /* Store :288 */
    }
    orc_layernorm(x, m->ln_out_weight, m->ln_out_bias, D, 1e-5f, normed);   /* :290 */
    orc_gemv_cpuvm(m->head_format, m->head, normed, logits, m->vocab, D, threads);
    free(x); free(row); free(normed); free(xm); free(r); free(k); free(v); free(wl); free(al); free(g); free(vl);
    free(h1); free(att); free(proj); free(v_first); free(hid);
    return orc_argmax(logits, m->vocab);
}

/* ------------------------------------------------------------------------ */

double orc_now_seconds(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

int orc_max_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
