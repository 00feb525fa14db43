/*
 * libsharpinference_hip — C ABI of the MI355X (gfx950) backend for
 * SharpInference's quantized matrix-vector hot path.
 *
 * The managed side of SharpInference binds these entry points by P/Invoke
 * from a HIP executor that mirrors SharpInference.Backends.D3D12Vm's
 * D3D12VmExecutor, one [DllImport] per entry point below.  The
 * reference has no native layer, so every entry point below names the
 * managed member whose job it takes over.
 *
 * Conventions
 *   - Every function returns an si_hip_status (0 = success).  On failure the
 *     context's message is set and si_hip_last_error(ctx) returns it; nothing
 *     falls back to another path (doc/vm-execution-program.md:16,57 of the
 *     reference: execution failures never trigger a silent retry).
 *   - Device pointers are plain `void*` from si_hip_alloc (or any device
 *     allocation of the same GPU).  Sizes are bytes unless named otherwise.
 *   - All work is ordered on the context's single HIP stream (default
 *     priority).  A context is locked internally: calls on one context from
 *     several threads serialise, like D3D12VmExecutor's `gate`
 *     (D3D12VmExecutor.cs:153,285,307).
 *   - Matrices are GGUF tensors [rows, cols] with `cols` contiguous
 *     (GGUF ne0 = cols, ne1 = rows), kept in their native block layout.
 */
#ifndef SHARPINFERENCE_HIP_H
#define SHARPINFERENCE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SI_HIP_ABI_VERSION 1

typedef struct si_hip_context si_hip_context;
typedef struct si_hip_plan si_hip_plan;

typedef enum si_hip_status {
    SI_HIP_OK = 0,
    SI_HIP_ERR_ARGUMENT = 1,      /* ArgumentException / ArgumentOutOfRangeException */
    SI_HIP_ERR_UNSUPPORTED = 2,   /* NotSupportedException (e.g. unknown tensor type) */
    SI_HIP_ERR_ADAPTATION = 3,    /* InstructionAdaptationException (shape/signature) */
    SI_HIP_ERR_DEVICE = 4,        /* HIP runtime failure */
    SI_HIP_ERR_OUT_OF_MEMORY = 5,
    SI_HIP_ERR_STATE = 6,         /* call not valid in the context's current state */
    SI_HIP_ERR_FORMAT = 7,        /* InvalidDataException: malformed or truncated GGUF data */
    SI_HIP_ERR_IO = 8,            /* the file cannot be opened or mapped */
} si_hip_status;

/* GGUF tensor type ids, as GgufModelTensorType (GgufModelFile.cs:24-46). */
typedef enum si_hip_format {
    SI_HIP_F32 = 0,
    SI_HIP_F16 = 1,
    SI_HIP_Q4_0 = 2,
    SI_HIP_Q8_0 = 8,
    SI_HIP_Q4_K = 12,
    SI_HIP_BF16 = 30,
} si_hip_format;

/* ---- library and device --------------------------------------------------- */

/* SI_HIP_ABI_VERSION of the loaded library. */
int si_hip_abi_version(void);

/* Number of visible HIP devices (no context needed). */
int si_hip_device_count(int* count);

/* Selects `device` and creates a context with its own stream.
 * Replaces: D3D12VmDeviceFactory adapter selection + the executor's queue and
 * fence creation (D3D12VmExecutor.cs:80-86). */
int si_hip_init(int device, si_hip_context** out);

/* Destroys the context (waits for its stream first).  NULL is accepted.
 * Replaces: D3D12VmExecutor.Dispose. */
int si_hip_destroy(si_hip_context* ctx);

/* Message of the last failed call on `ctx` (or of the calling thread when
 * ctx is NULL).  Valid until the next call on the same context/thread. */
const char* si_hip_last_error(const si_hip_context* ctx);

/* ---- memory ----------------------------------------------------------------- */

/* Bytes of a [rows, cols] tensor of `format`; fails (ARGUMENT) when cols is
 * not a whole number of blocks.  Replaces: GgufModelFile.GetByteLength
 * (GgufModelFile.cs:301-331), extended with Q4_K (144 bytes / 256). */
int si_hip_tensor_bytes(int format, int64_t rows, int64_t cols, uint64_t* bytes);

/* Device buffer of `bytes` (256-byte aligned).  Replaces: the executor's
 * one committed resource per slot (D3D12VmExecutor.cs:93-97). */
int si_hip_alloc(si_hip_context* ctx, uint64_t bytes, void** device_ptr);
int si_hip_free(si_hip_context* ctx, void* device_ptr);

/* Synchronous host -> device copy of raw bytes (GGUF blocks are uploaded
 * as-is, never repacked).  Replaces: D3D12VmExecutor.Upload
 * (D3D12VmExecutor.cs:595-625). */
int si_hip_upload(si_hip_context* ctx, void* device_dst, const void* host_src, uint64_t bytes);

/* Synchronous device -> host copy.  Replaces: D3D12VmExecutor.Readback
 * (D3D12VmExecutor.cs:682-696). */
int si_hip_readback(si_hip_context* ctx, void* host_dst, const void* device_src, uint64_t bytes);

/* Device -> device copy, ordered on the context stream. */
int si_hip_copy(si_hip_context* ctx, void* device_dst, const void* device_src, uint64_t bytes);

/* Fills `count` 32-bit words with `value` by a kernel (no memset nodes, so
 * it may be recorded into a plan). */
int si_hip_fill_u32(si_hip_context* ctx, void* device_dst, uint32_t value, uint64_t count);

/* Checksum of a device buffer: parts[0..SI_HIP_CHECKSUM_PARTS) receive
 * partial sums (mod 2^32) of the 32-bit words of device_src, whose total is
 * the buffer's word sum; one streaming read of `bytes` (a non-zero multiple
 * of 4; src 16-byte aligned), e.g. to check uploaded tensors against a host
 * checksum without reading them back.  No counterpart in the reference; a
 * plain read of known size also gives the read bandwidth a kernel of the
 * same bytes can reach. */
#define SI_HIP_CHECKSUM_PARTS 1024
int si_hip_checksum(si_hip_context* ctx, const void* device_src, uint64_t bytes, uint32_t* parts);

/* Waits for all work queued on the context.  Replaces: the executor's fence
 * wait after a submission (Submit / WaitForCompletion, D3D12VmExecutor.cs:875-890). */
int si_hip_sync(si_hip_context* ctx);

/* ---- hot path ---------------------------------------------------------------- */

/* y[rows] = W[rows, cols] . x[cols] (+ residual[rows] when residual != NULL),
 * W in GGUF Q8_0 / Q4_0 / Q4_K block layout, x, y, residual FP32.  FP32
 * arithmetic and accumulation.  `path` (optional) receives 1 for the tiled
 * gfx950 kernel, 2 for the any-shape kernel (one wave per row) and 3 for the
 * short-row kernel (rows of at most 32 blocks and 2048 columns, one lane per
 * block).
 * Replaces: the core.mat-vec instruction (cooperative form
 * GpuTierZeroInstruction.cs:44-89 on D3D12, CpuInstructionNumerics.MatVec
 * CpuInstructionNumerics.cs:16-23 on CpuVm) for block-quantized weights,
 * which the reference rejects (TierZeroOperationContracts.cs:161). */
int si_hip_gemv(si_hip_context* ctx, int format, const void* w, const float* x, float* y,
                int64_t rows, int64_t cols, const float* residual, int* path);

/* Batched prefill product Y[m, rows] = X[m, cols] . W[rows, cols]^T: m token
 * rows of bf16 activations (16-byte aligned) against a block-quantized W,
 * FP32 output (one row of `rows` values per token), FP32 accumulation on
 * MFMA; W is decoded exactly and rounded to bf16 for the matrix cores.
 * W and X must each be smaller than 4 GiB (UNSUPPORTED otherwise).
 * Replaces: the transpose_right matrix multiply of the CpuVm path
 * (CpuInstructionNumerics.MatrixMultiply, CpuInstructionNumerics.cs:66-77)
 * and the batched prefill matvec of the D3D12 transformer program
 * (GpuBatchTransformerInstructions.cs:224-279). */
int si_hip_gemm_prefill(si_hip_context* ctx, int format, const void* w, const void* x_bf16, float* y,
                        int64_t m, int64_t rows, int64_t cols);

/* out[rows, cols] = exact FP32 values of the blocks of W.  Test and
 * inspection entry point for the block decoder used by the products.
 * Replaces: the FP16 -> FP32 row conversion step of the CPU matvec
 * (CpuHalfMatrixOperators.cs:34-36), for quantized blocks. */
int si_hip_dequant(si_hip_context* ctx, int format, const void* w, float* out, int64_t rows, int64_t cols);

/* ---- decode-step operators ------------------------------------------------------ */

/* Transforms of x fused into the staging of a GEMV. */
typedef enum si_hip_xform {
    SI_HIP_X_PLAIN = 0,
    SI_HIP_X_RMSNORM = 1,        /* x_i * (1 / sqrt(sum(x^2) / cols + eps)) * norm_weight_i   */
    SI_HIP_X_SWIGLU = 2,         /* x = [gate | up] (2 * cols values): gate / (1 + exp(-gate)) * up */
    SI_HIP_X_LAYERNORM = 3,      /* ((x - mean) * (1 / sqrt(var + eps))) * norm_weight + norm_bias */
    SI_HIP_X_LAYERNORM_MIX = 4,  /* ln = LAYERNORM(x); ln + (prev - ln) * mix                   */
} si_hip_xform;

/* Functions applied to each output value of a GEMV. */
typedef enum si_hip_output {
    SI_HIP_OUT_PLAIN = 0,        /* y = W.x (+ residual)                                        */
    SI_HIP_OUT_SWIGLU_ROWS = 1,  /* W = [gate rows; up rows] (2 * rows rows): g / (1 + exp(-g)) * u */
    SI_HIP_OUT_RELU_SQUARE = 2,  /* max(v, 0)^2, NaN kept                                       */
    SI_HIP_OUT_TANH = 3,
    SI_HIP_OUT_SIGMOID = 4,      /* 1 / (1 + exp(-v))                                            */
} si_hip_output;

/* si_hip_gemv with a transform of x applied on the fly (x itself is not
 * modified).  Replaces the RMSNorm (Phi4TextModel.cs:107-128) and SwiGLU
 * (Phi4TextModel.cs:84-89) steps that precede a projection, and the
 * transformer.rms-norm / swiglu dispatches of the D3D12 decode program
 * (Phi4D3D12TextSession.cs:870-912).  xform is PLAIN, RMSNORM or SWIGLU;
 * transforms need cols in {1024, 2048, 3072, 4096, 6144, 8192}. */
int si_hip_gemv_fused(si_hip_context* ctx, int format, const void* w, const float* x, float* y,
                      int64_t rows, int64_t cols, const float* residual, int xform,
                      const float* norm_weight, float eps, int* path);

/* One product of si_hip_gemv_batch: y = output(W . input_xform(x)). */
typedef struct si_hip_gemv_op {
    int32_t format;              /* SI_HIP_Q8_0 / Q4_0 / Q4_K / F16 / F32                      */
    int32_t input_xform;         /* si_hip_xform                                               */
    int32_t output;              /* si_hip_output                                              */
    int32_t reserved;            /* 0                                                          */
    const void* weight;          /* [rows (2 * rows for SWIGLU_ROWS), cols] GGUF blocks         */
    const float* x;              /* [cols] ([2 * cols] for SI_HIP_X_SWIGLU)                    */
    float* y;                    /* [rows]                                                     */
    const float* residual;       /* SI_HIP_OUT_PLAIN only: y = W.x + residual; may equal y     */
    const float* norm_weight;    /* RMSNORM, LAYERNORM*: [cols]                                */
    const float* norm_bias;      /* LAYERNORM*: [cols]                                         */
    const float* mix;            /* LAYERNORM_MIX: [cols]                                      */
    const float* prev;           /* LAYERNORM_MIX: [cols]                                      */
    float* norm_out;             /* LAYERNORM*, optional: receives the normalised x (pre-mix)  */
    int64_t rows;
    int64_t cols;
    float eps;
    int32_t reserved2;           /* 0                                                          */
} si_hip_gemv_op;

/* Runs `count` (1..64) products that have no data dependence on each other:
 * no op may read or write what another op of the batch writes (y,
 * norm_out).  Consecutive ops with the same format (and, for the tiled
 * kernel, the same cols) share one launch, up to 8 per launch.  Replaces a
 * run of core.mat-vec dispatches between two barriers of a D3D12 entry
 * (D3D12VmSchedule.cs:74-99, whose pending-write rule this batch enforces),
 * e.g. the RWKV-7 r/k/v and LoRA projections of one layer
 * (PortableRwkv7GraphProvider.cs:219-233).  paths (optional) receives
 * each op's kernel as si_hip_gemv reports it (1 tiled, 2 any-shape,
 * 3 short rows). */
int si_hip_gemv_batch(si_hip_context* ctx, const si_hip_gemv_op* ops, int count, int* paths);

/* out[cols] = FP32 values of row *index of a block-quantized [rows, cols]
 * table; an index outside 0..rows-1 yields NaN values (no out-of-bounds
 * read).  `index` is a device int32.  Replaces: core.gather-row
 * (GpuTierZeroInstruction.cs:397-405, CpuInstructionNumerics.cs:25-30) for a
 * quantized embedding table. */
int si_hip_gather_row(si_hip_context* ctx, int format, const void* table, int64_t rows, int64_t cols,
                      const int32_t* index, float* out);

/* Grouped-query attention of one new token over an fp16 KV cache. */
typedef struct si_hip_attention {
    const float* qkv;          /* [heads*128 q | kv_heads*128 k | kv_heads*128 v], before the rotary embedding */
    const int32_t* position;   /* device scalar: the new token's index = its cache slot */
    void* k_cache;             /* fp16 [kv_heads][capacity][128], 16-byte aligned */
    void* v_cache;             /* fp16 [kv_heads][capacity][128], 16-byte aligned */
    float* out;                /* [heads * 128] */
    float* workspace;          /* si_hip_attention_workspace_bytes: chunk partials and the rotary table; any
                                  contents on entry (each call prepares it); calls that share one workspace
                                  must not overlap on the GPU */
    int heads;
    int kv_heads;              /* heads / kv_heads in 1..4 */
    int head_dim;              /* 128 */
    int rotary_dim;            /* rotate-half over the first rotary_dim values of each head */
    int capacity;              /* 1..16384 */
    float rope_base;
    float rope_scale;
} si_hip_attention;

int si_hip_attention_workspace_bytes(int heads, int capacity, uint64_t* bytes);

/* Applies the rotary embedding to q and k at *position, rounds k and v to
 * fp16 and appends them at slot *position, then attends over slots
 * 0..*position: out_h = softmax(q_h . K^T / sqrt(128)) . V for every query
 * head h with KV head h / (heads / kv_heads).  A position outside
 * 0..capacity-1 writes nothing and yields NaN.  Replaces: ApplyRotary +
 * Phi4KeyValueCache.Append + ComputeAttention (Phi4TextModel.cs:64-72,
 * 212-273) and the rope-kv-write / grouped-query-attention dispatches
 * (Phi4D3D12TextSession.cs:873-890). */
int si_hip_attention_decode(si_hip_context* ctx, const si_hip_attention* args);

/* si_hip_attention_decode without a workspace: args->workspace must be
 * NULL, and the chunk partials and rotary table go to a device array of the
 * library (2 MiB per GPU, held until the process ends), so the call
 * allocates nothing (no hipMalloc, no allocating library routine).  Requests
 * whose workspace (si_hip_attention_workspace_bytes) exceeds 2 MiB, i.e.
 * heads * ceil(capacity / 64) > 4032, fail with SI_HIP_ERR_UNSUPPORTED.
 * Every context on one GPU shares the array: calls that overlap on one GPU
 * (other contexts' streams, or this one's with another thread's work) race.
 * No counterpart in the reference; it is for callers that cannot allocate
 * device memory (code under graph capture, tight serving loops, hosts that
 * forbid allocation after start-up). */
int si_hip_attention_decode_noalloc(si_hip_context* ctx, const si_hip_attention* args);

int si_hip_argmax_workspace_bytes(uint64_t* bytes);

/* *index = first index of the maximum of values[0..n).  Replaces:
 * transformer.argmax (GpuTransformerInstructionCollection.cs:697-748). */
int si_hip_argmax(si_hip_context* ctx, const float* values, int64_t n, void* workspace, int32_t* index);

/* ---- transformer operators, one launch each ------------------------------------ */

/* The operators of the reference's D3D12 decode program as separate
 * launches, for VM programs that dispatch them one by one (the fused
 * si_hip_phi4_decode step keeps its own layout).  KV caches here are
 * [context][kv_heads][head_size] rows, FP32 as in the reference or fp16. */

/* output[j] = input[j] * (1 / sqrt(sum(input^2) / n + eps)) * weight[j], n in
 * 1..1048576, eps finite and >= 0.  Replaces: transformer.rms-norm
 * (GpuTransformerInstructionCollection.cs:323-368). */
int si_hip_rms_norm(si_hip_context* ctx, const float* input, const float* weight, float* output, int64_t n,
                    float eps);

/* updated = hidden + residual, output = updated * (1 / sqrt(sum(updated^2) / n
 * + eps)) * weight; outputs may not overlap any input.  Replaces:
 * transformer.residual-rms-norm (GpuTransformerInstructionCollection.cs:370-417). */
int si_hip_residual_rms_norm(si_hip_context* ctx, const float* hidden, const float* residual, const float* weight,
                             float* updated, float* output, int64_t n, float eps);

/* output[i] = g_i / (1 + exp(-g_i)) * u_i for gate_up = [g (n values) | u (n
 * values)].  Replaces: transformer.swiglu (GpuTransformerInstructionCollection.cs:419-443). */
int si_hip_swiglu(si_hip_context* ctx, const float* gate_up, float* output, int64_t n);

typedef struct si_hip_rope_kv_write_args {
    const float* qkv;          /* [query_size | kv_size | kv_size] of one token */
    const int32_t* position;   /* device scalar: the cache row written */
    const float* frequencies;  /* [rotary_size / 2]: angle of pair i = position * frequencies[i] */
    float* query;              /* [query_size] rotated queries */
    void* key_cache;           /* [context][kv_size], cache_format */
    void* value_cache;
    int32_t cache_format;      /* SI_HIP_F32 or SI_HIP_F16 (rounded to nearest even) */
    int32_t query_size;        /* a multiple of head_size */
    int32_t kv_size;           /* kv_heads * head_size */
    int32_t head_size;
    int32_t rotary_size;       /* even, <= head_size */
    int32_t context;
    float rope_scale;          /* multiplies cos and sin */
} si_hip_rope_kv_write_args;

/* Rotate-half rotary embedding of the first rotary_size values of every q
 * and k head, q to `query`, k and v to row *position of the caches; a
 * position outside 0..context-1 writes nothing.  Replaces:
 * transformer.rope-kv-write (GpuTransformerInstructionCollection.cs:445-543). */
int si_hip_rope_kv_write(si_hip_context* ctx, const si_hip_rope_kv_write_args* args);

typedef struct si_hip_gqa_args {
    const float* query;        /* [query_heads * head_size], 16-byte aligned */
    const void* key_cache;     /* [context][kv_heads][head_size], 16-byte aligned */
    const void* value_cache;
    const int32_t* position;   /* device scalar */
    float* output;             /* [query_heads * head_size] */
    int32_t cache_format;      /* SI_HIP_F32 or SI_HIP_F16 */
    int32_t query_heads;       /* a multiple of kv_heads */
    int32_t kv_heads;
    int32_t head_size;         /* 64, 128 or 256 */
    int32_t context;           /* 1..16384 */
    float* workspace;          /* si_hip_gqa_workspace_bytes: per-chunk partials; any contents on entry;
                                  calls sharing one workspace must not overlap on the GPU */
} si_hip_gqa_args;

int si_hip_gqa_workspace_bytes(int query_heads, int head_size, int context, uint64_t* bytes);

/* output_h = softmax(q_h . K^T / sqrt(head_size)) . V over cache rows
 * 0..min(max(*position, 0), context - 1) of KV head h / (query_heads /
 * kv_heads), in 64-row chunks merged by a second launch.  Replaces: transformer.grouped-query-attention
 * (GpuTransformerInstructionCollection.cs:46-143). */
int si_hip_grouped_query_attention(si_hip_context* ctx, const si_hip_gqa_args* args);

/* ---- batched (prefill) transformer operators -------------------------------------- */

/* The operators of the reference's D3D12 prefill program
 * (GpuBatchTransformerInstructions.cs), one launch each (batch-gqa-values:
 * two).  Every one takes control = device int32[2] {start, valid}: the
 * batch's buffers hold `batch` rows (1..16), row r < valid is the token at
 * position start + r, rows r >= valid are neither read nor written.
 * Matrices are row-major [batch][width]; KV caches [context][kv_heads][128]
 * (FP32 as in the reference, or fp16). */

/* output[r] = table[start + r] for r < valid and 0 <= start + r < table_rows.
 * Replaces: transformer.batch-gather-rows (GpuBatchTransformerInstructions.cs:646-679). */
int si_hip_batch_gather_rows(si_hip_context* ctx, const float* table, int64_t table_rows, int64_t width,
                             const int32_t* control, float* output, int batch);

/* Per live row: output = input * (1 / sqrt(sum(input^2) / width + eps)) * weight.
 * Replaces: transformer.batch-rms-norm (GpuBatchTransformerInstructions.cs:101-156). */
int si_hip_batch_rms_norm(si_hip_context* ctx, const float* input, const float* weight, const int32_t* control,
                          float* output, int batch, int64_t width, float eps);

/* Per live row: updated = hidden + residual, output = rms-norm(updated).
 * Replaces: transformer.batch-residual-rms-norm (GpuBatchTransformerInstructions.cs:158-222). */
int si_hip_batch_residual_rms_norm(si_hip_context* ctx, const float* hidden, const float* residual,
                                   const float* weight, const int32_t* control, float* updated, float* output,
                                   int batch, int64_t width, float eps);

/* output[r] = W . input[r] for live rows, W [rows, columns] in any matrix
 * format (Q8_0, Q4_0, Q4_K, F16, F32; columns % 32 == 0, Q4_K % 256), FP32
 * products and sums on the matrix cores (v_mfma_f32_16x16x4_f32).  Replaces:
 * transformer.batch-shared-matvec (GpuBatchTransformerInstructions.cs:224-279),
 * whose weight is F16. */
int si_hip_batch_matvec(si_hip_context* ctx, int format, const void* weight, const float* input,
                        const int32_t* control, float* output, int batch, int64_t rows, int64_t columns);

/* Per live row: output[i] = g_i / (1 + exp(-g_i)) * u_i over gate_up[r] = [g | u].
 * Replaces: transformer.batch-swiglu (GpuBatchTransformerInstructions.cs:281-316). */
int si_hip_batch_swiglu(si_hip_context* ctx, const float* gate_up, const int32_t* control, float* output,
                        int batch, int64_t width);

typedef struct si_hip_batch_rope_args {
    const float* qkv;          /* [batch][query_size | kv_size | kv_size] */
    const int32_t* control;
    const float* frequencies;  /* [rotary_size / 2] */
    float* query;              /* [batch][query_size] rotated queries */
    void* key_cache;           /* [context][kv_size], cache_format */
    void* value_cache;
    int32_t cache_format;      /* SI_HIP_F32 or SI_HIP_F16 (rounded to nearest even) */
    int32_t batch;
    int32_t query_size;        /* a multiple of head_size */
    int32_t kv_size;           /* kv_heads * head_size */
    int32_t head_size;
    int32_t rotary_size;       /* even, <= head_size */
    int32_t context;
    float rope_scale;
} si_hip_batch_rope_args;

/* Per live row r at position p = start + r inside the cache: rotate-half
 * rotary embedding of q and k (angle p * frequencies[i], cos and sin times
 * rope_scale), q to query[r], k and v to cache row p.  Replaces:
 * transformer.batch-rope-kv-write (GpuBatchTransformerInstructions.cs:318-413). */
int si_hip_batch_rope_kv_write(si_hip_context* ctx, const si_hip_batch_rope_args* args);

typedef struct si_hip_batch_attention_args {
    const float* query;          /* scores: [batch][query_heads * 128], 16-byte aligned */
    const float* probabilities;  /* values: [batch][query_heads][context] */
    const void* cache;           /* scores: key cache; values: value cache ([context][kv_heads][128]) */
    const int32_t* control;
    float* output;               /* scores: [batch][query_heads][context]; values: [batch][query_heads * 128] */
    float* workspace;            /* values: si_hip_batch_values_workspace_bytes; any contents on entry;
                                    calls sharing one workspace must not overlap on the GPU */
    int32_t cache_format;        /* SI_HIP_F32 or SI_HIP_F16 */
    int32_t batch;
    int32_t query_heads;         /* a multiple of kv_heads, at most 8 per KV head */
    int32_t kv_heads;
    int32_t head_size;           /* 128 */
    int32_t context;             /* 1..16384 */
} si_hip_batch_attention_args;

/* scores[r][h][j] = q[r][h] . k[j][h / group] / sqrt(128) for j <= start + r,
 * -FLT_MAX for every other column.  Replaces: transformer.batch-gqa-scores
 * (GpuBatchTransformerInstructions.cs:415-470). */
int si_hip_batch_gqa_scores(si_hip_context* ctx, const si_hip_batch_attention_args* args);

/* probabilities[r][h][j] = exp(s_j - max) / sum over j <= start + r, 0 for
 * the other columns.  Replaces: transformer.batch-causal-softmax
 * (GpuBatchTransformerInstructions.cs:472-542). */
int si_hip_batch_causal_softmax(si_hip_context* ctx, const float* scores, const int32_t* control,
                                float* probabilities, int batch, int heads, int64_t context);

/* output[r][h][d] = sum over j <= start + r of p[r][h][j] v[j][h / group][d],
 * in 64-column chunks added by a second launch.  Replaces:
 * transformer.batch-gqa-values (GpuBatchTransformerInstructions.cs:544-598). */
int si_hip_batch_gqa_values(si_hip_context* ctx, const si_hip_batch_attention_args* args);

/* si_hip_batch_gqa_scores, si_hip_batch_causal_softmax and
 * si_hip_batch_gqa_values in two launches, for callers that never read the
 * scores or probabilities: args->query, args->cache (the key cache),
 * args->output (the values' output) and args->workspace (at least
 * si_hip_batch_values_workspace_bytes) as for those calls,
 * args->probabilities unused, and the value cache.  The output equals the
 * three calls' up to FP32 rounding (each 64-position chunk's exponentials
 * are taken against the chunk's own largest score and the chunks rescaled
 * when they are added).  No counterpart in the reference: the C++ host's
 * executor uses it when it fuses those three dispatches of a program. */
int si_hip_batch_gqa_attention(si_hip_context* ctx, const si_hip_batch_attention_args* args,
                               const void* value_cache);

int si_hip_batch_values_workspace_bytes(int batch, int query_heads, int context, uint64_t* bytes);

/* output = input[valid - 1] when 0 < valid <= batch.  Replaces:
 * transformer.batch-select-last (GpuBatchTransformerInstructions.cs:600-625). */
int si_hip_batch_select_last(si_hip_context* ctx, const float* input, const int32_t* control, float* output,
                             int batch, int64_t width);

/* ---- Phi-4 decode step ------------------------------------------------------------ */

typedef struct si_hip_phi4_layer {
    const float* attn_norm;    /* FP32 [hidden] */
    const void* qkv;           /* [hidden + 2*kv_heads*128, hidden] */
    const void* o;             /* [hidden, hidden] */
    const float* ffn_norm;     /* FP32 [hidden] */
    const void* up;            /* [2*ffn, hidden]: gate rows then up rows */
    const void* down;          /* [hidden, ffn] */
    void* k_cache;             /* fp16 [kv_heads][capacity][128] */
    void* v_cache;
} si_hip_phi4_layer;

typedef struct si_hip_phi4_model {
    int layers, hidden, heads, kv_heads, head_dim, rotary_dim, ffn, vocab, capacity;
    int weight_format;         /* layer projections (e.g. Q4_K) */
    int embed_format;          /* embedding table (e.g. Q8_0) */
    int head_format;           /* vocabulary projection (e.g. Q8_0) */
    float rms_eps, rope_base, rope_scale;
    const void* embed;         /* [vocab, hidden] */
    const void* lm_head;       /* [vocab, hidden] */
    const float* output_norm;  /* FP32 [hidden] */
    const si_hip_phi4_layer* layer;   /* host array of `layers` entries */
    int32_t* control;          /* device [token, position] */
    float* hidden_state;       /* [hidden] */
    float* qkv;                /* [hidden + 2*kv_heads*128] */
    float* attn;               /* [hidden] */
    float* gate_up;            /* [2*ffn] scratch (the step uses the first ffn values) */
    float* logits;             /* [vocab] */
    void* workspace;           /* si_hip_phi4_workspace_bytes */
    int32_t* next_token;       /* device int32: argmax of the logits */
} si_hip_phi4_model;

int si_hip_phi4_workspace_bytes(const si_hip_phi4_model* model, uint64_t* bytes);

/* Launches one decode step for token control[0] at position control[1]:
 * embedding, every layer (updating the KV caches at control[1]), logits and
 * next_token.  Inside si_hip_plan_begin/end it records the whole step as
 * one plan (replayed per token with si_hip_plan_launch).  Replaces: the
 * Phi-4 decode program (Phi4D3D12TextSession.Build, Phi4D3D12TextSession.cs:
 * 866-919) and Phi4TextSession.ForwardToken (Phi4TextModel.cs:329-344). */
int si_hip_phi4_decode(si_hip_context* ctx, const si_hip_phi4_model* model);

/* The same step for positions up to a bound: every layer's attention covers
 * only the first position_bound / 128 + 1 chunks of 128 cache positions
 * and requests their K / V rows together with the position (the full-cache
 * step waits for the position first).  Serves every position below
 * limit = min(capacity, 128 * (position_bound / 128 + 1)); replayed with
 * control[1] >= limit, the step writes NaN attention outputs (so NaN
 * logits) and appends nothing to the caches.  0 <= position_bound <
 * capacity and rotary_dim a multiple of 16, else an error.  No counterpart
 * in the reference (its program attends over the cache it is given each
 * token): for callers that record one plan per range of positions, as the
 * Phi-4 session here does (one per 128 positions, recorded on first use). */
int si_hip_phi4_decode_bounded(si_hip_context* ctx, const si_hip_phi4_model* model, int position_bound);

/* ---- RWKV-7 decode step ------------------------------------------------------------ */

/* out[b][r] = sum_c matrix[b][r][c] * vector[b][c], FP32.  Replaces:
 * core.tensor.batched-mat-vec (CpuPrimitiveGraphExecutor.cs:780-791,
 * GpuTierZeroInstruction.cs:447-451). */
int si_hip_batched_matvec(si_hip_context* ctx, const float* matrix, const float* vector, float* out,
                          int batch, int rows, int cols);

/* out = ((x - mean) * (1 / sqrt(var + eps))) * weight + bias over n <= 8192
 * values (mean and var over the n values).  Replaces: the Normalize +
 * Affine node chain of the RWKV-7 graph (PortableRwkv7GraphProvider.cs:
 * 163-170, 180-182). */
int si_hip_layernorm(si_hip_context* ctx, const float* x, const float* weight, const float* bias, int n,
                     float eps, float* out);

/* Time-mix core of one RWKV-7 layer after its projections, vectors
 * [heads * 64]:
 *   decay = exp(-0.606531 * sigmoid(w_lora + w0)), a = sigmoid(a_lora + a0)
 *   kn = per-head unit vector of k * k_k;  key = (k + a * (k * k_a)) - k * k_a
 *   value = v (first layer, also stored to v_first) or
 *           v + (v_first - v) * sigmoid(v_lora + v0)
 *   S'[h,i,j] = (S[h,i,j] * decay[j] + value[i] * key[j]) - (S[h,i,:].kn) * kn[j] * a[j]
 *   y = S' . r;  out = (GroupNorm64e-5(y) * lnx_weight + lnx_bias + value * sum(key * r * r_k)) * gate
 * with the state updated in place.  Replaces the WKV node chain
 * (PortableRwkv7GraphProvider.cs:224-276: batched mat-vecs, head outer
 * products, broadcasts and the pointwise ops around them). */
typedef struct si_hip_rwkv7_wkv_args {
    int32_t heads;             /* head size is 64 */
    int32_t first_layer;
    const float* r, *k, *v;
    const float* w_lora, *a_lora, *gate, *v_lora;   /* v_lora unused when first_layer */
    const float* w0, *a0, *v0, *k_k, *k_a, *r_k, *lnx_weight, *lnx_bias;
    float* v_first;            /* [heads * 64] */
    float* state;              /* FP32 [heads][64][64], 16-byte aligned */
    float* out;                /* [heads * 64] */
} si_hip_rwkv7_wkv_args;

int si_hip_rwkv7_wkv(si_hip_context* ctx, const si_hip_rwkv7_wkv_args* args);

typedef struct si_hip_rwkv7_layer {
    const float* ln1_weight, *ln1_bias, *ln2_weight, *ln2_bias;   /* FP32 [hidden] */
    const float* mix;          /* att.x_rwkvag FP32 [6][hidden]: r, w, k, v, a, g */
    const void* receptance, *key, *value, *output;   /* [hidden, hidden] */
    const void* w1, *w2;       /* [rank_w, hidden], [hidden, rank_w] */
    const void* a1, *a2;       /* [rank_a, hidden], [hidden, rank_a] */
    const void* g1, *g2;       /* [rank_g, hidden], [hidden, rank_g] */
    const void* v1, *v2;       /* [rank_v, hidden], [hidden, rank_v]; unused in layer 0 */
    const float* w0, *a0, *v0, *k_k, *k_a, *r_k, *lnx_weight, *lnx_bias;   /* FP32 [hidden] */
    const float* ffn_mix;      /* ffn.x_k FP32 [hidden] */
    const void* ffn_key;       /* [ffn, hidden] */
    const void* ffn_value;     /* [hidden, ffn] */
    float* att_prev;           /* state FP32 [hidden] */
    float* ffn_prev;           /* state FP32 [hidden] */
    float* wkv;                /* state FP32 [heads][64][64] */
} si_hip_rwkv7_layer;

typedef struct si_hip_rwkv7_model {
    int32_t layers, hidden, heads, ffn, vocab;   /* hidden = heads * 64 */
    int32_t rank_w, rank_a, rank_v, rank_g;
    int32_t weight_format;     /* every projection, LoRA included (e.g. Q8_0) */
    int32_t embed_format, head_format;
    const void* embed;         /* [vocab, hidden] */
    const float* ln0_weight, *ln0_bias;
    const si_hip_rwkv7_layer* layer;   /* host array of `layers` entries */
    const float* ln_out_weight, *ln_out_bias;
    const void* head;          /* [vocab, hidden] */
    const int32_t* control;    /* device [token] */
    float* hidden_state;       /* [hidden] */
    float* logits;             /* [vocab] */
    void* workspace;           /* si_hip_rwkv7_workspace_bytes */
    int32_t* next_token;       /* device int32: argmax of the logits */
} si_hip_rwkv7_model;

int si_hip_rwkv7_workspace_bytes(const si_hip_rwkv7_model* model, uint64_t* bytes);

/* Launches one RWKV-7 token step for token control[0]: ln0(embedding),
 * every layer (updating its att_prev / ffn_prev / wkv state), ln_out +
 * head, argmax.  Six launches per layer: the seven time-mix projections
 * with LayerNorm + token mix fused (one launch), the four LoRA outputs (one
 * launch), the time-mix core, the output projection, the channel-mix key
 * projection with LayerNorm + mix + relu^2 fused, and the value projection.
 * Inside si_hip_plan_begin/end it records the step as one plan.  Replaces:
 * the portable RWKV-7 forward-token graph (PortableRwkv7GraphProvider.cs:
 * 190-292) run by a VM executor. */
int si_hip_rwkv7_decode(si_hip_context* ctx, const si_hip_rwkv7_model* model);

/* ---- T0 primitive and portable tensor operators ---------------------------------- */

/* The operators an unfused logical graph dispatches between its mat-vecs
 * (the portable RWKV-7 forward-token graph, PortableRwkv7GraphProvider.cs:
 * 13-295), one launch each, on dense FP32 tensors.  An output that overlaps
 * an input is rejected (ARGUMENT), as the reference rejects in-place
 * operator writes (GpuTierZeroInstruction.cs:461-463). */
typedef enum si_hip_t0_op {
    SI_HIP_T0_COPY = 0,        /* core.copy          input                                       */
    SI_HIP_T0_ADD = 1,         /* core.add           left + right                                */
    SI_HIP_T0_SUBTRACT = 2,    /* core.subtract      left - right                                */
    SI_HIP_T0_MULTIPLY = 3,    /* core.multiply      left * right                                */
    SI_HIP_T0_DIVIDE = 4,      /* core.divide        left / right                                */
    SI_HIP_T0_MAXIMUM = 5,     /* core.maximum       NaN if either is NaN; +0 above -0            */
    SI_HIP_T0_EXP = 6,         /* core.exp                                                       */
    SI_HIP_T0_TANH = 7,        /* core.tanh          tanh(0) = 0 exactly                         */
    SI_HIP_T0_SIGMOID = 8,     /* core.sigmoid       1 / (1 + exp(-x))                           */
    SI_HIP_T0_RSQRT = 9,       /* core.rsqrt         1 / sqrt(x)                                 */
    SI_HIP_T0_SQUARE = 10,     /* core.square        x * x                                       */
    SI_HIP_T0_RELU = 11,       /* core.relu          maximum(x, 0)                               */
} si_hip_t0_op;

/* output[i] = op(left[i]) or op(left[i], right[i]) for i < count (right is
 * ignored by the unary operators).  Replaces: the elementwise T0 operators
 * (GpuTierZeroInstruction.cs:376-386, CpuPrimitiveOperatorBackend.cs:25-90). */
int si_hip_t0_elementwise(si_hip_context* ctx, int op, const float* left, const float* right, float* output,
                          int64_t count);
/* output[i] = FP32 value of the fp16 input[i].  Replaces: core.tensor.cast-f16-f32
 * (PortableTensorOperationContracts.cs:54, GpuTierZeroInstruction.cs:425-428). */
int si_hip_t0_cast_f16_f32(si_hip_context* ctx, const void* input, float* output, int64_t count);
/* output[i] = value (finite).  Replaces: core.tensor.fill (PortableTensorOperationContracts.cs:12-20,53). */
int si_hip_t0_fill(si_hip_context* ctx, float value, float* output, int64_t count);
/* output[r] = sum over c of input[r][c], divided by cols when mean != 0.
 * Replaces: core.tensor.reduce-last-sum / -mean (rows = the leading
 * dimensions' product) and core.reduce-sum / -mean (rows = 1)
 * (PortableTensorOperationContracts.cs:59-60,166-172; GpuTierZeroInstruction.cs:387-393,446-451). */
int si_hip_t0_reduce_last(si_hip_context* ctx, int mean, const float* input, float* output, int64_t rows,
                          int64_t cols);
/* Broadcast of a rank 1..4 tensor to a rank 1..4 shape: trailing
 * dimensions aligned, each input axis 1 (repeated) or equal to the
 * output's.  Replaces: core.tensor.broadcast (PortableTensorOperationContracts.cs:58,158-164). */
int si_hip_t0_broadcast(si_hip_context* ctx, const float* input, int input_rank, const int64_t* input_dims,
                        float* output, int output_rank, const int64_t* output_dims);
/* output = input[..., start:start+length, ...] along `axis` (rank kept,
 * row-major).  Replaces: core.tensor.slice (PortableTensorOperationContracts.cs:
 * 24-40,56,138-149). */
int si_hip_t0_slice(si_hip_context* ctx, const float* input, int rank, const int64_t* input_dims, int axis,
                    int64_t start, int64_t length, float* output);
/* output[h][i][j] = left[h][i] * right[h][j].  Replaces: core.tensor.head-outer
 * (PortableTensorOperationContracts.cs:61,174-182). */
int si_hip_t0_head_outer(si_hip_context* ctx, const float* left, const float* right, float* output, int64_t heads,
                         int64_t rows, int64_t cols);
/* si_hip_gemv pinned to the any-shape kernel (one wave per output row,
 * path 2) whatever the shape: the mat-vec a program selects as serial.
 * Replaces: the serial core.mat-vec form (GpuTierZeroInstruction.cs:386-396),
 * chosen by GpuMatVecMode.Serial (GpuMatVecOptimization.cs:36-37). */
int si_hip_gemv_any_shape(si_hip_context* ctx, int format, const void* w, const float* x, float* y, int64_t rows,
                          int64_t cols);

/* ---- GGUF model files ------------------------------------------------------------ */

/* A GGUF v3 file mapped read-only: metadata, tensor directory and the
 * tensors' bytes.  Replaces: GgufModelFile (SharpInference.Gguf/
 * GgufModelFile.cs:49-199) with the same validation (magic, version 3,
 * counts, unique non-blank keys and names, rank 1..8, non-empty dimensions,
 * power-of-two general.alignment, every tensor inside the file), plus byte
 * lengths for the K-quant types (256-element super-blocks: Q2_K 84, Q3_K
 * 110, Q4_K 144, Q5_K 176, Q6_K 210, Q8_K 292 bytes) and tensors above
 * 2 GiB.  Errors: SI_HIP_ERR_IO (open/map), SI_HIP_ERR_FORMAT (malformed),
 * SI_HIP_ERR_UNSUPPORTED (tensor type without a byte length); the message is
 * si_hip_last_error(NULL). */
typedef struct si_gguf si_gguf;

typedef enum si_gguf_value_type {
    SI_GGUF_U8 = 0, SI_GGUF_I8 = 1, SI_GGUF_U16 = 2, SI_GGUF_I16 = 3, SI_GGUF_U32 = 4, SI_GGUF_I32 = 5,
    SI_GGUF_F32 = 6, SI_GGUF_BOOL = 7, SI_GGUF_STRING = 8, SI_GGUF_ARRAY = 9, SI_GGUF_U64 = 10,
    SI_GGUF_I64 = 11, SI_GGUF_F64 = 12,
} si_gguf_value_type;

typedef struct si_gguf_file_info {
    uint32_t version;
    uint32_t reserved;
    uint64_t alignment;        /* general.alignment or 32 */
    uint64_t data_start;       /* file offset of the tensor data section */
    uint64_t file_bytes;
    int64_t tensor_count;
    int64_t metadata_count;
} si_gguf_file_info;

typedef struct si_gguf_tensor {
    const char* name;          /* valid until si_gguf_close */
    int32_t type;              /* GGUF tensor type id (si_hip_format values and the other GGML ids) */
    int32_t rank;
    uint64_t dims[8];          /* dims[0] is the contiguous axis (columns); unused entries are 1 */
    uint64_t offset;           /* absolute file offset of the first byte */
    uint64_t bytes;
    const void* data;          /* host address inside the read-only mapping */
} si_gguf_tensor;

typedef struct si_gguf_value {
    const char* key;
    int32_t type;              /* si_gguf_value_type */
    int32_t array_type;        /* element type when type == SI_GGUF_ARRAY, else -1 */
    uint64_t count;            /* elements (1 for a scalar) */
    const void* data;          /* numbers and bools: count values in native layout (bool = uint8);
                                  strings: count const char* (NUL-terminated UTF-8) */
    const uint64_t* lengths;   /* strings: byte length of each; NULL otherwise */
} si_gguf_value;

int si_gguf_open(const char* path, si_gguf** out);
int si_gguf_close(si_gguf* file);
int si_gguf_info(const si_gguf* file, si_gguf_file_info* info);
int si_gguf_tensor_at(const si_gguf* file, int64_t index, si_gguf_tensor* out);
/* *index = the tensor's index, or -1 when the file has no such tensor. */
int si_gguf_find_tensor(const si_gguf* file, const char* name, int64_t* index);
int si_gguf_metadata_at(const si_gguf* file, int64_t index, si_gguf_value* out);
/* *index = the key's index, or -1 when absent. */
int si_gguf_find_metadata(const si_gguf* file, const char* key, int64_t* index);

/* Copies tensor `index`'s bytes, unchanged, from the mapping into device
 * memory at device_dst (dst_bytes >= the tensor's bytes) and waits.
 * Replaces: executor.Upload(slot, tensor.Bytes) of the model tensors
 * (Phi4D3D12TextSession.cs:55-58, D3D12VmExecutor.cs:595-625). */
int si_gguf_upload(si_hip_context* ctx, const si_gguf* file, int64_t index, void* device_dst, uint64_t dst_bytes);

/* ---- recorded entries and timing -------------------------------------------- */

/* Starts recording: until si_hip_plan_end, launches on `ctx` are recorded
 * instead of executed (uploads, readbacks, allocations and syncs are
 * rejected with SI_HIP_ERR_STATE).  A plan is the HIP form of a recorded VM
 * entry (D3D12VmSchedule.Create, D3D12VmSchedule.cs:48-111): one graph,
 * replayed with one submission. */
int si_hip_plan_begin(si_hip_context* ctx);
int si_hip_plan_end(si_hip_context* ctx, si_hip_plan** out);
int si_hip_plan_destroy(si_hip_plan* plan);

/* Replays the plan on the context stream (asynchronous).
 * Replaces: D3D12VmExecutor.Execute(entry) (D3D12VmExecutor.cs:283-292). */
int si_hip_plan_launch(si_hip_plan* plan);

/* Launches plans[i % nplans] for i in [0, steps) back to back (asynchronous). */
int si_hip_plan_launch_sequence(si_hip_plan* const* plans, int nplans, int64_t steps);

/* GPU microseconds per replay over `repetitions` back-to-back replays,
 * measured with events on the context stream; repetitions outside 1..1024
 * is ARGUMENT, and a call while the context's timer_begin is open is STATE
 * (both use the same event pair).  Replaces:
 * D3D12VmExecutor.MeasureGpuMicroseconds (D3D12VmExecutor.cs:452-478). */
int si_hip_plan_measure_us(si_hip_plan* plan, int repetitions, double* microseconds);

/* Event pair on the context stream: begin records the start event, end
 * records the stop event, waits for it and returns the elapsed ms. */
int si_hip_timer_begin(si_hip_context* ctx);
int si_hip_timer_end(si_hip_context* ctx, double* milliseconds);

#ifdef __cplusplus
}
#endif
#endif
