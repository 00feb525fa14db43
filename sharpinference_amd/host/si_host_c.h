/*
 * C entry points of libsharpinference_hip_host.so for callers that cannot
 * bind C++ (the Python package): a Phi-4 decode program built dispatch by
 * dispatch (BuildPhi4DecodeProgram) and run by its HipVmExecutor.  Status
 * codes are si_hip_status values; the message of the calling thread's last
 * failure is sih_last_error().
 */
#ifndef SI_HOST_C_H
#define SI_HOST_C_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sih_program sih_program;

typedef struct sih_phi4_shape {
    int32_t layers, hidden, heads, kv_heads, head_dim, rotary_dim, ffn, vocab, context;
    int32_t weight_format, embed_format, head_format;   /* GGUF type ids */
    int32_t tied;                                       /* vocabulary projection onto token_embedding */
    int32_t cache_fp16;                                 /* 1: Float16 KV cache, 0: Float32 */
    float rms_eps, rope_base, rope_scale;
    int32_t prompt_rows;                                /* > 0: fused_embeddings [prompt_rows, hidden] and
                                                           the prefill_fused_16 entry */
} sih_phi4_shape;

/* Builds the program, creates its executor on `device` (every slot zeroed)
 * and uploads rope_frequencies. */
int sih_phi4_program_create(const sih_phi4_shape* shape, int device, sih_program** out);
int sih_program_destroy(sih_program* program);
int sih_program_slot_bytes(const sih_program* program, const char* slot, uint64_t* bytes);
int sih_program_upload(sih_program* program, const char* slot, const void* bytes, uint64_t length);
int sih_program_readback(sih_program* program, const char* slot, void* bytes, uint64_t length);
/* Executes an entry (recorded once as a plan, replayed, waited for). */
int sih_program_execute(sih_program* program, const char* entry);
int sih_program_measure_us(sih_program* program, const char* entry, int repetitions, double* microseconds);
int sih_program_dispatch_count(const sih_program* program, const char* entry, int* count);
/* Dispatch fusion of the executor (on by default; HipVmExecutor's comment
 * lists the fused pairs): on = 0 switches it off (plans are re-recorded). */
int sih_program_set_fusion(sih_program* program, int on);
/* Launches one execution of `entry` makes with the current fusion setting. */
int sih_program_launch_count(sih_program* program, const char* entry, int* count);
/* VmProgram XML of the program (the reference's schema, target "Hip"):
 * with buffer NULL only *length (bytes, without a terminator) is set. */
int sih_program_serialize(const sih_program* program, char* buffer, uint64_t capacity, uint64_t* length);
/* A program from VmProgram XML, every operator re-adapted on the HIP
 * target, with its executor on `device` (every slot zeroed). */
int sih_program_create_from_xml(const char* xml, int device, sih_program** out);
/* The program as a HIP VM artifact (ZIP: program.xml + hashed manifest). */
int sih_program_export_artifact(const sih_program* program, void* buffer, uint64_t capacity, uint64_t* length);
int sih_program_import_artifact(const void* bytes, uint64_t length, int device, sih_program** out);
const char* sih_last_error(void);

/* VmProgram XML read (every operator re-adapted on the HIP target, no
 * device) and written again. */
int sih_program_xml_roundtrip(const char* xml, char* buffer, uint64_t capacity, uint64_t* length);

/* ---- logical graphs (si_graph.hpp) ------------------------------------------------- */

/* One tensor of a model catalog. */
typedef struct sih_model_tensor {
    const char* name;
    int32_t type;        /* GGUF type id: F32, F16, Q8_0, Q4_0, Q4_K */
    int32_t rank;        /* 1..4 */
    int64_t dims[4];     /* the catalog's dimensions (GGML order: a matrix is [input, output]) */
} sih_model_tensor;

/* VmOptimizationOptions of the lowering. */
typedef struct sih_graph_options {
    int32_t reuse_local_storage;   /* 1: local intermediates share slots (GraphResourceAllocator.PlanLocal) */
    int32_t weight_views;          /* 1: reshapes / casts of weights become views */
    int32_t native_half_weights;   /* 1: FP16 weights feed the matrix operators directly */
    int32_t matvec_mode;           /* -1: no settings (cooperative by default); 0 Serial, 1 Cooperative,
                                      3 Default (GpuMatVecMode; Profile needs the C++ interface) */
    uint32_t threads_per_group;    /* 1..1024 */
} sih_graph_options;

/* The portable RWKV-7 forward-token graph of a catalog
 * (PortableRwkv7GraphProvider.Build), lowered to a HIP VM program
 * (VmGraphOptimizer.OptimizeWithReport) with its executor on `device`; the
 * program's slots are "weight.<name>", "state.<layer>.<suffix>", "token",
 * "logits" and "local.<n>", its entry "forward". */
int sih_rwkv7_graph_program_create(const sih_model_tensor* tensors, int count, int64_t vocabulary, int64_t embedding,
                                   int64_t layers, const sih_graph_options* options, int device, sih_program** out);
/* The lowering's report (OptimizationReportJson) of a graph program. */
int sih_program_report(const sih_program* program, char* buffer, uint64_t capacity, uint64_t* length);
/* Without a device: the logical graph as JSON (resources, nodes with
 * operation, bindings and attributes), the lowering report and the lowered
 * program's XML.  Each buffer may be NULL (only its length is set). */
int sih_rwkv7_graph_describe(const sih_model_tensor* tensors, int count, int64_t vocabulary, int64_t embedding,
                             int64_t layers, const sih_graph_options* options, char* graph_json, uint64_t graph_capacity,
                             uint64_t* graph_length, char* report_json, uint64_t report_capacity,
                             uint64_t* report_length, char* xml, uint64_t xml_capacity, uint64_t* xml_length);

#ifdef __cplusplus
}
#endif
#endif
