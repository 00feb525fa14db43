// Context and plan state shared by the C-ABI translation units, plus the
// error helpers every entry point uses.  Not part of the public ABI.
#pragma once

#include "sharpinference_hip.h"
#include "si_internal.hpp"

#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

struct si_hip_context {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t t0 = nullptr;
    hipEvent_t t1 = nullptr;
    bool timer_open = false;
    bool recording = false;
    float* attention_scratch = nullptr;   // device address of the library's attention scratch on `device`
    void* prefill_split = nullptr;        // si::PREFILL_SPLIT_BYTES for the prefill's split-K partial sums (or null)
    std::string error;
    std::recursive_mutex gate;
};

struct si_hip_plan {
    si_hip_context* ctx = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace si_abi {

int fail(si_hip_context* ctx, int code, const char* fmt, ...);
const char* thread_error();
int hip_fail(si_hip_context* ctx, hipError_t e, const char* what);

// Locks the context and makes its device current on this thread.
struct Enter {
    std::unique_lock<std::recursive_mutex> lock;
    hipError_t err;
    explicit Enter(si_hip_context* ctx) : lock(ctx->gate), err(hipSetDevice(ctx->device)) {}
};

inline bool overlaps(const void* a, uint64_t an, const void* b, uint64_t bn)
{
    const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
    return an != 0 && bn != 0 && pa < pb + bn && pb < pa + an;
}

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

bool is_quant(int fmt);
const char* fmt_name(int fmt);
int check_matrix(si_hip_context* ctx, const char* op, int fmt, const void* w, int64_t rows, int64_t cols,
                 uint64_t* wbytes);

}  // namespace si_abi
