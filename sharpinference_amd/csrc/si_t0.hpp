// T0 primitive and portable tensor operators (si_t0.hip), shared by the C
// ABI (si_t0_abi.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace si {

// Elementwise operators; the values are the C ABI's si_hip_t0_op.
enum T0Op : int {
    T0_COPY = 0,
    T0_ADD = 1,
    T0_SUBTRACT = 2,
    T0_MULTIPLY = 3,
    T0_DIVIDE = 4,
    T0_MAXIMUM = 5,
    T0_EXP = 6,
    T0_TANH = 7,
    T0_SIGMOID = 8,
    T0_RSQRT = 9,
    T0_SQUARE = 10,
    T0_RELU = 11,
};
constexpr int T0_OP_COUNT = 12;
inline bool t0_binary(int op) { return op >= T0_ADD && op <= T0_MAXIMUM; }

// Output coordinates -> input element: in[base + sum_a coord_a * strides[a]].
constexpr int T0_MAX_RANK = 4;
struct GatherShape {
    int rank;
    int64_t count;                  // product of dims
    int64_t dims[T0_MAX_RANK];      // output dimensions, row-major
    int64_t strides[T0_MAX_RANK];   // input element stride per output axis (0: repeated)
    int64_t base;
};

// out[i] = op(l[i]) or op(l[i], r[i]) for i < n.
hipError_t launch_t0_elementwise(int op, const float* l, const float* r, float* o, int64_t n, hipStream_t s);
hipError_t launch_t0_cast_f16(const void* in, float* o, int64_t n, hipStream_t s);
hipError_t launch_t0_fill(float* o, float v, int64_t n, hipStream_t s);
// out[r] = sum (or mean) of in[r][0..cols).
hipError_t launch_t0_reduce_last(bool mean, const float* in, float* o, int64_t rows, int64_t cols, hipStream_t s);
hipError_t launch_t0_gather(const float* in, float* o, const GatherShape& g, hipStream_t s);
// out[h][i][j] = l[h][i] * r[h][j].
hipError_t launch_t0_head_outer(const float* l, const float* r, float* o, int64_t heads, int64_t rows, int64_t cols,
                                hipStream_t s);

}  // namespace si
