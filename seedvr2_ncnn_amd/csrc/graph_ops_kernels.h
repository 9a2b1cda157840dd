// Launchers of the graph built-in layers' kernels (graph_ops_kernels.hip).
// Element kinds are the s2_dtype codes (0 fp32, 1 bf16, 2 fp16); row strides
// are in elements.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace s2 {

struct BinaryArgs {
    int op;
    const void* a;
    int a_kind;
    long a_rs;   // 0: a row broadcast over the rows
    int a_cs;    // 1, or 0: an element broadcast over the columns
    const void* b;   // null: b_scalar
    int b_kind;
    long b_rs;
    int b_cs;
    float b_scalar;
    void* y;
    int y_kind;
    long y_rs;
    int rows, cols;
};

hipError_t launch_binary(const BinaryArgs& p, hipStream_t stream);
hipError_t launch_unary(int op, const void* x, int x_kind, void* y, int y_kind, size_t n,
                        hipStream_t stream);
// axis 1: each row to one value (y[rows]); axis 0: each column (y[cols])
hipError_t launch_reduce(int op, float coeff, int axis, const void* x, int x_kind, long x_rs,
                         int rows, int cols, void* y, int y_kind, hipStream_t stream);
hipError_t launch_rms_norm(const void* x, int x_kind, long x_rs, int rows, int cols,
                           const float* gamma, float eps, void* y, int y_kind, long y_rs,
                           hipStream_t stream);
hipError_t launch_copy2d(const void* src, int s_kind, long s_rs, void* dst, int d_kind, long d_rs,
                         int rows, int cols, hipStream_t stream);

}  // namespace s2
