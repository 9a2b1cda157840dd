// Host launchers of the DiT block's norm and AdaSingle modulation kernels
// (block_kernels.hip): the operations between the block's inputs, its
// modulation vectors and the SharedLinear / window-attention hot path.
#pragma once

#include <hip/hip_runtime.h>

namespace s2 {

// samples per launch (video and text each)
constexpr int kAdaMaxBatch = 64;
// widest hidden size the kernels hold in registers
constexpr int kAdaMaxDim = 4096;

// Rows of the two streams of one launch: video rows [0, video_rows) then text
// rows; end[b] / end[kAdaMaxBatch + b] are the cumulative row ends of video /
// text sample b.
struct AdaRows {
    int batch;
    int video_rows, text_rows;
    int end[2 * kAdaMaxBatch];
};

// Element types: 0 fp32, 1 bf16, 2 fp16 (the s2_dtype values).  Strides are
// in elements; dim % 4 == 0, dim <= kAdaMaxDim, 16-byte aligned fp32 rows and
// 8-byte aligned 16-bit rows.
struct AdaInArgs {
    const void* x[2];   // video, text
    long x_stride;
    int x_kind;
    void* out[2];
    long out_stride;
    int out_kind;
    int dim;
    float eps;
    const float* shift_a;   // [batch][dim]
    const float* scale_a;
    const float* shift_b[2];   // [dim] per stream, or null
    const float* scale_b[2];
    AdaRows rows;
};

struct AdaOutArgs {
    const void* x[2];
    long x_stride;
    void* out[2];   // may equal x
    long out_stride;
    int x_kind;     // residual and out element type
    const void* y[2];
    long y_stride;
    int y_kind;
    int dim;
    const float* gate_a;      // [batch][dim]
    const float* gate_b[2];   // [dim] per stream, or null
    AdaRows rows;
    // norm != 0: also h = norm(out) * (scale_a[b] + scale_b) + (shift_a[b] +
    // shift_b) of the stored out rows, into h (element type h_kind)
    int norm;
    void* h[2];
    long h_stride;
    int h_kind;
    float eps;
    const float* shift_a;
    const float* scale_a;
    const float* shift_b[2];
    const float* scale_b[2];
};

// out = norm(x) * (scale_a[b] + scale_b) + (shift_a[b] + shift_b)
hipError_t launch_ada_in(const AdaInArgs& a, hipStream_t stream);
// out = x + y * (gate_a[b] + gate_b), and with a.norm the modulated norm of
// out (the next ada_in) in the same pass
hipError_t launch_ada_out(const AdaOutArgs& a, hipStream_t stream);

}  // namespace s2
