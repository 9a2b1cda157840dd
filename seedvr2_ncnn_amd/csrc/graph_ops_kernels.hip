// gfx950 kernels of the ncnn built-in layers that exported SeedVR2 graphs
// place around the custom layers: elementwise BinaryOp / UnaryOp / Sigmoid /
// Swish, Reduction, RMSNorm, and a strided 2-D copy with element-type
// conversion (Slice, Concat, Crop, Reshape).  The reference runs these as
// ncnn's Vulkan built-ins (the graphs of src/seedvr2/seedvr2_dit.cpp:603-633;
// Reduction_vulkan is patched for large row counts in
// patches/ncnn/0002-seedvr2-large-vulkan-workloads.patch:256-284).
//
// All of them stream HBM: one read of every operand element and one write
// of every output element.  Elements are fp32, bf16 or fp16 (s2_dtype codes
// 0/1/2) and computed in fp32.  Rows run along blockIdx.y chunks, columns
// along threads, so every access of a wave is contiguous.
#include <math.h>

#include <algorithm>

#include "graph_ops_kernels.h"
#include "s2_device.h"

namespace s2 {

namespace {

__device__ __forceinline__ float ld(const void* p, long i, int kind) {
    if (kind == 1) return bf16_to_f32(((const uint16_t*)p)[i]);
    if (kind == 2) return (float)((const _Float16*)p)[i];
    return ((const float*)p)[i];
}

__device__ __forceinline__ void st(void* p, long i, int kind, float v) {
    if (kind == 1)
        ((uint16_t*)p)[i] = f32_to_bf16(v);
    else if (kind == 2)
        ((_Float16*)p)[i] = f32_to_f16(v);
    else
        ((float*)p)[i] = v;
}

// ncnn BinaryOp op_type: 0 add, 1 sub, 2 mul, 3 div, 4 max, 5 min, 6 pow,
// 7 rsub, 8 rdiv, 9 rpow, 10 atan2, 11 ratan2
__device__ __forceinline__ float binary(int op, float a, float b) {
    switch (op) {
        case 0: return a + b;
        case 1: return a - b;
        case 2: return a * b;
        case 3: return a / b;
        case 4: return fmaxf(a, b);
        case 5: return fminf(a, b);
        case 6: return powf(a, b);
        case 7: return b - a;
        case 8: return b / a;
        case 9: return powf(b, a);
        case 10: return atan2f(a, b);
        default: return atan2f(b, a);
    }
}

// ncnn UnaryOp op_type 0..19, then this build's codes 100 sigmoid, 101 swish
__device__ __forceinline__ float unary(int op, float x) {
    switch (op) {
        case 0: return fabsf(x);
        case 1: return -x;
        case 2: return floorf(x);
        case 3: return ceilf(x);
        case 4: return x * x;
        case 5: return sqrtf(x);
        case 6: return 1.f / sqrtf(x);
        case 7: return expf(x);
        case 8: return logf(x);
        case 9: return sinf(x);
        case 10: return cosf(x);
        case 11: return tanf(x);
        case 12: return asinf(x);
        case 13: return acosf(x);
        case 14: return atanf(x);
        case 15: return 1.f / x;
        case 16: return tanhf(x);
        case 17: return log10f(x);
        case 18: return rintf(x);
        case 19: return truncf(x);
        case 100: return 1.f / (1.f + expf(-x));
        default: return x / (1.f + expf(-x));
    }
}

constexpr int kThreads = 256;

// y[r][c] = op(a[r * ar][c * ac], b[r * br][c * bc]); ar/ac/br/bc are 0 on a
// broadcast axis.  b == null: the scalar bs.
__global__ void binary_kernel(BinaryArgs p) {
    const int c = blockIdx.x * kThreads + threadIdx.x;
    if (c >= p.cols) return;
    for (int r = blockIdx.y; r < p.rows; r += gridDim.y) {
        const float a = ld(p.a, (long)r * p.a_rs + (long)c * p.a_cs, p.a_kind);
        const float b = p.b ? ld(p.b, (long)r * p.b_rs + (long)c * p.b_cs, p.b_kind) : p.b_scalar;
        st(p.y, (long)r * p.y_rs + c, p.y_kind, binary(p.op, a, b));
    }
}

__global__ void unary_kernel(int op, const void* x, int x_kind, void* y, int y_kind, size_t n) {
    for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n;
         i += (size_t)gridDim.x * kThreads)
        st(y, (long)i, y_kind, unary(op, ld(x, (long)i, x_kind)));
}

// Reduction operations (ncnn's ids): 0 sum, 1 asum, 2 sumsq, 3 mean, 4 max,
// 5 min, 6 prod, 7 l1, 8 l2, 9 logsum, 10 logsumexp.  The pre-map, the
// combine and the final map of each.
__device__ __forceinline__ float red_pre(int op, float x) {
    switch (op) {
        case 1: case 7: return fabsf(x);
        case 2: case 8: return x * x;
        case 10: return expf(x);
        default: return x;
    }
}
__device__ __forceinline__ float red_id(int op) {
    if (op == 4) return -INFINITY;
    if (op == 5) return INFINITY;
    if (op == 6) return 1.f;
    return 0.f;
}
__device__ __forceinline__ float red_comb(int op, float a, float b) {
    if (op == 4) return fmaxf(a, b);
    if (op == 5) return fminf(a, b);
    if (op == 6) return a * b;
    return a + b;
}
__device__ __forceinline__ float red_post(int op, float v, int n, float coeff) {
    if (op == 3) v = v / (float)n;
    if (op == 8) v = sqrtf(v);
    if (op == 9 || op == 10) v = logf(v);
    return v * coeff;
}

// One workgroup per row (a grid-stride over rows): per-thread partials in
// column order, then a tree over the workgroup.
__global__ void reduce_rows_kernel(int op, float coeff, const void* x, int x_kind, long x_rs,
                                   int rows, int cols, void* y, int y_kind) {
    __shared__ float part[kThreads];
    for (int r = blockIdx.x; r < rows; r += gridDim.x) {
        float acc = red_id(op);
        for (int c = threadIdx.x; c < cols; c += kThreads)
            acc = red_comb(op, acc, red_pre(op, ld(x, (long)r * x_rs + c, x_kind)));
        part[threadIdx.x] = acc;
        __syncthreads();
        for (int s = kThreads / 2; s > 0; s >>= 1) {
            if (threadIdx.x < s) part[threadIdx.x] = red_comb(op, part[threadIdx.x], part[threadIdx.x + s]);
            __syncthreads();
        }
        if (threadIdx.x == 0) st(y, r, y_kind, red_post(op, part[0], cols, coeff));
        __syncthreads();
    }
}

// One thread per column, rows in order.
__global__ void reduce_cols_kernel(int op, float coeff, const void* x, int x_kind, long x_rs,
                                   int rows, int cols, void* y, int y_kind) {
    const int c = blockIdx.x * kThreads + threadIdx.x;
    if (c >= cols) return;
    float acc = red_id(op);
    for (int r = 0; r < rows; ++r) acc = red_comb(op, acc, red_pre(op, ld(x, (long)r * x_rs + c, x_kind)));
    st(y, c, y_kind, red_post(op, acc, rows, coeff));
}

// y = x / sqrt(mean(x^2) + eps) [* gamma]: one workgroup per row.
__global__ void rms_norm_kernel(const void* x, int x_kind, long x_rs, int rows, int cols,
                                const float* gamma, float eps, void* y, int y_kind, long y_rs) {
    __shared__ float part[kThreads];
    for (int r = blockIdx.x; r < rows; r += gridDim.x) {
        float ss = 0.f;
        for (int c = threadIdx.x; c < cols; c += kThreads) {
            const float v = ld(x, (long)r * x_rs + c, x_kind);
            ss = fmaf(v, v, ss);
        }
        part[threadIdx.x] = ss;
        __syncthreads();
        for (int s = kThreads / 2; s > 0; s >>= 1) {
            if (threadIdx.x < s) part[threadIdx.x] += part[threadIdx.x + s];
            __syncthreads();
        }
        const float inv = 1.f / sqrtf(part[0] / (float)cols + eps);
        for (int c = threadIdx.x; c < cols; c += kThreads) {
            float v = ld(x, (long)r * x_rs + c, x_kind) * inv;
            if (gamma) v *= gamma[c];
            st(y, (long)r * y_rs + c, y_kind, v);
        }
        __syncthreads();
    }
}

__global__ void copy2d_kernel(const void* src, int s_kind, long s_rs, void* dst, int d_kind,
                              long d_rs, int rows, int cols) {
    const int c = blockIdx.x * kThreads + threadIdx.x;
    if (c >= cols) return;
    for (int r = blockIdx.y; r < rows; r += gridDim.y)
        st(dst, (long)r * d_rs + c, d_kind, ld(src, (long)r * s_rs + c, s_kind));
}

dim3 grid2d(int rows, int cols) {
    const unsigned gx = (unsigned)((cols + kThreads - 1) / kThreads);
    // enough row chunks to fill the chip several times over
    const unsigned gy = (unsigned)std::max(1, std::min(rows, std::max(1, 8192 / (int)gx)));
    return dim3(gx, gy);
}

}  // namespace

hipError_t launch_binary(const BinaryArgs& p, hipStream_t stream) {
    if (p.rows <= 0 || p.cols <= 0) return hipSuccess;
    binary_kernel<<<grid2d(p.rows, p.cols), kThreads, 0, stream>>>(p);
    return hipGetLastError();
}

hipError_t launch_unary(int op, const void* x, int x_kind, void* y, int y_kind, size_t n,
                        hipStream_t stream) {
    if (n == 0) return hipSuccess;
    const size_t blocks = std::min<size_t>((n + kThreads - 1) / kThreads, 16384);
    unary_kernel<<<(unsigned)blocks, kThreads, 0, stream>>>(op, x, x_kind, y, y_kind, n);
    return hipGetLastError();
}

hipError_t launch_reduce(int op, float coeff, int axis, const void* x, int x_kind, long x_rs,
                         int rows, int cols, void* y, int y_kind, hipStream_t stream) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    if (axis == 1) {
        reduce_rows_kernel<<<(unsigned)std::min(rows, 65536), kThreads, 0, stream>>>(
            op, coeff, x, x_kind, x_rs, rows, cols, y, y_kind);
    } else {
        reduce_cols_kernel<<<(unsigned)((cols + kThreads - 1) / kThreads), kThreads, 0, stream>>>(
            op, coeff, x, x_kind, x_rs, rows, cols, y, y_kind);
    }
    return hipGetLastError();
}

hipError_t launch_rms_norm(const void* x, int x_kind, long x_rs, int rows, int cols,
                           const float* gamma, float eps, void* y, int y_kind, long y_rs,
                           hipStream_t stream) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    rms_norm_kernel<<<(unsigned)std::min(rows, 65536), kThreads, 0, stream>>>(
        x, x_kind, x_rs, rows, cols, gamma, eps, y, y_kind, y_rs);
    return hipGetLastError();
}

hipError_t launch_copy2d(const void* src, int s_kind, long s_rs, void* dst, int d_kind, long d_rs,
                         int rows, int cols, hipStream_t stream) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    copy2d_kernel<<<grid2d(rows, cols), kThreads, 0, stream>>>(src, s_kind, s_rs, dst, d_kind, d_rs,
                                                               rows, cols);
    return hipGetLastError();
}

}  // namespace s2
