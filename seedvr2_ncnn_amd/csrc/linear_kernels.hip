// gfx950 kernels of the SharedLinear projection (src/seedvr2/shared_linear.cpp:83-96):
// y = act(x W^T + b) for the video and the text stream in one grouped launch.
//
// x [m][k] and W [n][k] are both k-contiguous, which is the natural operand
// layout of v_mfma_f32_32x32x16_bf16 (each lane supplies 8 consecutive k of
// one row of A and one column of B), so both tiles are staged in LDS
// unchanged.  fp32 activations are rounded to bf16 while they are staged.
#include <math.h>

#include "awa_kernels.h"
#include "s2_device.h"

namespace s2 {

namespace {

__device__ __forceinline__ uint4 load_chunk(const uint16_t* p) {
    return *reinterpret_cast<const uint4*>(p);
}

__device__ __forceinline__ uint4 load_chunk(const float* p) {
    float v[8];
    load8(p, v);
    uint16_t h[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = f32_to_bf16(v[i]);
    return pack8_bf16(h);
}

__device__ __forceinline__ float gelu_erf(float x) {
    return 0.5f * x * (1.f + erff(x * 0.70710678118654752f));
}

}  // namespace

// Block tile 128x128, k-step 64, four waves in a 2x2 grid of 64x64 wave tiles
// (2x2 MFMA 32x32 accumulators per wave).  LDS double buffered, rows padded
// by 16 bytes against bank conflicts.
template <typename TX, bool Y_BF16, int ACT>
__global__ __launch_bounds__(256, 2) void shared_linear_kernel(
    const TX* __restrict__ x0, int m0, const TX* __restrict__ x1, int m1,
    const uint16_t* __restrict__ wgt, const float* __restrict__ bias, int n, int k,
    void* __restrict__ y0, void* __restrict__ y1, int mt0, int mtiles, int ntiles) {
    constexpr int BM = 128, BN = 128, BK = 64, P = BK + 8;
    constexpr int A_CHUNKS = BM * BK / 8 / 256;
    constexpr int B_CHUNKS = BN * BK / 8 / 256;
    constexpr int GROUP = 8;
    __shared__ __attribute__((aligned(16))) uint16_t a_lds[2][BM * P];
    __shared__ __attribute__((aligned(16))) uint16_t b_lds[2][BN * P];

    // XCD-aware, grouped rasterisation: consecutive logical tiles share an
    // XCD's L2, and GROUP m-tiles sweep the n-tiles together.
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int group_size = GROUP * ntiles;
    const int first_m = (lid / group_size) * GROUP;
    const int gm = min(mtiles - first_m, GROUP);
    const int mt = first_m + (lid % group_size) % gm;
    const int nt = (lid % group_size) / gm;

    const TX* x;
    int m, row0;
    void* y;
    if (mt < mt0) {
        x = x0; m = m0; y = y0; row0 = mt * BM;
    } else {
        x = x1; m = m1; y = y1; row0 = (mt - mt0) * BM;
    }
    const int col0 = nt * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l32 = lane & 31;
    const int g = lane >> 5;
    const int wm = wave >> 1;
    const int wn = wave & 1;

    uint4 areg[A_CHUNKS], breg[B_CHUNKS];
    auto load_tile = [&](int kt) {
        const int k0 = kt * BK;
#pragma unroll
        for (int c = 0; c < A_CHUNKS; ++c) {
            const int idx = tid + 256 * c;
            const int r = idx / (BK / 8);
            const int kc = k0 + (idx % (BK / 8)) * 8;
            areg[c] = make_uint4(0, 0, 0, 0);
            if (row0 + r < m && kc < k) areg[c] = load_chunk(x + (long)(row0 + r) * k + kc);
        }
#pragma unroll
        for (int c = 0; c < B_CHUNKS; ++c) {
            const int idx = tid + 256 * c;
            const int r = idx / (BK / 8);
            const int kc = k0 + (idx % (BK / 8)) * 8;
            breg[c] = make_uint4(0, 0, 0, 0);
            if (col0 + r < n && kc < k) breg[c] = load_chunk(wgt + (long)(col0 + r) * k + kc);
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int c = 0; c < A_CHUNKS; ++c) {
            const int idx = tid + 256 * c;
            *reinterpret_cast<uint4*>(&a_lds[buf][(idx / (BK / 8)) * P + (idx % (BK / 8)) * 8]) =
                areg[c];
        }
#pragma unroll
        for (int c = 0; c < B_CHUNKS; ++c) {
            const int idx = tid + 256 * c;
            *reinterpret_cast<uint4*>(&b_lds[buf][(idx / (BK / 8)) * P + (idx % (BK / 8)) * 8]) =
                breg[c];
        }
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int nk = (k + BK - 1) / BK;
    load_tile(0);
    store_tile(0);
    __syncthreads();
#pragma unroll 1
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load_tile(kt + 1);
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            bf16x8 a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                a[i] = as_bf16x8(*reinterpret_cast<const uint4*>(
                    &a_lds[buf][(wm * 64 + 32 * i + l32) * P + 16 * kk + 8 * g]));
#pragma unroll
            for (int j = 0; j < 2; ++j)
                b[j] = as_bf16x8(*reinterpret_cast<const uint4*>(
                    &b_lds[buf][(wn * 64 + 32 * j + l32) * P + 16 * kk + 8 * g]));
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store_tile(buf ^ 1);
        __syncthreads();
    }

    // Epilogue: register r of a 32x32 accumulator is row 8(r/4) + 4g + r%4,
    // column l32; bias and the activation are applied in fp32.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int col = col0 + wn * 64 + 32 * j + l32;
        if (col >= n) continue;
        const float b = bias ? bias[col] : 0.f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = row0 + wm * 64 + 32 * i + 8 * (r >> 2) + 4 * g + (r & 3);
                if (row >= m) continue;
                float v = acc[i][j][r] + b;
                if (ACT == S2_ACT_GELU) v = gelu_erf(v);
                if (Y_BF16)
                    ((uint16_t*)y)[(long)row * n + col] = f32_to_bf16(v);
                else
                    ((float*)y)[(long)row * n + col] = v;
            }
    }
}

__global__ void cast_f32_bf16_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst,
                                     size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = f32_to_bf16(src[i]);
}

__global__ void cast_bf16_f32_kernel(const uint16_t* __restrict__ src, float* __restrict__ dst,
                                     size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = bf16_to_f32(src[i]);
}

hipError_t launch_cast_f32_bf16(const float* src, uint16_t* dst, size_t n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    cast_f32_bf16_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(src, dst, n);
    return hipGetLastError();
}

hipError_t launch_cast_bf16_f32(const uint16_t* src, float* dst, size_t n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    cast_bf16_f32_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(src, dst, n);
    return hipGetLastError();
}

template <typename TX, bool Y_BF16, int ACT>
static hipError_t linear_impl(const void* x0, int m0, const void* x1, int m1, const uint16_t* w,
                              const float* bias, int n, int k, void* y0, void* y1,
                              hipStream_t stream) {
    const int mt0 = (m0 + 127) / 128;
    const int mt1 = (m1 + 127) / 128;
    const int ntiles = (n + 127) / 128;
    const int mtiles = mt0 + mt1;
    const long blocks = (long)mtiles * ntiles;
    if (blocks == 0) return hipSuccess;
    shared_linear_kernel<TX, Y_BF16, ACT><<<(unsigned)blocks, 256, 0, stream>>>(
        (const TX*)x0, m0, (const TX*)x1, m1, w, bias, n, k, y0, y1, mt0, mtiles, ntiles);
    return hipGetLastError();
}

template <typename TX, bool Y_BF16>
static hipError_t linear_act(int act, const void* x0, int m0, const void* x1, int m1,
                             const uint16_t* w, const float* bias, int n, int k, void* y0,
                             void* y1, hipStream_t stream) {
    if (act == S2_ACT_GELU)
        return linear_impl<TX, Y_BF16, S2_ACT_GELU>(x0, m0, x1, m1, w, bias, n, k, y0, y1, stream);
    return linear_impl<TX, Y_BF16, S2_ACT_NONE>(x0, m0, x1, m1, w, bias, n, k, y0, y1, stream);
}

hipError_t launch_shared_linear(const void* x0, int m0, const void* x1, int m1, bool x_bf16,
                                const uint16_t* w, const float* bias, int n, int k, int act,
                                void* y0, void* y1, bool y_bf16, hipStream_t stream) {
    if (x_bf16)
        return y_bf16 ? linear_act<uint16_t, true>(act, x0, m0, x1, m1, w, bias, n, k, y0, y1, stream)
                      : linear_act<uint16_t, false>(act, x0, m0, x1, m1, w, bias, n, k, y0, y1, stream);
    return y_bf16 ? linear_act<float, true>(act, x0, m0, x1, m1, w, bias, n, k, y0, y1, stream)
                  : linear_act<float, false>(act, x0, m0, x1, m1, w, bias, n, k, y0, y1, stream);
}

}  // namespace s2
