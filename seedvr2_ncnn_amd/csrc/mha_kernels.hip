// gfx950 kernels of the VAE's VAEChunkedMHA (src/seedvr2/vae_chunked_mha.cpp:223-281):
// ncnn MultiHeadAttention over one blob, i.e. self attention of seq tokens of
// width qdim.
//
// The VAE attends with one head of width 512 over every pixel of a latent
// frame (14,400 tokens at 720p).  At that head width a flash kernel holds
// few query rows per wave (a 16-row x 512 fp32 output tile is 128 registers
// per lane) and its K/V fragment reads from LDS outgrow the matrix-core
// time.  With 288 GB of HBM the score matrix fits many times over, so the
// forward runs through the SharedLinear GEMM instead: the projections, S =
// Q K^T in fp32, a row softmax into bf16 P, O = P V, and the output
// projection.  This file holds the kernels between the GEMMs.
#include <math.h>

#include "mha_kernels.h"
#include "s2_device.h"

namespace s2 {
namespace {

// rows [0, rows) of x (element type `kind`, row stride qdim) -> bf16 rows of
// xp [rows_padded][qdim]; rows at or above `rows` are zero
template <int KIND>
__global__ __launch_bounds__(256) void mha_stage_kernel(const void* __restrict__ x, int rows,
                                                        int rows_padded, int qdim,
                                                        uint16_t* __restrict__ xp) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    const long total = (long)rows_padded * qdim;
    if (i >= total) return;
    const long r = i / qdim;
    float v = 0.f;
    if (r < rows) {
        if (KIND == 1)
            v = __builtin_bit_cast(float, (uint32_t)((const uint16_t*)x)[i] << 16);
        else if (KIND == 2)
            v = (float)((const _Float16*)x)[i];
        else
            v = ((const float*)x)[i];
    }
    xp[i] = f32_to_bf16(v);
}

// weights: fp32 -> bf16, times `scale`
__global__ __launch_bounds__(256) void mha_weight_kernel(const float* __restrict__ w, long n,
                                                         float scale, uint16_t* __restrict__ out) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = f32_to_bf16(w[i] * scale);
}

__global__ __launch_bounds__(256) void mha_bias_kernel(const float* __restrict__ b, int n,
                                                       float scale, float* __restrict__ out) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = b[i] * scale;
}

// One block per row of S [rows][ld_s] (fp32, scores already scaled):
// P[r][c] = exp(S - max) / sum for c < cols, 0 for cols <= c < ld_p.  The
// row is read once from HBM for the running (max, sum) and once more, from
// L2, to write P.
__global__ __launch_bounds__(256) void mha_softmax_kernel(const float* __restrict__ s, long ld_s,
                                                          int cols, int ld_p,
                                                          uint16_t* __restrict__ p) {
    constexpr float kLog2e = 1.4426950408889634f;
    __shared__ float red_m[4], red_s[4];
    const float* row = s + (long)blockIdx.x * ld_s;
    uint16_t* out = p + (long)blockIdx.x * ld_p;
    const int t = threadIdx.x;
    float m = -INFINITY, sum = 0.f;
    for (int c = t; c < cols; c += 256) {
        const float v = row[c];
        if (v > m) {
            sum = sum * __builtin_amdgcn_exp2f((m - v) * kLog2e) + 1.f;
            m = v;
        } else {
            sum += __builtin_amdgcn_exp2f((v - m) * kLog2e);
        }
    }
    // combine (max, sum) over the wave, then over the four waves
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float om = __shfl_xor(m, off), os = __shfl_xor(sum, off);
        const float nm = fmaxf(m, om);
        sum = (m == -INFINITY ? 0.f : sum * __builtin_amdgcn_exp2f((m - nm) * kLog2e)) +
              (om == -INFINITY ? 0.f : os * __builtin_amdgcn_exp2f((om - nm) * kLog2e));
        m = nm;
    }
    if ((t & 63) == 0) {
        red_m[t >> 6] = m;
        red_s[t >> 6] = sum;
    }
    __syncthreads();
    m = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
    sum = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w)
        if (red_m[w] != -INFINITY) sum += red_s[w] * __builtin_amdgcn_exp2f((red_m[w] - m) * kLog2e);
    const float inv = 1.f / sum;
    for (int c = t; c < ld_p; c += 256)
        out[c] = c < cols ? f32_to_bf16(__builtin_amdgcn_exp2f((row[c] - m) * kLog2e) * inv)
                          : (uint16_t)0;
}

// The same softmax with the row held in registers: thread t owns the float4
// groups t, t + 256, ... (NV of them, so rows up to NV * 1024 columns).  All
// loads are issued at once and the row is read from HBM once.  VEC: the row
// stride and the row start allow 16-byte loads.
template <int NV, bool VEC>
__global__ __launch_bounds__(256) void mha_softmax_reg_kernel(const float* __restrict__ s,
                                                              long ld_s, int cols, int ld_p,
                                                              uint16_t* __restrict__ p) {
    constexpr float kLog2e = 1.4426950408889634f;
    __shared__ float red[4];
    const float* row = s + (long)blockIdx.x * ld_s;
    uint16_t* out = p + (long)blockIdx.x * ld_p;
    const int t = threadIdx.x;
    float v[NV][4];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = (i * 256 + t) * 4;
        if (VEC && c + 3 < cols) {
            const float4 f = *reinterpret_cast<const float4*>(row + c);
            v[i][0] = f.x, v[i][1] = f.y, v[i][2] = f.z, v[i][3] = f.w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[i][e] = c + e < cols ? row[c + e] : -INFINITY;
        }
    }
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) m = fmaxf(m, v[i][e]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((t & 63) == 0) red[t >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();   // red is reused for the sums
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[i][e] = __builtin_amdgcn_exp2f((v[i][e] - m) * kLog2e);   // -inf -> 0
            sum += v[i][e];
        }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) sum += __shfl_xor(sum, off);
    if ((t & 63) == 0) red[t >> 6] = sum;
    __syncthreads();
    const float inv = 1.f / ((red[0] + red[1]) + (red[2] + red[3]));
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = (i * 256 + t) * 4;
        if (c >= ld_p) continue;
        // columns past `cols` hold exp(-inf) = 0; ld_p is a multiple of 4
        *reinterpret_cast<uint2*>(out + c) =
            make_uint2(pack2_bf16_rne(v[i][0] * inv, v[i][1] * inv),
                       pack2_bf16_rne(v[i][2] * inv, v[i][3] * inv));
    }
}

// head h's output [rows][d] (bf16) into columns [h*d, (h+1)*d) of O [rows][embed]
__global__ __launch_bounds__(256) void mha_interleave_kernel(const uint16_t* __restrict__ oh,
                                                             int rows, int d, int embed, int h,
                                                             uint16_t* __restrict__ o) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)rows * d) return;
    const long r = i / d;
    o[r * embed + (long)h * d + (i - r * d)] = oh[i];
}

unsigned blocks(long n) { return (unsigned)((n + 255) / 256); }

}  // namespace

hipError_t launch_mha_stage(const void* x, int kind, int rows, int rows_padded, int qdim,
                            uint16_t* xp, hipStream_t stream) {
    const long total = (long)rows_padded * qdim;
    if (total <= 0) return hipSuccess;
    if (kind == 1)
        mha_stage_kernel<1><<<blocks(total), 256, 0, stream>>>(x, rows, rows_padded, qdim, xp);
    else if (kind == 2)
        mha_stage_kernel<2><<<blocks(total), 256, 0, stream>>>(x, rows, rows_padded, qdim, xp);
    else
        mha_stage_kernel<0><<<blocks(total), 256, 0, stream>>>(x, rows, rows_padded, qdim, xp);
    return hipGetLastError();
}

hipError_t launch_mha_weight(const float* w, long n, float scale, uint16_t* out,
                             hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    mha_weight_kernel<<<blocks(n), 256, 0, stream>>>(w, n, scale, out);
    return hipGetLastError();
}

hipError_t launch_mha_bias(const float* b, int n, float scale, float* out, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    mha_bias_kernel<<<blocks(n), 256, 0, stream>>>(b, n, scale, out);
    return hipGetLastError();
}

template <int NV>
static void softmax_reg(const float* s, long ld_s, int rows, int cols, int ld_p, uint16_t* p,
                        hipStream_t stream) {
    if (ld_s % 4 == 0 && ((uintptr_t)s % 16) == 0)
        mha_softmax_reg_kernel<NV, true><<<(unsigned)rows, 256, 0, stream>>>(s, ld_s, cols, ld_p, p);
    else
        mha_softmax_reg_kernel<NV, false><<<(unsigned)rows, 256, 0, stream>>>(s, ld_s, cols, ld_p, p);
}

hipError_t launch_mha_softmax(const float* s, long ld_s, int rows, int cols, int ld_p,
                              uint16_t* p, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    // rows of up to 16,384 columns live in registers (up to 64 floats per
    // thread); longer rows take the streaming kernel
    const int groups = (ld_p + 1023) / 1024;   // float4 groups per thread
    if (ld_p % 4 != 0 || groups > 16)
        mha_softmax_kernel<<<(unsigned)rows, 256, 0, stream>>>(s, ld_s, cols, ld_p, p);
    else if (groups <= 2)
        softmax_reg<2>(s, ld_s, rows, cols, ld_p, p, stream);
    else if (groups <= 4)
        softmax_reg<4>(s, ld_s, rows, cols, ld_p, p, stream);
    else if (groups <= 8)
        softmax_reg<8>(s, ld_s, rows, cols, ld_p, p, stream);
    else
        softmax_reg<16>(s, ld_s, rows, cols, ld_p, p, stream);
    return hipGetLastError();
}

hipError_t launch_mha_interleave(const uint16_t* oh, int rows, int d, int embed, int h,
                                 uint16_t* o, hipStream_t stream) {
    const long n = (long)rows * d;
    if (n <= 0) return hipSuccess;
    mha_interleave_kernel<<<blocks(n), 256, 0, stream>>>(oh, rows, d, embed, h, o);
    return hipGetLastError();
}

}  // namespace s2
