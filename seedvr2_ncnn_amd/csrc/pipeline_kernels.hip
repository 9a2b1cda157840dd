// gfx950 kernels of the steps either side of the DiT block stack: the video
// patchify and timestep embedding of the frontend, the unpatchify of the
// tail, and the sampler's classifier-free guidance and Euler update.
//
// All of them are HBM-bound moves of fp32 data.  The permutations are laid out
// so that both sides of every copy are contiguous runs (no gathers), and the
// transposes between the channel-planar latent and token-major rows go through
// LDS.  The arithmetic is the reference's fp32 operation sequence with every
// product and sum rounded on its own (no FMA contraction), so guidance and
// the Euler update reproduce the reference's x86-64 results bit for bit; the
// guidance rescale statistics are accumulated in fp64 like the reference's.
#include <math.h>


#include "pipeline_kernels.h"
#include "stream_scratch.h"

namespace s2 {
namespace {

constexpr int kThreads = 256;
constexpr int kTilePatches = 32;   // patches of one patch row per transposing block

unsigned blocks_for(long work, int per_block) { return (unsigned)((work + per_block - 1) / per_block); }

// ---- patchify (seedvr2_dit.cpp:167-230) --------------------------------------
//
// Patch (f, py, px) is [token (2py, 2px) | (2py, 2px+1) | (2py+1, 2px) |
// (2py+1, 2px+1)], 33 floats each.  Tokens 2px and 2px+1 of one token row are
// adjacent, so a patch is two 66-float runs, floats px*66 .. px*66+65 of token
// rows 2py and 2py+1, and token row 2*(f*ph + py) + y of the sample is the y-th
// row of patch row f*ph + py.  Runs start at even floats (width is even): the
// copy moves float2s.
__global__ void __launch_bounds__(kThreads) patchify_kernel(const float2* __restrict__ src,
                                                            int pw, int per_row, int blocks_per_row,
                                                            float2* __restrict__ dst) {
    const int prow = blockIdx.x / blocks_per_row;          // f*ph + py
    const int j = (blockIdx.x - prow * blocks_per_row) * kThreads + threadIdx.x;
    if (j >= per_row) return;                               // per_row = pw*66 float2s
    const int px = j / 66;
    const int r = j - px * 66;
    const int y = r >= 33;
    const int k = r - 33 * y;
    const long row = 2L * prow + y;
    dst[(long)prow * per_row + j] = src[row * pw * 33 + px * 33 + k];
}

// ---- latent + condition -> patches (seedvr2_pipeline.cpp:296-317, then
// seedvr2_dit.cpp:167-230) -----------------------------------------------------
//
// Token t of the sample is [latent[0..15][t] | condition[0..15][t] | 1].  One
// block builds 32 patches of one patch row: it reads the 64 token columns of
// both token rows from each of the 32 planes (256-byte runs), transposes them
// in LDS to [y][column][33] and writes the 32 patches as one contiguous
// 16.5 KB run.
__global__ void __launch_bounds__(kThreads) latent_patches_kernel(
    const float* __restrict__ latent, const float* __restrict__ condition, long cstride,
    int width, int pw, int tiles_per_row, float* __restrict__ dst) {
    __shared__ float tile[2 * 64 * 33];
    const int prow = blockIdx.x / tiles_per_row;
    const int px0 = (blockIdx.x - prow * tiles_per_row) * kTilePatches;
    const int npatch = min(kTilePatches, pw - px0);
    const int ncol = 2 * npatch;
    const int tid = threadIdx.x;
    const int col = tid & 63;
    const long col0 = 2L * px0;
#pragma unroll 4
    for (int cy = tid >> 6; cy < 64; cy += 4) {
        const int c = cy >> 1, y = cy & 1;
        const float* plane = c < 16 ? latent + c * cstride : condition + (c - 16) * cstride;
        const long tok = (2L * prow + y) * width + col0 + col;
        if (col < ncol) tile[(y * 64 + col) * 33 + c] = plane[tok];
    }
    if (tid < 128) tile[tid * 33 + 32] = 1.f;
    __syncthreads();
    float* out = dst + ((long)prow * pw + px0) * 132;
    const int total = npatch * 132;
    for (int o = tid; o < total; o += kThreads) {
        const int p = o / 132;
        const int rem = o - p * 132;
        const int y = rem >= 66;
        out[o] = tile[y * 2112 + p * 66 + (rem - 66 * y)];
    }
}

// ---- unpatchify (seedvr2_dit.cpp:255-326) -----------------------------------
//
// Token row yy of frame f reads patch row f*ph + yy/2: its tokens 2px, 2px+1
// are the 32-float run at float (yy&1)*32 of patch px.  The copy moves float4s.
__global__ void __launch_bounds__(kThreads) unpatchify_kernel(const float4* __restrict__ src,
                                                              int pw, int per_row, int blocks_per_row,
                                                              float4* __restrict__ dst) {
    const int row = blockIdx.x / blocks_per_row;           // f*height + yy
    const int j = (blockIdx.x - row * blocks_per_row) * kThreads + threadIdx.x;
    if (j >= per_row) return;                               // per_row = width*4 float4s
    const int px = j >> 3;
    const long prow = row >> 1;                             // f*ph + yy/2
    dst[(long)row * per_row + j] = src[(prow * pw + px) * 16 + (row & 1) * 8 + (j & 7)];
}

// ---- timestep embedding (seedvr2_dit.cpp:232-253) ---------------------------

struct Timesteps {
    float t[64];
};

// ln(10000) rounded to fp32 (0x41135D8E), the value of logf(10000.f)
constexpr float kLn10000 = 9.21034049987793f;

// Row s: [sin(t_s f_i) | cos(t_s f_i)], f_i = exp(-ln(10000) i / 128).  The
// exponent and the phase are the reference's fp32 products; exp, sin and cos
// are evaluated in fp64 and rounded once, which gives the correctly rounded
// fp32 value.
__global__ void __launch_bounds__(128) timestep_kernel(Timesteps ts, float* __restrict__ out) {
#pragma clang fp contract(off)
    const int i = threadIdx.x;
    const float exponent = (-kLn10000 * (float)i) / 128.f;
    const float freq = (float)exp((double)exponent);
    const float phase = ts.t[blockIdx.x] * freq;
    float* row = out + (long)blockIdx.x * 256;
    row[i] = (float)sin((double)phase);
    row[i + 128] = (float)cos((double)phase);
}

// ---- classifier-free guidance (seedvr2_pipeline.cpp:171-210) -----------------
//
// cfg = neg + scale (pos - neg).  With rescale, cfg *= (float)(rescale
// std(pos)/std(cfg) + (1 - rescale)), the sample standard deviations over all
// elements, unless std(cfg) is 0.  The statistics pass keeps, per block, the
// count, mean and sum of squared deviations (M2) of pos and cfg in fp64 and
// merges chunks and blocks with the pairwise update of Chan et al.: the same
// two-pass quantities as the reference's, summed in another order.

constexpr int kStatChunk = 4096;           // elements per block iteration, 16 per thread
constexpr int kMaxStatBlocks = 1024;

struct Moments {
    double n, mp, qp, mc, qc;   // count; mean and M2 of pos; mean and M2 of cfg
};

__device__ __forceinline__ void merge(Moments& a, const Moments& b) {
    if (b.n == 0.0) return;
    if (a.n == 0.0) {
        a = b;
        return;
    }
    const double n = a.n + b.n;
    const double wb = b.n / n;
    const double dp = b.mp - a.mp, dc = b.mc - a.mc;
    a.mp += dp * wb;
    a.qp += b.qp + dp * dp * a.n * wb;
    a.mc += dc * wb;
    a.qc += b.qc + dc * dc * a.n * wb;
    a.n = n;
}

struct CfgScratch {
    Moments rec[kMaxStatBlocks];
    int arrivals;       // blocks of the running statistics pass; 0 between launches
    float factor[2];    // {factor, 1 = apply / 0 = leave cfg unscaled}
};

__device__ __forceinline__ float cfg_value(float p, float n, float scale) {
#pragma clang fp contract(off)
    return n + scale * (p - n);
}

// Sum of two doubles over the block, the same value in every thread.
__device__ __forceinline__ void block_sum2(double& a, double& b, double* red) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        a += __shfl_xor(a, m);
        b += __shfl_xor(b, m);
    }
    const int wave = threadIdx.x >> 6;
    __syncthreads();   // red[] is free (its last readers are past this barrier)
    if ((threadIdx.x & 63) == 0) {
        red[2 * wave] = a;
        red[2 * wave + 1] = b;
    }
    __syncthreads();
    a = (red[0] + red[2]) + (red[4] + red[6]);
    b = (red[1] + red[3]) + (red[5] + red[7]);
}

// Pass 1: cfg (stored when out is non-null) and the moments of pos and cfg.
// The last block to finish merges the per-block moments in block order and
// writes the factor.
__global__ void __launch_bounds__(kThreads) cfg_stats_kernel(const float* __restrict__ pos,
                                                             const float* __restrict__ neg,
                                                             long count, float scale, float rescale,
                                                             float* __restrict__ out,
                                                             CfgScratch* sc) {
    __shared__ double red[8];
    __shared__ Moments all[kThreads];
    __shared__ int last;
    const int tid = threadIdx.x;
    const long chunks = (count + kStatChunk - 1) / kStatChunk;
    Moments acc = {0.0, 0.0, 0.0, 0.0, 0.0};
    for (long ch = blockIdx.x; ch < chunks; ch += gridDim.x) {
        const long base = ch * kStatChunk;
        float p[16], g[16];
        bool ok[16];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const long i = base + j * 1024 + tid * 4;
            if (i + 3 < count) {
                const float4 a = *reinterpret_cast<const float4*>(pos + i);
                const float4 b = *reinterpret_cast<const float4*>(neg + i);
                p[4 * j] = a.x, p[4 * j + 1] = a.y, p[4 * j + 2] = a.z, p[4 * j + 3] = a.w;
                g[4 * j] = cfg_value(a.x, b.x, scale);
                g[4 * j + 1] = cfg_value(a.y, b.y, scale);
                g[4 * j + 2] = cfg_value(a.z, b.z, scale);
                g[4 * j + 3] = cfg_value(a.w, b.w, scale);
                ok[4 * j] = ok[4 * j + 1] = ok[4 * j + 2] = ok[4 * j + 3] = true;
                if (out)
                    *reinterpret_cast<float4*>(out + i) =
                        make_float4(g[4 * j], g[4 * j + 1], g[4 * j + 2], g[4 * j + 3]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    ok[4 * j + e] = i + e < count;
                    p[4 * j + e] = ok[4 * j + e] ? pos[i + e] : 0.f;
                    const float nv = ok[4 * j + e] ? neg[i + e] : 0.f;
                    g[4 * j + e] = cfg_value(p[4 * j + e], nv, scale);
                    if (out && ok[4 * j + e]) out[i + e] = g[4 * j + e];
                }
            }
        }
        double sp = 0.0, sg = 0.0;
#pragma unroll
        for (int e = 0; e < 16; ++e)
            if (ok[e]) {
                sp += (double)p[e];
                sg += (double)g[e];
            }
        block_sum2(sp, sg, red);
        const double n = (double)min((long)kStatChunk, count - base);
        const double mp = sp / n, mg = sg / n;
        double qp = 0.0, qg = 0.0;
#pragma unroll
        for (int e = 0; e < 16; ++e)
            if (ok[e]) {
                const double dp = (double)p[e] - mp, dg = (double)g[e] - mg;
                qp += dp * dp;
                qg += dg * dg;
            }
        block_sum2(qp, qg, red);
        merge(acc, Moments{n, mp, qp, mg, qg});
    }
    if (tid == 0) {
        sc->rec[blockIdx.x] = acc;
        // release: the record is visible device-wide before the arrival counts
        const int before = __hip_atomic_fetch_add(&sc->arrivals, 1, __ATOMIC_ACQ_REL,
                                                  __HIP_MEMORY_SCOPE_AGENT);
        last = before == (int)gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    Moments m = {0.0, 0.0, 0.0, 0.0, 0.0};
    for (int b = tid; b < (int)gridDim.x; b += kThreads) merge(m, sc->rec[b]);
    all[tid] = m;
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1) {
        if (tid < s) merge(all[tid], all[tid + s]);
        __syncthreads();
    }
    if (tid == 0) {
        const double denom = (double)(count - 1);
        const double pos_std = sqrt(all[0].qp / denom);
        const double cfg_std = sqrt(all[0].qc / denom);
        float factor = 1.f, apply = 0.f;
        if (!(cfg_std == 0.0)) {
            factor = (float)((double)rescale * pos_std / cfg_std + (double)(1.f - rescale));
            apply = 1.f;
        }
        sc->factor[0] = factor;
        sc->factor[1] = apply;
        __hip_atomic_store(&sc->arrivals, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

__global__ void __launch_bounds__(kThreads) cfg_kernel(const float* __restrict__ pos,
                                                       const float* __restrict__ neg, long count,
                                                       float scale, float* __restrict__ out) {
    const long i = ((long)blockIdx.x * kThreads + threadIdx.x) * 4;
    if (i + 3 < count) {
        const float4 a = *reinterpret_cast<const float4*>(pos + i);
        const float4 b = *reinterpret_cast<const float4*>(neg + i);
        *reinterpret_cast<float4*>(out + i) =
            make_float4(cfg_value(a.x, b.x, scale), cfg_value(a.y, b.y, scale),
                        cfg_value(a.z, b.z, scale), cfg_value(a.w, b.w, scale));
    } else {
        for (long e = i; e < count; ++e) out[e] = cfg_value(pos[e], neg[e], scale);
    }
}

// Pass 2 of apply_cfg: cfg *= factor, skipped when std(cfg) was 0.
__global__ void __launch_bounds__(kThreads) cfg_scale_kernel(float* __restrict__ out, long count,
                                                             const float* __restrict__ factor) {
#pragma clang fp contract(off)
    if (factor[1] == 0.f) return;
    const float f = factor[0];
    const long i = ((long)blockIdx.x * kThreads + threadIdx.x) * 4;
    if (i + 3 < count) {
        float4 v = *reinterpret_cast<const float4*>(out + i);
        v.x *= f, v.y *= f, v.z *= f, v.w *= f;
        *reinterpret_cast<float4*>(out + i) = v;
    } else {
        for (long e = i; e < count; ++e) out[e] *= f;
    }
}

// ---- Euler update (seedvr2_pipeline.cpp:575-588) ----------------------------
//
// One block moves 256 tokens: their [256][16] prediction rows are read as
// float4s, transposed in LDS, and each thread updates its token in the 16
// latent planes (256-byte runs per wave).
__global__ void __launch_bounds__(kThreads) euler_kernel(float* __restrict__ latent, long cstride,
                                                         const float* __restrict__ pred,
                                                         long tokens, float delta) {
#pragma clang fp contract(off)
    __shared__ float tile[kThreads * 17];
    const int tid = threadIdx.x;
    const long t0 = (long)blockIdx.x * kThreads;
    const int nt = (int)min((long)kThreads, tokens - t0);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = (j * kThreads + tid) * 4;   // element of the block's [256][16]
        const int t = e >> 4, c = e & 15;
        if (t < nt) {
            const float4 v = *reinterpret_cast<const float4*>(pred + (t0 + t) * 16 + c);
            float* d = tile + t * 17 + c;
            d[0] = v.x, d[1] = v.y, d[2] = v.z, d[3] = v.w;
        }
    }
    __syncthreads();
    if (tid >= nt) return;
    float* dst = latent + t0 + tid;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
        const float step = delta * tile[tid * 17 + c];
        dst[c * cstride] = dst[c * cstride] + step;
    }
}

// ---- fused sampler update ----------------------------------------------------
//
// The block of 32 patches of one patch row covers token columns 2*px0 ..
// 2*px0+63 of token rows 2py and 2py+1.  It reads the patch rows (float4s,
// contiguous), forms the guided prediction, transposes it in LDS to
// [y][column][16] and updates the 16 latent planes (256-byte runs per wave).
// The products are the reference's: cfg = neg + scale (pos - neg), cfg *=
// factor, step = delta * cfg, latent += step.
__global__ void __launch_bounds__(kThreads) denoise_update_kernel(
    const float* __restrict__ pos, const float* __restrict__ neg, float scale,
    const float* __restrict__ factor, float delta, float* __restrict__ latent, long cstride,
    int width, int pw, int tiles_per_row) {
#pragma clang fp contract(off)
    __shared__ float tile[2 * 64 * 17];
    const int prow = blockIdx.x / tiles_per_row;
    const int px0 = (blockIdx.x - prow * tiles_per_row) * kTilePatches;
    const int npatch = min(kTilePatches, pw - px0);
    const int tid = threadIdx.x;
    const bool scaled = factor && factor[1] != 0.f;
    const float f = factor ? factor[0] : 1.f;
    const long pbase = ((long)prow * pw + px0) * 64;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int e = (j * kThreads + tid) * 4;   // element of the block's [32][64]
        const int p = e >> 6, rem = e & 63;
        if (p < npatch) {
            float4 v = *reinterpret_cast<const float4*>(pos + pbase + e);
            if (neg) {
                const float4 b = *reinterpret_cast<const float4*>(neg + pbase + e);
                v = make_float4(cfg_value(v.x, b.x, scale), cfg_value(v.y, b.y, scale),
                                cfg_value(v.z, b.z, scale), cfg_value(v.w, b.w, scale));
                if (scaled) v.x *= f, v.y *= f, v.z *= f, v.w *= f;
            }
            // rem = y*32 + x*16 + c: token column 2p + x of token row y
            const int y = rem >> 5, x = (rem >> 4) & 1, c = rem & 15;
            float* d = tile + (y * 64 + 2 * p + x) * 17 + c;
            d[0] = v.x, d[1] = v.y, d[2] = v.z, d[3] = v.w;
        }
    }
    __syncthreads();
    const int col = tid & 63;
    if (col >= 2 * npatch) return;
    const long colg = 2L * px0 + col;
#pragma unroll
    for (int cy = tid >> 6; cy < 32; cy += 4) {
        const int c = cy >> 1, y = cy & 1;
        float* dst = latent + c * cstride + (2L * prow + y) * width + colg;
        const float step = delta * tile[(y * 64 + col) * 17 + c];
        *dst = *dst + step;
    }
}

// ---- scratch of the guidance statistics ------------------------------------
// One CfgScratch per (device, stream): rescaling calls on different streams
// never share it.

hipError_t cfg_scratch(hipStream_t stream, CfgScratch** out) {
    return stream_scratch(kScratchCfg, stream, sizeof(CfgScratch), (void**)out);
}

hipError_t launch_stats(const float* pos, const float* neg, long count, float scale, float rescale,
                        float* out, CfgScratch* sc, hipStream_t stream) {
    const long chunks = (count + kStatChunk - 1) / kStatChunk;
    const unsigned grid = (unsigned)min(chunks, (long)kMaxStatBlocks);
    cfg_stats_kernel<<<grid, kThreads, 0, stream>>>(pos, neg, count, scale, rescale, out, sc);
    return hipGetLastError();
}

bool fits_int(long v) { return v >= 0 && v <= 0x7fffffffL; }

}  // namespace

size_t cfg_scratch_bytes() { return sizeof(CfgScratch); }

hipError_t launch_patchify(const float* tokens, int frames, int height, int width, float* patches,
                           hipStream_t stream) {
    const int pw = width / 2;
    const long prows = (long)frames * (height / 2);
    const long per_row = (long)pw * 66;
    const long bpr = (per_row + kThreads - 1) / kThreads;
    if (prows == 0 || per_row == 0) return hipSuccess;
    if (!fits_int(per_row) || !fits_int(prows * bpr)) return hipErrorInvalidValue;
    patchify_kernel<<<(unsigned)(prows * bpr), kThreads, 0, stream>>>(
        (const float2*)tokens, pw, (int)per_row, (int)bpr, (float2*)patches);
    return hipGetLastError();
}

hipError_t launch_latent_patches(const float* latent, const float* condition, long channel_stride,
                                 int frames, int height, int width, float* patches,
                                 hipStream_t stream) {
    const int pw = width / 2;
    const long prows = (long)frames * (height / 2);
    const long tpr = (pw + kTilePatches - 1) / kTilePatches;
    if (prows == 0 || pw == 0) return hipSuccess;
    if (!fits_int(prows * tpr)) return hipErrorInvalidValue;
    latent_patches_kernel<<<(unsigned)(prows * tpr), kThreads, 0, stream>>>(
        latent, condition, channel_stride, width, pw, (int)tpr, patches);
    return hipGetLastError();
}

hipError_t launch_unpatchify(const float* patches, int frames, int height, int width,
                             float* tokens, hipStream_t stream) {
    const long rows = (long)frames * height;
    const long per_row = (long)width * 4;
    const long bpr = (per_row + kThreads - 1) / kThreads;
    if (rows == 0 || per_row == 0) return hipSuccess;
    if (!fits_int(per_row) || !fits_int(rows * bpr)) return hipErrorInvalidValue;
    unpatchify_kernel<<<(unsigned)(rows * bpr), kThreads, 0, stream>>>(
        (const float4*)patches, width / 2, (int)per_row, (int)bpr, (float4*)tokens);
    return hipGetLastError();
}

hipError_t launch_timestep_embedding(const float* timesteps, int count, float* embedding,
                                     hipStream_t stream) {
    for (int s0 = 0; s0 < count; s0 += 64) {
        Timesteps ts = {};
        const int n = count - s0 < 64 ? count - s0 : 64;
        for (int i = 0; i < n; ++i) ts.t[i] = timesteps[s0 + i];
        timestep_kernel<<<n, 128, 0, stream>>>(ts, embedding + (long)s0 * 256);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_cfg(const float* pos, const float* neg, long count, float scale, float rescale,
                      float* out, hipStream_t stream) {
    if (count <= 0) return hipSuccess;
    const unsigned grid = blocks_for((count + 3) / 4, kThreads);
    if (rescale == 0.f || count < 2) {
        cfg_kernel<<<grid, kThreads, 0, stream>>>(pos, neg, count, scale, out);
        return hipGetLastError();
    }
    CfgScratch* sc = nullptr;
    hipError_t e = cfg_scratch(stream, &sc);
    if (e != hipSuccess) return e;
    e = launch_stats(pos, neg, count, scale, rescale, out, sc, stream);
    if (e != hipSuccess) return e;
    cfg_scale_kernel<<<grid, kThreads, 0, stream>>>(out, count, sc->factor);
    return hipGetLastError();
}

hipError_t launch_euler(float* latent, long channel_stride, const float* prediction, long tokens,
                        float delta, hipStream_t stream) {
    if (tokens <= 0) return hipSuccess;
    euler_kernel<<<blocks_for(tokens, kThreads), kThreads, 0, stream>>>(
        latent, channel_stride, prediction, tokens, delta);
    return hipGetLastError();
}

hipError_t launch_denoise_update(const float* pos_patches, const float* neg_patches, int frames,
                                 int height, int width, float scale, float rescale, float delta,
                                 float* latent, long channel_stride, hipStream_t stream) {
    const int pw = width / 2;
    const long prows = (long)frames * (height / 2);
    const long tpr = (pw + kTilePatches - 1) / kTilePatches;
    if (prows == 0 || pw == 0) return hipSuccess;
    if (!fits_int(prows * tpr)) return hipErrorInvalidValue;
    const float* factor = nullptr;
    const long count = prows * pw * 64;
    if (neg_patches && rescale != 0.f && count >= 2) {
        CfgScratch* sc = nullptr;
        hipError_t e = cfg_scratch(stream, &sc);
        if (e != hipSuccess) return e;
        e = launch_stats(pos_patches, neg_patches, count, scale, rescale, nullptr, sc, stream);
        if (e != hipSuccess) return e;
        factor = sc->factor;
    }
    denoise_update_kernel<<<(unsigned)(prows * tpr), kThreads, 0, stream>>>(
        pos_patches, neg_patches, scale, factor, delta, latent, channel_stride, width, pw,
        (int)tpr);
    return hipGetLastError();
}

}  // namespace s2
