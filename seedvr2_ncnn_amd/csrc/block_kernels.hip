// gfx950 kernels of the DiT block around the hot path: the norm before the
// attention and the MLP (RMSNorm without affine) with the AdaSingle
// modulation "in", and the modulation "out" with the residual sum.  The
// block graph receives the per-sample modulation vectors as its inputs
// in4..in9 (src/seedvr2/seedvr2_dit.cpp:441-448, 734-738).
//
// Both kernels are HBM-bound streams over [rows][dim].  The grid is
// persistent (as many workgroups as fit on the device at once); workgroup i
// takes the groups of four consecutive rows i, i + grid, ..., one row per
// wave, held in registers (NG float4 per lane), so each row is read from HBM
// once.  The workgroup keeps the summed modulation vectors of the sample of
// its current group's first row in LDS and refills them only when that
// sample changes (never, for one sample); a row of another sample than its
// group's first sums them from global memory.

#include <math.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

#include "block_kernels.h"
#include "s2_device.h"

#pragma clang fp contract(off)

namespace s2 {
namespace {

constexpr int kBlockRows = 4;   // rows per workgroup and group, one per wave

template <int K>
__device__ __forceinline__ void load4(const void* base, long idx, float (&v)[4]) {
    if (K == 0) {
        const float4 f = *reinterpret_cast<const float4*>((const float*)base + idx);
        v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
    } else {
        const uint2 u = *reinterpret_cast<const uint2*>((const uint16_t*)base + idx);
        const uint32_t w[2] = {u.x, u.y};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint16_t h = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
            v[e] = K == 1 ? __uint_as_float((uint32_t)h << 16)
                          : (float)__builtin_bit_cast(_Float16, h);
        }
    }
}

// a + b (b null: a) for 4 consecutive values
__device__ __forceinline__ float4 sum4(const float* a, const float* b, int c) {
    const float4 x = *reinterpret_cast<const float4*>(a + c);
    if (!b) return x;
    const float4 y = *reinterpret_cast<const float4*>(b + c);
    return make_float4(x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w);
}

// stream (0 video, 1 text), row within the stream and sample of global row r
__device__ __forceinline__ void locate(const AdaRows& rows, int r, int& stream, int& local,
                                       int& sample) {
    stream = r >= rows.video_rows;
    local = stream ? r - rows.video_rows : r;
    const int* end = rows.end + stream * kAdaMaxBatch;
    int b = 0;
    while (b + 1 < rows.batch && local >= end[b]) ++b;
    sample = b;
}

// shared memory of a workgroup: up to three summed vectors of kAdaMaxDim
extern __shared__ float4 ada_lds[];

// Writes norm(v) * sc + sh of the row held in v (NG float4 per lane) to row
// `oo` of o (element type ok).  sc / sh come from LDS when `home`, else are
// summed from the sample's vectors.
template <int NG>
__device__ __forceinline__ void norm_modulate(const float (&v)[NG][4], int lane, int dim, float eps,
                                              bool home, const float4* lsc, const float4* lsh,
                                              const float* sca, const float* scb, const float* sha,
                                              const float* shb, void* o, long oo, int ok) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NG; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) ss += v[i][e] * v[i][e];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    const float rs = 1.0f / sqrtf(ss / (float)dim + eps);
#pragma unroll
    for (int i = 0; i < NG; ++i) {
        const int c = (i * 64 + lane) * 4;
        if (c >= dim) break;
        float4 sc4, sh4;
        if (home) {
            sc4 = lsc[c / 4];
            sh4 = lsh[c / 4];
        } else {
            sc4 = sum4(sca, scb, c);
            sh4 = sum4(sha, shb, c);
        }
        const float sc[4] = {sc4.x, sc4.y, sc4.z, sc4.w};
        const float sh[4] = {sh4.x, sh4.y, sh4.z, sh4.w};
        float r[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float n = v[i][e] * rs;
            const float m = n * sc[e];
            r[e] = m + sh[e];
        }
        store4(o, oo + c, r[0], r[1], r[2], r[3], ok);
    }
}

// the value an element of type K stores for x
template <int K>
__device__ __forceinline__ float stored(float x) {
    if (K == 1) return bf16_to_f32(f32_to_bf16(x));
    if (K == 2) return (float)f32_to_f16(x);
    return x;
}

template <int NG, int XK, int OK>
__global__ __launch_bounds__(256) void ada_in_kernel(AdaInArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int total = a.rows.video_rows + a.rows.text_rows;
    const int groups = (total + kBlockRows - 1) / kBlockRows;
    const int g4 = a.dim / 4;
    float4* lsc = ada_lds;
    float4* lsh = ada_lds + g4;
    int cur = -1;   // (stream, sample) of the vectors in LDS
    for (int grp = blockIdx.x; grp < groups; grp += gridDim.x) {
        int hs, hl, hb;
        locate(a.rows, grp * kBlockRows, hs, hl, hb);
        if (hs * kAdaMaxBatch + hb != cur) {   // uniform over the workgroup
            cur = hs * kAdaMaxBatch + hb;
            __syncthreads();   // the old vectors are no longer read
            for (int i = threadIdx.x; i < g4; i += 256) {
                lsc[i] = sum4(a.scale_a + (long)hb * a.dim, a.scale_b[hs], 4 * i);
                lsh[i] = sum4(a.shift_a + (long)hb * a.dim, a.shift_b[hs], 4 * i);
            }
            __syncthreads();
        }
        const int r = grp * kBlockRows + wave;
        if (r >= total) continue;
        int stream, local, b;
        locate(a.rows, r, stream, local, b);
        const bool home = stream == hs && b == hb;
        const void* xr = stream ? a.x[1] : a.x[0];
        const long xo = (long)local * a.x_stride;
        float v[NG][4];
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            const int c = (i * 64 + lane) * 4;
            if (c < a.dim) {
                load4<XK>(xr, xo + c, v[i]);
            } else {
                v[i][0] = v[i][1] = v[i][2] = v[i][3] = 0.f;
            }
        }
        norm_modulate<NG>(v, lane, a.dim, a.eps, home, lsc, lsh, a.scale_a + (long)b * a.dim,
                          a.scale_b[stream], a.shift_a + (long)b * a.dim, a.shift_b[stream],
                          stream ? a.out[1] : a.out[0], (long)local * a.out_stride, OK);
    }
}

template <int NG, int XK, int YK, bool NORM>
__global__ __launch_bounds__(256) void ada_out_kernel(AdaOutArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int total = a.rows.video_rows + a.rows.text_rows;
    const int groups = (total + kBlockRows - 1) / kBlockRows;
    const int g4 = a.dim / 4;
    float4* lgt = ada_lds;
    float4* lsc = ada_lds + g4;
    float4* lsh = ada_lds + 2 * g4;
    int cur = -1;
    for (int grp = blockIdx.x; grp < groups; grp += gridDim.x) {
        int hs, hl, hb;
        locate(a.rows, grp * kBlockRows, hs, hl, hb);
        if (hs * kAdaMaxBatch + hb != cur) {   // uniform over the workgroup
            cur = hs * kAdaMaxBatch + hb;
            __syncthreads();
            for (int i = threadIdx.x; i < g4; i += 256) {
                lgt[i] = sum4(a.gate_a + (long)hb * a.dim, a.gate_b[hs], 4 * i);
                if (NORM) {
                    lsc[i] = sum4(a.scale_a + (long)hb * a.dim, a.scale_b[hs], 4 * i);
                    lsh[i] = sum4(a.shift_a + (long)hb * a.dim, a.shift_b[hs], 4 * i);
                }
            }
            __syncthreads();
        }
        const int r = grp * kBlockRows + wave;
        if (r >= total) continue;
        int stream, local, b;
        locate(a.rows, r, stream, local, b);
        const bool home = stream == hs && b == hb;
        const void* xr = stream ? a.x[1] : a.x[0];
        const void* yr = stream ? a.y[1] : a.y[0];
        void* orow = stream ? a.out[1] : a.out[0];
        const long xo = (long)local * a.x_stride, yo = (long)local * a.y_stride;
        const long oo = (long)local * a.out_stride;
        float xv[NG][4], yv[NG][4];
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            const int c = (i * 64 + lane) * 4;
            if (c < a.dim) {
                load4<XK>(xr, xo + c, xv[i]);
                load4<YK>(yr, yo + c, yv[i]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) xv[i][e] = yv[i][e] = 0.f;
            }
        }
#pragma unroll
        for (int i = 0; i < NG; ++i) {
            const int c = (i * 64 + lane) * 4;
            if (c >= a.dim) break;
            const float4 g4v = home ? lgt[c / 4]
                                    : sum4(a.gate_a + (long)b * a.dim, a.gate_b[stream], c);
            const float g[4] = {g4v.x, g4v.y, g4v.z, g4v.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float p = yv[i][e] * g[e];
                xv[i][e] = xv[i][e] + p;
            }
            store4(orow, oo + c, xv[i][0], xv[i][1], xv[i][2], xv[i][3], XK);
            if (NORM) {
                // the norm reads the residual as stored
#pragma unroll
                for (int e = 0; e < 4; ++e) xv[i][e] = stored<XK>(xv[i][e]);
            }
        }
        if (NORM)
            norm_modulate<NG>(xv, lane, a.dim, a.eps, home, lsc, lsh, a.scale_a + (long)b * a.dim,
                              a.scale_b[stream], a.shift_a + (long)b * a.dim, a.shift_b[stream],
                              stream ? a.h[1] : a.h[0], (long)local * a.h_stride, a.h_kind);
    }
}

// Workgroups of a persistent launch of `func`: as many as fit on the device
// at once (the occupancy of that kernel at `lds` bytes, per device), at most
// one per group of rows.
unsigned persistent_grid(const void* func, size_t lds, const AdaRows& r) {
    static std::mutex mu;
    static std::map<std::pair<int, std::pair<const void*, size_t>>, int> cache;
    const long groups = ((long)r.video_rows + r.text_rows + kBlockRows - 1) / kBlockRows;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return (unsigned)groups;
    int slots = 0;
    {
        std::lock_guard<std::mutex> lock(mu);
        const auto key = std::make_pair(dev, std::make_pair(func, lds));
        auto it = cache.find(key);
        if (it != cache.end()) {
            slots = it->second;
        } else {
            int per_cu = 0, cus = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, func, 256, lds) !=
                    hipSuccess ||
                hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                    hipSuccess)
                return (unsigned)groups;
            slots = std::max(1, per_cu) * std::max(1, cus);
            cache[key] = slots;
        }
    }
    return (unsigned)std::min<long>(groups, slots);
}

// float4 groups per lane for a row of `dim` values
int ada_groups(int dim) {
    const int g = (dim + 255) / 256;
    return g <= 4 ? 4 : g <= 8 ? 8 : g <= 10 ? 10 : g <= 12 ? 12 : 16;
}

template <int NG, int XK, int OK>
void ada_in_launch(const AdaInArgs& a, hipStream_t stream) {
    const size_t lds = 2 * (size_t)a.dim * sizeof(float);
    const void* f = reinterpret_cast<const void*>(&ada_in_kernel<NG, XK, OK>);
    ada_in_kernel<NG, XK, OK><<<persistent_grid(f, lds, a.rows), 256, lds, stream>>>(a);
}

template <int NG, int XK>
void ada_in_launch(const AdaInArgs& a, hipStream_t stream) {
    if (a.out_kind == 1)
        ada_in_launch<NG, XK, 1>(a, stream);
    else if (a.out_kind == 2)
        ada_in_launch<NG, XK, 2>(a, stream);
    else
        ada_in_launch<NG, XK, 0>(a, stream);
}

template <int NG>
void ada_in_x_kind(const AdaInArgs& a, hipStream_t stream) {
    if (a.x_kind == 1)
        ada_in_launch<NG, 1>(a, stream);
    else if (a.x_kind == 2)
        ada_in_launch<NG, 2>(a, stream);
    else
        ada_in_launch<NG, 0>(a, stream);
}

template <int NG, int XK, int YK, bool NORM>
void ada_out_launch(const AdaOutArgs& a, hipStream_t stream) {
    const size_t lds = (NORM ? 3 : 1) * (size_t)a.dim * sizeof(float);
    const void* f = reinterpret_cast<const void*>(&ada_out_kernel<NG, XK, YK, NORM>);
    ada_out_kernel<NG, XK, YK, NORM><<<persistent_grid(f, lds, a.rows), 256, lds, stream>>>(a);
}

template <int NG, int XK, bool NORM>
void ada_out_launch(const AdaOutArgs& a, hipStream_t stream) {
    if (a.y_kind == 1)
        ada_out_launch<NG, XK, 1, NORM>(a, stream);
    else if (a.y_kind == 2)
        ada_out_launch<NG, XK, 2, NORM>(a, stream);
    else
        ada_out_launch<NG, XK, 0, NORM>(a, stream);
}

template <int NG, int XK>
void ada_out_launch(const AdaOutArgs& a, hipStream_t stream) {
    if (a.norm)
        ada_out_launch<NG, XK, true>(a, stream);
    else
        ada_out_launch<NG, XK, false>(a, stream);
}

template <int NG>
void ada_out_x_kind(const AdaOutArgs& a, hipStream_t stream) {
    if (a.x_kind == 1)
        ada_out_launch<NG, 1>(a, stream);
    else if (a.x_kind == 2)
        ada_out_launch<NG, 2>(a, stream);
    else
        ada_out_launch<NG, 0>(a, stream);
}

bool ada_shape_ok(int dim, const AdaRows& r) {
    return dim > 0 && dim % 4 == 0 && dim <= kAdaMaxDim && r.batch > 0 &&
           r.batch <= kAdaMaxBatch && r.video_rows >= 0 && r.text_rows >= 0;
}

}  // namespace

hipError_t launch_ada_in(const AdaInArgs& a, hipStream_t stream) {
    if (!ada_shape_ok(a.dim, a.rows)) return hipErrorInvalidValue;
    if (a.rows.video_rows + a.rows.text_rows == 0) return hipSuccess;
    switch (ada_groups(a.dim)) {
        case 4: ada_in_x_kind<4>(a, stream); break;
        case 8: ada_in_x_kind<8>(a, stream); break;
        case 10: ada_in_x_kind<10>(a, stream); break;
        case 12: ada_in_x_kind<12>(a, stream); break;
        default: ada_in_x_kind<16>(a, stream); break;
    }
    return hipGetLastError();
}

hipError_t launch_ada_out(const AdaOutArgs& a, hipStream_t stream) {
    if (!ada_shape_ok(a.dim, a.rows)) return hipErrorInvalidValue;
    if (a.rows.video_rows + a.rows.text_rows == 0) return hipSuccess;
    switch (ada_groups(a.dim)) {
        case 4: ada_out_x_kind<4>(a, stream); break;
        case 8: ada_out_x_kind<8>(a, stream); break;
        case 10: ada_out_x_kind<10>(a, stream); break;
        case 12: ada_out_x_kind<12>(a, stream); break;
        default: ada_out_x_kind<16>(a, stream); break;
    }
    return hipGetLastError();
}

}  // namespace s2
