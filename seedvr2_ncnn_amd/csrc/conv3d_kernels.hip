// gfx950 kernels of DecomposedConv3D (src/seedvr2/decomposed_conv3d.cpp:605-755):
// a causal 3-D convolution whose temporal prefix is either head_frames
// copies of the first frame or the cached last frames of the previous slice.
//
// The reference gathers one input frame per temporal tap, runs an ncnn 2-D
// Convolution on it and adds the frame results.  Here the whole
// kt x kh x kw window is one implicit GEMM on the matrix cores:
//   rows    M = output pixels (t, y, x) of the launch,
//   columns N = output channels,
//   depth   K = (tap, ky, kx, ci), ci fastest,
// A[m][k] = staged[frame(t, tap)][y*sh + ky*dh - ph][x*sw + kx*dw - pw][ci]
// (zero outside the image), B[n][k] = packed weights.  The staged input is
// channel-last bf16, so for one window position the 64 channels of a k-step
// are one 128-byte run of a pixel: the A tile streams into LDS with the
// same buffer_load ... lds DMA as the SharedLinear GEMM, each row from its
// own pixel, and a row whose pixel falls in the zero padding gets an offset
// past the end of the buffer, which the hardware returns as zeros.
#include <limits.h>

#include "conv3d_kernels.h"
#include "s2_device.h"
#include "stream_scratch.h"

namespace s2 {
namespace {

constexpr int kStageThreads = 256;

__device__ __forceinline__ int lds_swizzle(int r) { return ((r >> 1) ^ ((r & 1) << 2)) & 7; }

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// ---- staging: planar -> channel-last bf16 ------------------------------------

template <int KIND>
__device__ __forceinline__ float load_elem(const void* p, long i) {
    if (KIND == 1) return __builtin_bit_cast(float, (uint32_t)((const uint16_t*)p)[i] << 16);
    if (KIND == 2) return (float)((const _Float16*)p)[i];
    return ((const float*)p)[i];
}

// One block moves P pixels x 64 channels (P = 128; 64 for layers of at most
// 32 input channels, whose blocks have few channel rows to read).  Lane l of
// a load reads 16 bytes (8 elements of a 16-bit blob, 4 of an fp32 one;
// single elements when the rows are not 16-byte aligned, `vec` false) of
// channel l at one run of pixels, and writes them to an LDS tile stored
// pixel-major ([pixel][68 floats]: consecutive lanes, consecutive words);
// a pixel's 8-channel parts then come out as two 16-byte LDS reads and leave
// as one 16-byte store, 8 consecutive threads covering a 128-byte channel run
// (cpad channels when cpad is 8, 16 or 32).  Channels at or above cin are
// written as zeros.
template <int KIND, int P>
__global__ __launch_bounds__(kStageThreads) void conv3d_stage_kernel(
    const void* __restrict__ in, long cstep, int cin, long pixels, int cpad, int vec,
    uint16_t* __restrict__ staged, uint16_t* __restrict__ tail, long tail_q0) {
    static_assert(P == 128 || P == 64, "pixels per block");
    constexpr int PITCH = 68;                 // floats per pixel row (16-byte multiple)
    constexpr int EL = KIND == 0 ? 4 : 8;     // elements per 16-byte load
    __shared__ __attribute__((aligned(16))) float tile[P * PITCH];
    const long q0 = (long)blockIdx.x * P;
    const int c0 = blockIdx.y * 64;
    const int t = threadIdx.x;
    const bool full = vec && q0 + P <= pixels;
#pragma unroll
    for (int i = 0; i < 64 * (P / EL) / kStageThreads; ++i) {
        const int item = i * kStageThreads + t;
        const int cl = item & 63;
        const int qe = (item >> 6) * EL;
        const int c = c0 + cl;
        float v[EL];
#pragma unroll
        for (int e = 0; e < EL; ++e) v[e] = 0.f;
        if (c < cin) {
            const long base = (long)c * cstep + q0 + qe;
            if (full) {
                if (KIND == 0) {
                    const float4 f = *reinterpret_cast<const float4*>((const float*)in + base);
                    v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
                } else {
                    const uint4 u = *reinterpret_cast<const uint4*>((const uint16_t*)in + base);
                    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                    for (int e = 0; e < EL; ++e) {
                        const uint16_t h = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
                        v[e] = KIND == 1 ? __uint_as_float((uint32_t)h << 16)
                                         : (float)__builtin_bit_cast(_Float16, h);
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < EL; ++e)
                    if (q0 + qe + e < pixels) v[e] = load_elem<KIND>(in, base + e);
            }
        }
#pragma unroll
        for (int e = 0; e < EL; ++e) tile[(qe + e) * PITCH + cl] = v[e];
    }
    __syncthreads();
    // a pixel holds cpad channels: with cpad 8, 16 or 32 only the first
    // cpad / 8 parts of 8 channels are written
    const int parts = min(8, (cpad - c0) / 8);
#pragma unroll
    for (int i = 0; i < P * 8 / kStageThreads; ++i) {
        const int idx = i * kStageThreads + t;
        const int q = idx >> 3, part = idx & 7;
        if (part >= parts || q0 + q >= pixels) continue;
        const float4 lo = *reinterpret_cast<const float4*>(&tile[q * PITCH + part * 8]);
        const float4 hi = *reinterpret_cast<const float4*>(&tile[q * PITCH + part * 8 + 4]);
        const uint4 val = make_uint4(pack2_bf16_rne(lo.x, lo.y), pack2_bf16_rne(lo.z, lo.w),
                                     pack2_bf16_rne(hi.x, hi.y), pack2_bf16_rne(hi.z, hi.w));
        *reinterpret_cast<uint4*>(staged + (q0 + q) * cpad + c0 + part * 8) = val;
        // pixels from tail_q0 on are the next temporal memory as well
        if (tail && q0 + q >= tail_q0)
            *reinterpret_cast<uint4*>(tail + (q0 + q - tail_q0) * cpad + c0 + part * 8) = val;
    }
}

// Staging for at least 64 channel slots (cpad a multiple of 64) and 16-byte
// aligned channel rows, without LDS: a thread loads 8 pixels of 8 channels
// (one 16-byte run per channel, two for fp32), transposes them in registers
// and stores 8 pixels' 16-byte channel runs.  Eight consecutive lanes hold the
// eight channel groups of a 64-channel block for one pixel run, the next
// eight lanes the next run: a load instruction reads 128 contiguous bytes of
// each of 8 channel rows, a store instruction writes 128 contiguous bytes
// (the block's 64 channels) of each of 8 pixels.  A block covers 256 pixels
// of 64 channels; pixels past the end are not written, channels at and above
// cin are written as zeros.
template <int KIND>
__global__ __launch_bounds__(256) void conv3d_stage_t_kernel(
    const void* __restrict__ in, long cstep, int cin, long pixels, int cpad,
    uint16_t* __restrict__ staged, uint16_t* __restrict__ tail, long tail_q0) {
    const int t = threadIdx.x;
    const int h = (t & 7);                // channel group within the block
    const int g = (t >> 3) & 31;          // pixel run within the block
    const long q = (long)blockIdx.x * 256 + 8 * g;
    const int c0 = blockIdx.y * 64 + 8 * h;
    if (q >= pixels) return;
    const bool full = q + 8 <= pixels;
    uint32_t w[8][4];   // channel i, pixel pair d (bf16 pairs)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int c = c0 + i;
        uint32_t v[4] = {0u, 0u, 0u, 0u};
        if (c < cin) {
            const long base = (long)c * cstep + q;
            if (KIND == 0) {
                float f[8];
                if (full) {
                    const float4 a = *reinterpret_cast<const float4*>((const float*)in + base);
                    const float4 b = *reinterpret_cast<const float4*>((const float*)in + base + 4);
                    f[0] = a.x, f[1] = a.y, f[2] = a.z, f[3] = a.w;
                    f[4] = b.x, f[5] = b.y, f[6] = b.z, f[7] = b.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) f[e] = q + e < pixels ? ((const float*)in)[base + e] : 0.f;
                }
#pragma unroll
                for (int d = 0; d < 4; ++d) v[d] = pack2_bf16_rne(f[2 * d], f[2 * d + 1]);
            } else {
                uint4 u = make_uint4(0, 0, 0, 0);
                if (full) {
                    u = *reinterpret_cast<const uint4*>((const uint16_t*)in + base);
                } else {
                    uint16_t e16[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) e16[e] = q + e < pixels ? ((const uint16_t*)in)[base + e] : 0;
                    u = make_uint4(e16[0] | (e16[1] << 16), e16[2] | (e16[3] << 16),
                                   e16[4] | (e16[5] << 16), e16[6] | (e16[7] << 16));
                }
                const uint32_t r[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    if (KIND == 2)
                        v[d] = pack2_bf16_rne((float)__builtin_bit_cast(_Float16, (uint16_t)(r[d] & 0xffffu)),
                                              (float)__builtin_bit_cast(_Float16, (uint16_t)(r[d] >> 16)));
                    else
                        v[d] = r[d];
                }
            }
        }
#pragma unroll
        for (int d = 0; d < 4; ++d) w[i][d] = v[d];
    }
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        if (!full && q + p >= pixels) break;
        uint32_t o[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t lo = w[2 * d][p >> 1], hi = w[2 * d + 1][p >> 1];
            o[d] = (p & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
        }
        const uint4 val = make_uint4(o[0], o[1], o[2], o[3]);
        *reinterpret_cast<uint4*>(staged + (q + p) * cpad + c0) = val;
        // pixels from tail_q0 on are the next temporal memory as well
        if (tail && q + p >= tail_q0)
            *reinterpret_cast<uint4*>(tail + (q + p - tail_q0) * cpad + c0) = val;
    }
}

// ---- weights: [kt][cout][cin][kh][kw] fp32 -> [cout][kp] bf16 ----------------

// row co of the packed weights: k = p * cpad + ci for window position p =
// (tap * kh + ky) * kw + kx, zero past the last position and for ci >= cin
__global__ __launch_bounds__(256) void conv3d_pack_kernel(const float* __restrict__ w,
                                                          Conv3dShape s, long kp, long total,
                                                          uint16_t* __restrict__ out) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int co = (int)(i / kp);
    const long k = i - (long)co * kp;
    const int p = (int)(k / s.cpad), ci = (int)(k - (long)p * s.cpad);
    float v = 0.f;
    if (p < s.kt * s.kh * s.kw && ci < s.cin) {
        const int kx = p % s.kw, r = p / s.kw;
        const int ky = r % s.kh, tap = r / s.kh;
        v = w[(((long)tap * s.cout + co) * s.cin + ci) * s.kh * s.kw + ky * s.kw + kx];
    }
    out[i] = f32_to_bf16(v);
}

// ---- the implicit GEMM ---------------------------------------------------------

struct ConvArgs {
    const uint16_t* staged;   // input frames fbase.. (staged layout)
    uint32_t staged_bytes;
    const uint16_t* memory;   // memory frames 0..mem-1 (staged layout)
    uint32_t memory_bytes;
    int mem;
    const uint16_t* packed;
    int kp;   // packed row length (conv3d_kp)
    const float* bias;
    void* out;
    long out_cstep;
    long out_off;
    int out_kind;
    int vec_ok;   // 4-pixel vector stores are aligned
    int H, W, Ho, Wo, M;
    int cpad, cout;
    int kt, kh, kw, st, dt, sh, sw, dh, dw, ph, pw;
    int shift, fbase, t0;
    int mtiles, ntiles;
    int ytiles, xtiles;   // halo kernel: output tiles per frame
    // k loop split into `splits` ranges of whole k-steps: workgroup row
    // blockIdx.y takes range blockIdx.y and stores its raw fp32 tile to part +
    // blockIdx.y * part_split (planar [cout][M]); null: the whole loop,
    // normal epilogue
    float* part;
    long part_split;
    int splits;
    // conv3d_pp_kernel with a split k loop: one 256x256 fp32 slot per
    // (tile, range) workgroup and one arrival counter per tile (zero between
    // launches); the last range of a tile to arrive sums the slots and runs
    // the normal epilogue, so no second pass reads part.  null: part.
    float* slots;
    int* counters;
};

// Epilogue of a TM x TN grid of 32x32 accumulators whose first row is GEMM
// row r0 and first column output channel c0: register r of an accumulator
// is row 8(r/4) + 4g + r%4, column l32, so each lane holds 4 consecutive
// output pixels of one output channel: one 16-byte (fp32) or 8-byte store
// into that plane.  part: the raw fp32 partial tile of k range blockIdx.y
// goes to part + blockIdx.y * part_split (planar [cout][M]) instead.
template <int TM, int TN, int OK>
__device__ __forceinline__ void conv3d_epilogue(const ConvArgs& a, const f32x16 (&acc)[TM][TN],
                                                int r0, int c0, int l32, int g, float* part) {
    if (part) {
        float* pp = part + (long)blockIdx.y * a.part_split;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = c0 + 32 * j + l32;
            if (col >= a.cout) continue;
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int rg = 0; rg < 4; ++rg) {
                    const int m = r0 + 32 * i + 8 * rg + 4 * g;
                    const long idx = (long)col * a.M + m;
                    if ((a.M & 3) == 0 && m + 3 < a.M) {
                        // m and M multiples of 4: a 16-byte aligned run
                        *reinterpret_cast<float4*>(pp + idx) =
                            make_float4(acc[i][j][4 * rg], acc[i][j][4 * rg + 1],
                                        acc[i][j][4 * rg + 2], acc[i][j][4 * rg + 3]);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (m + e < a.M) pp[idx + e] = acc[i][j][4 * rg + e];
                    }
                }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col = c0 + 32 * j + l32;
        if (col >= a.cout) continue;
        const float bv = a.bias ? a.bias[col] : 0.f;
        const long cbase = (long)col * a.out_cstep + a.out_off;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                const int m = r0 + 32 * i + 8 * rg + 4 * g;
                const float v0 = acc[i][j][4 * rg] + bv, v1 = acc[i][j][4 * rg + 1] + bv;
                const float v2 = acc[i][j][4 * rg + 2] + bv, v3 = acc[i][j][4 * rg + 3] + bv;
                if (a.vec_ok && m + 3 < a.M) {
                    store4(a.out, cbase + m, v0, v1, v2, v3, OK);
                } else {
                    const float v[4] = {v0, v1, v2, v3};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (m + e >= a.M) continue;
                        const long idx = cbase + m + e;
                        if (OK == 1)
                            ((uint16_t*)a.out)[idx] = f32_to_bf16(v[e]);
                        else if (OK == 2)
                            ((_Float16*)a.out)[idx] = f32_to_f16(v[e]);
                        else
                            ((float*)a.out)[idx] = v[e];
                    }
                }
            }
    }
}

// Eight waves in a grid of 128x64 wave tiles (4x2 MFMA 32x32x16
// accumulators, 128 fp32 per lane), as in the SharedLinear GEMM: BN = 256
// gives 256x256 block tiles, BN = 128 (output channels <= 128) 512x128
// tiles.  BN = 32 (output channels <= 32, e.g. a decoder's RGB output) uses
// 64x32 wave tiles in a 512x32 block, so a 3-channel output pays for 32
// columns, not 128.  Two 64-k LDS stages of (BM + BN) x 128 bytes are filled
// by DMA one stage ahead of the MFMAs; LDS rows use the GEMM's chunk swizzle.
// Wave w loads A rows [w*BM/8, (w+1)*BM/8) and its share of the B rows, 8
// rows per DMA instruction.  OK is the output type (0 fp32, 1 bf16, 2 fp16).
//
// The im2col addressing costs a few VALU operations per row and window
// position: each A row keeps the byte offset of its window origin
// (rpix), a bit mask of the (ky, kx) positions that fall inside the image
// (rmask), and the offset of its current temporal tap's frame (rbase,
// refreshed when the tap changes).  A position then adds one scalar offset.
// The k-steps walk (tap, ky, kx, channel chunk) with scalar counters.
//
// SMALL (at most 32 input channels, cpad = 8, 16 or 32): a 64-wide k-step
// spans 64 / cpad window positions of cpad channels.  Wave w then loads
// 16-byte chunk w of every A row (one window position and channel part per
// wave, decoded with scalar arithmetic), into a chunk-major A tile
// [8 chunks][BM rows] of 16 bytes; row r of a DMA instruction is lane r.
template <int BN, int OK, bool SMALL>
__global__ __launch_bounds__(512, 1) void conv3d_kernel(ConvArgs a) {
    // wave tile: TM x TN blocks of 32x32 (128x64, or 64x32 for BN = 32)
    constexpr int TM = BN >= 64 ? 4 : 2, TN = BN >= 64 ? 2 : 1;
    constexpr int WN = BN / (32 * TN), WM = 8 / WN;
    constexpr int BM = WM * 32 * TM;
    constexpr int BK = 64, RB = BK * 2;
    constexpr int TA = BM * RB, SB = TA + BN * RB;
    constexpr int ARPW = BM / 8, AJ = ARPW / 8;
    // B rows: BN / 8 per wave in 8-row DMA instructions; with BN = 32 the
    // first four waves load 8 rows each
    constexpr int BRPW = BN >= 64 ? BN / 8 : 8, BJ = BN >= 64 ? BRPW / 8 : 1;
    constexpr int BWAVES = BN / BRPW;
    constexpr int GROUP = 4;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * SB];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // the wave index is uniform; saying so keeps the DMA's LDS addresses in SGPRs
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int g = lane >> 5;
    const int wm = wave / WN;
    const int wn = wave % WN;
    const int sw = lds_swizzle(l32);
    const uint32_t lds_base = (uint32_t)(uintptr_t)lds;

    // grouped, XCD-aware raster: GROUP m-tiles share each sweep over the n-tiles
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int group_size = GROUP * a.ntiles;
    const int first_m = (lid / group_size) * GROUP;
    const int gm = min(a.mtiles - first_m, GROUP);
    const int mt = first_m + (lid % group_size) % gm;
    const int nt = (lid % group_size) / gm;
    const int row0 = mt * BM;
    const int col0 = nt * BN;

    const uint32_t pix = (uint32_t)(a.cpad * 2);
    const uint32_t frame_bytes = (uint32_t)(a.H * a.W) * pix;
    // A rows of this lane: padded frame of tap 0 (negative past M), window
    // origin offset (mod 2^32: the origin may lie in the padding), and mask
    const int hw = a.Ho * a.Wo;
    int rpf[AJ];
    uint32_t rpix[AJ], rmask[AJ];
#pragma unroll
    for (int j = 0; j < AJ; ++j) {
        const int row = SMALL ? j * 64 + lane : wave * ARPW + j * 8 + (lane >> 3);
        const int m = row0 + row;
        const uint32_t chk = SMALL ? 0u : (uint32_t)(((lane & 7) ^ lds_swizzle(row)) * 16);
        rpf[j] = INT_MIN / 2;
        rpix[j] = chk;
        rmask[j] = 0;
        if (m < a.M) {
            const int to = m / hw;
            const int rem = m - to * hw;
            const int yo = rem / a.Wo;
            const int xo = rem - yo * a.Wo;
            const int yb = yo * a.sh - a.ph, xb = xo * a.sw - a.pw;
            rpf[j] = (a.t0 + to) * a.st;
            rpix[j] = (uint32_t)(yb * a.W + xb) * pix + chk;
            uint32_t mk = 0;
            for (int ky = 0; ky < a.kh; ++ky) {
                if ((unsigned)(yb + ky * a.dh) >= (unsigned)a.H) continue;
                for (int kx = 0; kx < a.kw; ++kx)
                    if ((unsigned)(xb + kx * a.dw) < (unsigned)a.W) mk |= 1u << (ky * a.kw + kx);
            }
            rmask[j] = mk;
        }
    }
    uint32_t voffb[BJ];
#pragma unroll
    for (int j = 0; j < BJ; ++j) {
        const int row = (wave % BWAVES) * BRPW + j * 8 + (lane >> 3);
        voffb[j] = (uint32_t)(row * a.kp * 2 + (((lane & 7) ^ lds_swizzle(row)) * 16));
    }
    const i32x4 ra = wave_uniform(buffer_rsrc(a.staged, a.staged_bytes));
    const i32x4 rm = wave_uniform(buffer_rsrc(a.memory, a.memory_bytes));
    const i32x4 rb = wave_uniform(buffer_rsrc(
        a.packed + (long)col0 * a.kp, (uint32_t)(min(a.cout - col0, BN) * a.kp * 2)));

    // Temporal tap: padded frame p is frame v = max(p - shift, 0) of
    // [memory | input]; v < mem reads the memory buffer, otherwise input
    // frame v - mem of the staged buffer (based at input frame fbase).  The 8
    // rows of one DMA instruction lie in one output frame (the host passes
    // mem > 0 only when Ho*Wo % 8 == 0), so the buffer is the same for all.
    uint32_t rbase[AJ];
    int memsel[AJ];
    auto set_tap = [&](int tap) {
        const int dtap = tap * a.dt - a.shift;
#pragma unroll
        for (int j = 0; j < AJ; ++j) {
            const int v = max(rpf[j] + dtap, 0);
            const bool fm = v < a.mem;
            const int sf = fm ? v : v - a.mem - a.fbase;
            rbase[j] = (uint32_t)sf * frame_bytes + rpix[j];
            memsel[j] = __builtin_amdgcn_readfirstlane((int)fm);
        }
    };
    uint32_t voffa[AJ];
    auto set_pos = [&](int ky, int kx) {
        const uint32_t koff = (uint32_t)(ky * a.dh * a.W + kx * a.dw) * pix;
        const uint32_t bit = 1u << (ky * a.kw + kx);
#pragma unroll
        for (int j = 0; j < AJ; ++j) voffa[j] = (rmask[j] & bit) ? rbase[j] + koff : 0x80000000u;
    };
    const int cpc = SMALL ? 1 : a.cpad / 64;   // k-steps per window position
    // k-steps [kbase, kbase + nk) of the loop (all of them unless split)
    int kbase = 0, nk = a.kp / 64;
    if (!SMALL && a.part) {
        const int all = a.kt * a.kh * a.kw * cpc;
        kbase = (int)((long)blockIdx.y * all / a.splits);
        nk = (int)((long)(blockIdx.y + 1) * all / a.splits) - kbase;
    }
    // SMALL: this wave's 16-byte part of a pixel and window position within
    // a k-step; the position of k-step ks is ks * (64 / cpad) + its index
    const int parts = a.cpad / 8;
    const int my_part = wave % parts, my_pos = wave / parts;
    const int npos = a.kt * a.kh * a.kw;
    int cur_tap = -1;
    auto set_step_small = [&](int ks) {
        const int p = ks * (8 / parts) + my_pos;
        if (p >= npos) {
#pragma unroll
            for (int j = 0; j < AJ; ++j) voffa[j] = 0x80000000u;
            return;
        }
        const int khw = a.kh * a.kw;
        const int tap = p / khw, r = p - tap * khw;
        const int ky = r / a.kw, kx = r - ky * a.kw;
        if (tap != cur_tap) {
            set_tap(tap);
            cur_tap = tap;
        }
        const uint32_t koff = (uint32_t)(ky * a.dh * a.W + kx * a.dw) * pix + my_part * 16;
        const uint32_t bit = 1u << r;
#pragma unroll
        for (int j = 0; j < AJ; ++j) voffa[j] = (rmask[j] & bit) ? rbase[j] + koff : 0x80000000u;
    };
    auto issue = [&](int stage, int ks, int cc) {
        const uint32_t soffa = (uint32_t)(cc * RB);
        const uint32_t soffb = (uint32_t)((ks + kbase) * RB);
        const uint32_t st = lds_base + stage * SB;
        if (SMALL) {
#pragma unroll
            for (int j = 0; j < AJ; ++j)
                lds_dma16(ra, st + (wave * BM + j * 64) * 16, voffa[j], 0u);
        } else {
#pragma unroll
            for (int j = 0; j < AJ; ++j)
                lds_dma16(memsel[j] ? rm : ra, st + (wave * ARPW + j * 8) * RB, voffa[j], soffa);
        }
        if (wave < BWAVES) {
#pragma unroll
            for (int j = 0; j < BJ; ++j)
                lds_dma16(rb, st + TA + (wave * BRPW + j * 8) * RB, voffb[j], soffb);
        }
    };

    f32x16 acc[TM][TN];
    bf16x8 fa[2][TM], fb[2][TN];
    auto frag = [&](const uint8_t* st, int kk, int slot) {
        const int pc = ((2 * kk + g) ^ sw) * 16;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int row = wm * 32 * TM + 32 * i + l32;
            fa[slot][i] = as_bf16x8(*(const uint4*)(
                SMALL ? st + ((2 * kk + g) * BM + row) * 16 : st + row * RB + pc));
        }
#pragma unroll
        for (int j = 0; j < TN; ++j)
            fb[slot][j] = as_bf16x8(*(const uint4*)(st + TA + (wn * 32 * TN + 32 * j + l32) * RB + pc));
    };
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // window position and channel chunk of the next k-step to issue
    int cc = kbase % cpc, kx = (kbase / cpc) % a.kw, ky = (kbase / cpc / a.kw) % a.kh;
    int tap = kbase / cpc / a.kw / a.kh;
    if (SMALL) {
        set_step_small(0);
    } else {
        set_tap(tap);
        set_pos(ky, kx);
    }
    issue(0, 0, cc);
#pragma unroll 1
    for (int ks = 0; ks < nk; ++ks) {
        const int stage = ks & 1;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();   // stage ks visible to all waves; the other stage no longer read
        if (ks + 1 < nk) {
            if (SMALL) {
                set_step_small(ks + 1);
            } else if (++cc == cpc) {
                cc = 0;
                if (++kx == a.kw) {
                    kx = 0;
                    if (++ky == a.kh) {
                        ky = 0;
                        set_tap(++tap);
                    }
                }
                set_pos(ky, kx);
            }
            issue(stage ^ 1, ks + 1, cc);
        }
        const uint8_t* st = lds + stage * SB;
        frag(st, 0, 0);
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            __builtin_amdgcn_sched_barrier(0);
            if (kk + 1 < BK / 16) frag(st, kk + 1, (kk + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[kk & 1][i], fb[kk & 1][j],
                                                                         acc[i][j], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    conv3d_epilogue<TM, TN, OK>(a, acc, row0 + wm * 32 * TM, col0 + wn * 32 * TN, l32, g,
                                SMALL ? nullptr : a.part);
}

// ---- the implicit GEMM on the ping-pong schedule (more than 128 outputs) -----
//
// conv3d_kernel's tiles (256x256, wave tiles 128x64, 64-k steps of one
// window position and channel chunk, two LDS stages) with the SharedLinear
// GEMM's main loop: the two waves of each SIMD (group 0 = waves 0-3, tile
// rows 0-127; group 1 = waves 4-7, rows 128-255) take turns, one issuing the
// 32 MFMAs of a whole 64-k step from fragment registers while the other
// reads its next step's fragments from LDS, so the matrix core does not wait
// on LDS reads.  Every phase ends at a workgroup barrier; group 1 runs one
// phase behind group 0.  Each wave loads A rows and B rows 128 grp + 32 wq
// + 8 j + lane / 8 (j < 4) of a step, its group's half of the stage:
//
//   phase     2s                             2s + 1
//   group 0   DMA of step s + 1 into stage   MFMAs of step s,
//             (s + 1) % 2, read step s       wait for its DMA
//   group 1   MFMAs of step s - 1            read step s, wait for its DMA
//                                            of step s + 1, DMA of step s + 2
//                                            into stage s % 2
//
// Group 0 writes the stage both groups finished reading in phases 2s - 2
// and 2s - 1; group 1 the stage it has just read (group 0 read it in phase
// 2s).  A step's data is complete before the barrier that ends phase 2s + 1
// (group 0's half) or 2s - 1 (group 1's, issued two phases earlier), and
// group 0 reads step s + 1 in phase 2s + 2.
template <int OK>
__global__ __launch_bounds__(512, 1) void conv3d_pp_kernel(ConvArgs a) {
    constexpr int BN = 256, BM = 256, BK = 64, RB = BK * 2;
    constexpr int TA = BM * RB, SB = TA + BN * RB;
    constexpr int GROUP = 4;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * SB];
    // per loaded row: padded frame of tap 0 and window origin offset, read
    // when the tap changes (kept out of registers: the fragments of a whole
    // step and the accumulators take 224 of them)
    __shared__ uint2 rinfo[4 * 512];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2, wq = wave & 3;
    const int l32 = lane & 31;
    const int g = lane >> 5;
    const int sw = lds_swizzle(l32);
    const uint32_t lds_base = (uint32_t)(uintptr_t)lds;

    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int group_size = GROUP * a.ntiles;
    const int first_m = (lid / group_size) * GROUP;
    const int gm = min(a.mtiles - first_m, GROUP);
    const int mt = first_m + (lid % group_size) % gm;
    const int nt = (lid % group_size) / gm;
    const int row0 = mt * BM;
    const int col0 = nt * BN;

    const uint32_t pix = (uint32_t)(a.cpad * 2);
    const uint32_t frame_bytes = (uint32_t)(a.H * a.W) * pix;
    const int hw = a.Ho * a.Wo;
    // the tile rows this lane loads (A and B alike): lrow + 8 j; rows 8
    // apart have swizzles that differ in bit 2
    const int lrow = 128 * grp + 32 * wq + (lane >> 3);
    const uint32_t chk_even = (uint32_t)(((lane & 7) ^ lds_swizzle(lrow)) * 16);
    const uint32_t chk_odd = chk_even ^ 64u;
    uint32_t rmask[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int m = row0 + lrow + 8 * j;
        int rpf = INT_MIN / 2;
        uint32_t rpix = (j & 1) ? chk_odd : chk_even;
        rmask[j] = 0;
        if (m < a.M) {
            const int to = m / hw;
            const int rem = m - to * hw;
            const int yo = rem / a.Wo;
            const int xo = rem - yo * a.Wo;
            const int yb = yo * a.sh - a.ph, xb = xo * a.sw - a.pw;
            rpf = (a.t0 + to) * a.st;
            rpix += (uint32_t)(yb * a.W + xb) * pix;
            uint32_t mk = 0;
            for (int ky = 0; ky < a.kh; ++ky) {
                if ((unsigned)(yb + ky * a.dh) >= (unsigned)a.H) continue;
                for (int kx = 0; kx < a.kw; ++kx)
                    if ((unsigned)(xb + kx * a.dw) < (unsigned)a.W) mk |= 1u << (ky * a.kw + kx);
            }
            rmask[j] = mk;
        }
        rinfo[j * 512 + tid] = make_uint2((uint32_t)rpf, rpix);
    }
    const uint32_t voffb0 = (uint32_t)(lrow * a.kp * 2);
    const i32x4 ra = wave_uniform(buffer_rsrc(a.staged, a.staged_bytes));
    const i32x4 rm = wave_uniform(buffer_rsrc(a.memory, a.memory_bytes));
    const i32x4 rb = wave_uniform(buffer_rsrc(
        a.packed + (long)col0 * a.kp, (uint32_t)(min(a.cout - col0, BN) * a.kp * 2)));

    // temporal tap and window position of the step a wave issues next, as in
    // conv3d_kernel (each lane reads only its own rinfo entries)
    uint32_t rbase[4];
    int memsel[4];
    auto set_tap = [&](int tap) {
        const int dtap = tap * a.dt - a.shift;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint2 ri = rinfo[j * 512 + tid];
            const int v = max((int)ri.x + dtap, 0);
            const bool fm = v < a.mem;
            const int sf = fm ? v : v - a.mem - a.fbase;
            rbase[j] = (uint32_t)sf * frame_bytes + ri.y;
            memsel[j] = __builtin_amdgcn_readfirstlane((int)fm);
        }
    };
    const int cpc = a.cpad / 64;
    int kbase = 0, nk = a.kp / 64;
    if (a.part) {
        const int all = a.kt * a.kh * a.kw * cpc;
        kbase = (int)((long)blockIdx.y * all / a.splits);
        nk = (int)((long)(blockIdx.y + 1) * all / a.splits) - kbase;
    }
    // Steps walk (tap, channel chunk, ky, kx) with kx fastest: the nine
    // window positions of one 64-channel chunk follow each other, so the
    // shifted A tiles they read overlap in L2 (with the chunk fastest, as the
    // packed k order runs, a chunk is read again only nine positions later,
    // past what L2 holds for all the workgroups of an XCD).  The packed
    // weights are read at the matching k offset.
    const int khw = a.kh * a.kw;
    int tap = kbase / (cpc * khw);
    int cc = (kbase / khw) % cpc, ky = (kbase % khw) / a.kw, kx = kbase % a.kw;
    set_tap(tap);
    int next = 0;   // the step this wave issues next
    auto issue = [&](int stage) {
        const uint32_t st = lds_base + stage * SB + (uint32_t)((128 * grp + 32 * wq) * RB);
        const uint32_t soffa = (uint32_t)(cc * RB);
        const uint32_t soffb = (uint32_t)(((tap * khw + ky * a.kw + kx) * cpc + cc) * RB);
        const uint32_t koff = (uint32_t)(ky * a.dh * a.W + kx * a.dw) * pix;
        const uint32_t bit = 1u << (ky * a.kw + kx);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            lds_dma16(memsel[j] ? rm : ra, st + j * 8 * RB,
                      (rmask[j] & bit) ? rbase[j] + koff : 0x80000000u, soffa);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            lds_dma16(rb, st + TA + j * 8 * RB,
                      voffb0 + (uint32_t)(j * 8 * a.kp * 2) + ((j & 1) ? chk_odd : chk_even), soffb);
        if (++next < nk && ++kx == a.kw) {
            kx = 0;
            if (++ky == a.kh) {
                ky = 0;
                if (++cc == cpc) {
                    cc = 0;
                    set_tap(++tap);
                }
            }
        }
    };

    f32x16 acc[4][2];
    bf16x8 fa[4][4], fb[4][2];
    auto read_step = [&](int stage) {
        const uint8_t* st = lds + stage * SB;
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            const int pc = ((2 * kk + g) ^ sw) * 16;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                fa[kk][i] = as_bf16x8(*(const uint4*)(st + (grp * 128 + 32 * i + l32) * RB + pc));
#pragma unroll
            for (int j = 0; j < 2; ++j)
                fb[kk][j] = as_bf16x8(*(const uint4*)(st + TA + (wq * 64 + 32 * j + l32) * RB + pc));
        }
    };
    auto barrier = [] {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // steps 0 and 1 by both groups
    issue(0);
    if (nk > 1) issue(1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    barrier();
    if (grp == 1) barrier();
#pragma unroll 1
    for (int s = 0; s < nk; ++s) {
        // memory phase
        if (grp == 0 && s >= 1 && s + 1 < nk) issue((s + 1) & 1);
        read_step(s & 1);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (grp == 1) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // its half of step s + 1
            if (s + 2 < nk) issue(s & 1);
        }
        barrier();
        // MFMA phase
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[kk][i], fb[kk][j],
                                                                        acc[i][j], 0, 0, 0);
        __builtin_amdgcn_s_setprio(0);
        if (grp == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // its half of step s + 1
        barrier();
    }
    if (grp == 0) barrier();

    if (a.part && a.slots) {
        // slot layout: float4 c (4 accumulator registers) of thread tid at
        // byte (c * 512 + tid) * 16.  The stores write through; every wave
        // waits for its own before the barrier, and the arrival is an
        // agent-scope acquire-release read-modify-write that releases this
        // range's slot and, for the last range, acquires the others'.
        constexpr int kFlags = 1 | 16;   // coherent across the XCDs' L2s
        const int tile = lid;
        auto slot = [&](int r) {
            return __builtin_amdgcn_make_buffer_rsrc(
                a.slots + ((long)tile * a.splits + r) * (BM * BN), (short)0, BM * BN * 4, 0x00020000);
        };
        const __amdgpu_buffer_rsrc_t mine = slot((int)blockIdx.y);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const f32x4 v = {acc[i][j][4 * c], acc[i][j][4 * c + 1], acc[i][j][4 * c + 2],
                                     acc[i][j][4 * c + 3]};
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), mine,
                                                           tid * 16, ((i * 2 + j) * 4 + c) * 512 * 16,
                                                           kFlags);
                }
        __shared__ int arrival;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0)
            arrival = __hip_atomic_fetch_add(&a.counters[tile], 1, __ATOMIC_ACQ_REL,
                                             __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (arrival != a.splits - 1) return;
        // the sum of every range in range order, as conv3d_reduce_kernel adds
        // them, so the result does not depend on the order of arrival; with
        // two ranges the other range's slot is added to this one's registers
        // (p0 + p1 either way round)
        const bool two = a.splits == 2;
#pragma unroll 1
        for (int r = two ? 1 : 0; r < a.splits; ++r) {
            const __amdgpu_buffer_rsrc_t other = slot(two ? 1 - (int)blockIdx.y : r);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                __builtin_amdgcn_sched_barrier(0);
                f32x4 v[2][2][4];
#pragma unroll
                for (int iq = 0; iq < 2; ++iq)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
#pragma unroll
                        for (int c = 0; c < 4; ++c)
                            v[iq][j][c] = __builtin_bit_cast(
                                f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                           other, tid * 16, (((2 * h + iq) * 2 + j) * 4 + c) * 512 * 16,
                                           kFlags));
#pragma unroll
                for (int iq = 0; iq < 2; ++iq)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            f32x16& d = acc[2 * h + iq][j];
                            if (r == 0 && !two) {
                                d[4 * c] = v[iq][j][c].x;
                                d[4 * c + 1] = v[iq][j][c].y;
                                d[4 * c + 2] = v[iq][j][c].z;
                                d[4 * c + 3] = v[iq][j][c].w;
                            } else {
                                d[4 * c] += v[iq][j][c].x;
                                d[4 * c + 1] += v[iq][j][c].y;
                                d[4 * c + 2] += v[iq][j][c].z;
                                d[4 * c + 3] += v[iq][j][c].w;
                            }
                        }
            }
        }
        if (tid == 0)
            __hip_atomic_store(&a.counters[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        conv3d_epilogue<4, 2, OK>(a, acc, row0 + 128 * grp, col0 + 64 * wq, l32, g, nullptr);
        return;
    }
    conv3d_epilogue<4, 2, OK>(a, acc, row0 + 128 * grp, col0 + 64 * wq, l32, g, a.part);
}

// ---- 3x3 spatial windows, stride 1: the halo kernel --------------------------
//
// For a 3x3 spatial window with unit stride and dilation, the nine window
// positions of one output tile read nine shifted copies of the same input
// pixels.  This kernel tiles the output frame in 2-D blocks of TH x TW
// pixels (TW = 128, or 64 for frames whose width 128-pixel tiles fit
// badly; TH x TW = 512 GEMM rows at BN 128, 1024 at BN 32; a wave owns 128
// of them, i.e. 128 / TW output rows; times BN-channel tiles of the
// outputs) and loads, per k-chunk of 16 input
// channels and temporal tap, the (TH + 2) x (TW + 2) input halo once into LDS
// (32 bytes per pixel) together with the chunk's weights for all nine
// positions; the nine positions are then nine 16-k MFMA slices that read the
// halo at shifted pixel offsets.  Against one 64-channel A tile per window
// position, this cuts the LDS writes per MFMA by 3x and the A traffic from L2
// by about 6x, and takes one barrier per 144 k instead of per 64 k.
//
// LDS stage: halo [(TH + 2) * (TW + 2) pixels][2 chunks of 16 bytes], then weights
// [9 positions][BN rows][2 chunks]; chunk c of pixel (or row) p is stored at
// position c ^ ((p >> 3) & 1), which puts the 16 lanes of each ds_read_b128
// phase (16 consecutive pixels or rows) on distinct banks for any shift.
// Two stages: the next chunk's DMA overlaps this chunk's MFMAs.  Each tile
// lies in one output frame, so a tap's input frame, memory or staged, is
// the same for the whole tile.
// Output tile rows at tile width tw: 512 GEMM rows (128 x 64 wave tiles) at
// BN 128, 1024 (128 x 32 wave tiles) at BN 32.
constexpr int halo_tile_rows(int bn, int tw) { return (bn >= 64 ? 512 : 1024) / tw; }

template <int BN, int TW, int OK>
__global__ __launch_bounds__(512, 1) void conv3d_halo_kernel(ConvArgs a) {
    constexpr int TM = 4, TN = BN >= 64 ? 2 : 1;
    constexpr int WN = BN / (32 * TN), WM = 8 / WN;
    constexpr int BM = WM * 32 * TM;
    constexpr int TH = BM / TW;
    static_assert(TH == halo_tile_rows(BN, TW) && (TW == 128 || TW == 64), "tile shape");
    constexpr int kHaloW = TW + 2;              // halo width
    constexpr int FPR = TW / 32;                // fragments per image row
    constexpr int kHaloPix = (TH + 2) * kHaloW;
    constexpr int kHaloBytes = kHaloPix * 32;
    constexpr int BBYTES = 9 * BN * 32;
    constexpr int SB = kHaloBytes + BBYTES;
    constexpr int HSLOTS = kHaloPix * 2, HINS = (HSLOTS + 511) / 512;
    constexpr int BSLOTS = 9 * BN * 2, BINS = (BSLOTS + 511) / 512;
    constexpr uint32_t OOB = 0x80000000u;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * SB];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31;
    const int g = lane >> 5;
    const int wm = wave / WN;
    const int wn = wave % WN;
    const uint32_t lds_base = (uint32_t)(uintptr_t)lds;

    // tile: output channels [col0, col0 + BN) of output frame to, rows
    // [y0, y0 + TH), columns [x0, x0 + 128); the channel tiles of one block
    // of pixels are neighbours, so they share its halo in L2
    const int lid = xcd_remap(blockIdx.x, gridDim.x);
    const int nt = lid % a.ntiles;
    const int sp = lid / a.ntiles;
    const int xt = sp % a.xtiles;
    const int yt = (sp / a.xtiles) % a.ytiles;
    const int to = sp / (a.xtiles * a.ytiles);
    const int y0 = yt * TH, x0 = xt * TW;
    const int col0 = nt * BN;
    // this wave's 128 GEMM rows: output rows ty .. ty + 128 / TW - 1 of the
    // tile, fragment i at row ty + i / FPR, columns 32 (i % FPR) + [0, 32)
    const int ty = (wm * 32 * TM) / TW;

    const uint32_t pix = (uint32_t)(a.cpad * 2);
    const uint32_t frame_bytes = (uint32_t)(a.H * a.W) * pix;
    // Slot sl of a DMA instruction set: halo (pixel sl / 2, stored chunk
    // sl % 2) at the frame offset of that pixel and chunk; weights (position
    // q, row, stored chunk) at the row's k offset of q; the tap and channel
    // chunk go in soffset.  Recomputed per issue: a few VALU operations a
    // slot, against 72 MFMAs a chunk.
    auto halo_off = [&](int sl) -> uint32_t {
        const int p = sl >> 1;
        const int c = (sl & 1) ^ ((p >> 3) & 1);
        const int hy = p / kHaloW;
        const int yy = y0 - a.ph + hy;
        const int xx = x0 - a.pw + (p - hy * kHaloW);
        const bool in = (unsigned)yy < (unsigned)a.H && (unsigned)xx < (unsigned)a.W;
        return in ? (uint32_t)(yy * a.W + xx) * pix + c * 16 : OOB;
    };
    auto weight_off = [&](int sl) -> uint32_t {
        const int q = sl / (BN * 2);
        const int row = (sl >> 1) - q * BN;
        const int c = (sl & 1) ^ ((row >> 3) & 1);
        return (uint32_t)(row * a.kp + q * a.cpad) * 2 + c * 16;
    };
    const i32x4 ra = wave_uniform(buffer_rsrc(a.staged, a.staged_bytes));
    const i32x4 rm = wave_uniform(buffer_rsrc(a.memory, a.memory_bytes));
    const i32x4 rb = wave_uniform(buffer_rsrc(a.packed + (long)col0 * a.kp,
                                              (uint32_t)(min(a.cout - col0, BN) * a.kp * 2)));

    const int cpc = a.cpad / 16;   // 16-channel chunks per pixel
    const int nchunks = a.kt * cpc;
    const int tbase = (a.t0 + to) * a.st - a.shift;
    auto issue_halo = [&](int stage, int cs) {
        const int tap = cs / cpc, cc = cs - tap * cpc;
        const int v = max(tbase + tap * a.dt, 0);
        const bool fm = v < a.mem;
        const uint32_t fo = (uint32_t)(fm ? v : v - a.mem - a.fbase) * frame_bytes + cc * 32;
        const uint32_t st = lds_base + stage * SB;
#pragma unroll
        for (int j = 0; j < HINS; ++j) {
            const int sl0 = (j * 8 + wave) * 64;   // wave-uniform
            if (sl0 >= HSLOTS) break;
            if (sl0 + lane < HSLOTS)
                lds_dma16(fm ? rm : ra, st + sl0 * 16, halo_off(sl0 + lane),
                          __builtin_amdgcn_readfirstlane(fo));
        }
    };
    auto issue_weights = [&](int stage, int cs) {
        const int tap = cs / cpc, cc = cs - tap * cpc;
        const uint32_t st = lds_base + stage * SB;
        const uint32_t kb = (uint32_t)(tap * 9 * a.cpad + cc * 16) * 2;
#pragma unroll
        for (int j = 0; j < BINS; ++j) {
            const int sl0 = (j * 8 + wave) * 64;
            if (sl0 >= BSLOTS) break;
            if (sl0 + lane < BSLOTS)
                lds_dma16(rb, st + kHaloBytes + sl0 * 16, weight_off(sl0 + lane),
                          __builtin_amdgcn_readfirstlane(kb));
        }
    };

    // instruction p of this wave's DMA of chunk cs: halo instructions first,
    // then weight instructions
    auto issue_part = [&](int stage, int cs, int p) {
        const int tap = cs / cpc, cc = cs - tap * cpc;
        const uint32_t st = lds_base + stage * SB;
        if (p < HINS) {
            const int v = max(tbase + tap * a.dt, 0);
            const bool fm = v < a.mem;
            const uint32_t fo = (uint32_t)(fm ? v : v - a.mem - a.fbase) * frame_bytes + cc * 32;
            const int sl0 = (p * 8 + wave) * 64;   // wave-uniform
            if (sl0 < HSLOTS && sl0 + lane < HSLOTS)
                lds_dma16(fm ? rm : ra, st + sl0 * 16, halo_off(sl0 + lane),
                          __builtin_amdgcn_readfirstlane(fo));
        } else {
            const uint32_t kb = (uint32_t)(tap * 9 * a.cpad + cc * 16) * 2;
            const int sl0 = ((p - HINS) * 8 + wave) * 64;
            if (sl0 < BSLOTS && sl0 + lane < BSLOTS)
                lds_dma16(rb, st + kHaloBytes + sl0 * 16, weight_off(sl0 + lane),
                          __builtin_amdgcn_readfirstlane(kb));
        }
    };

    f32x16 acc[TM][TN];
    bf16x8 fa[2][TM], fb[2][TN];
    // fragments of window position q (ky = q / 3, kx = q % 3).  Within an
    // image row, fragment i is 32 pixels after the row's first, which keeps
    // the swizzle bit ((p >> 3) & 1): its address is that one's plus 1 KB.
    const int pa = ty * kHaloW + l32;
    const int rowb = wn * 32 * TN + l32;
    const int boffl = (rowb * 2 + (g ^ ((rowb >> 3) & 1))) * 16;
    auto frag = [&](const uint8_t* st, int q, int slot) {
        const int ky = q / 3, kx = q - 3 * ky;
#pragma unroll
        for (int r = 0; r < TM / FPR; ++r) {
            const int p = pa + (r + ky) * kHaloW + kx;
            const uint8_t* ab = st + (p * 2 + (g ^ ((p >> 3) & 1))) * 16;
#pragma unroll
            for (int i = 0; i < FPR; ++i)
                fa[slot][r * FPR + i] = as_bf16x8(*(const uint4*)(ab + 1024 * i));
        }
        const uint8_t* bb = st + kHaloBytes + q * BN * 32 + boffl;
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[slot][j] = as_bf16x8(*(const uint4*)(bb + 1024 * j));
    };
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    issue_halo(0, 0);
    issue_weights(0, 0);
#pragma unroll 1
    for (int cs = 0; cs < nchunks; ++cs) {
        const int stage = cs & 1;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();   // chunk cs visible to all waves; the other stage no longer read
        const uint8_t* st = lds + stage * SB;
        frag(st, 0, 0);
        // The next chunk's DMA into the other stage is issued behind the
        // positions' MFMAs, this wave's instructions spread over positions
        // 0..6 (instruction p after position 7p / NP): a wave whose memory
        // instruction is going out does not issue MFMAs, so the spread keeps
        // the two waves of a SIMD from stalling together, and the last ones
        // still land two positions before the next barrier (measured: 2-3%
        // faster than issuing all after positions 0 and 1).
        constexpr int NP = HINS + BINS;
#pragma unroll
        for (int q = 0; q < 9; ++q) {
            __builtin_amdgcn_sched_barrier(0);
            if (q + 1 < 9) frag(st, q + 1, (q + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[q & 1][i], fb[q & 1][j],
                                                                         acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (cs + 1 < nchunks) {
#pragma unroll
                for (int pi = 0; pi < NP; ++pi)
                    if (q == pi * 7 / NP) issue_part(stage ^ 1, cs + 1, pi);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    // Epilogue: register r of a 32x32 accumulator is GEMM row 8(r/4) + 4g +
    // r%4 of its block, i.e. 4 consecutive output pixels of one row.
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col = col0 + wn * 32 * TN + 32 * j + l32;
        if (col >= a.cout) continue;
        const float bv = a.bias ? a.bias[col] : 0.f;
        const long cbase = (long)col * a.out_cstep + a.out_off;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                const int y = y0 + ty + i / FPR;
                const int x = x0 + 32 * (i % FPR) + 8 * rg + 4 * g;
                if (y >= a.Ho || x >= a.Wo) continue;
                const long xrow = ((long)to * a.Ho + y) * a.Wo + x;
                const float v[4] = {acc[i][j][4 * rg] + bv, acc[i][j][4 * rg + 1] + bv,
                                    acc[i][j][4 * rg + 2] + bv, acc[i][j][4 * rg + 3] + bv};
                if (a.vec_ok && x + 3 < a.Wo) {
                    store4(a.out, cbase + xrow, v[0], v[1], v[2], v[3], OK);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        if (x + e >= a.Wo) continue;
                        const long idx = cbase + xrow + e;
                        if (OK == 1)
                            ((uint16_t*)a.out)[idx] = f32_to_bf16(v[e]);
                        else if (OK == 2)
                            ((_Float16*)a.out)[idx] = f32_to_f16(v[e]);
                        else
                            ((float*)a.out)[idx] = v[e];
                    }
                }
            }
    }
}

template <int BN, int TW>
void launch_conv3d_halo(const ConvArgs& a, hipStream_t stream) {
    const unsigned grid = (unsigned)a.mtiles;
    if (a.out_kind == 1)
        conv3d_halo_kernel<BN, TW, 1><<<grid, 512, 0, stream>>>(a);
    else if (a.out_kind == 2)
        conv3d_halo_kernel<BN, TW, 2><<<grid, 512, 0, stream>>>(a);
    else
        conv3d_halo_kernel<BN, TW, 0><<<grid, 512, 0, stream>>>(a);
}

// sum of the taps' partial tiles in tap order, plus the bias, stored as
// out_kind at out[col * out_cstep + out_off + m]
__global__ __launch_bounds__(256) void conv3d_reduce_kernel(const float* __restrict__ part,
                                                            int splits, long part_split, int cout,
                                                            int M, const float* __restrict__ bias,
                                                            void* __restrict__ out, int out_kind,
                                                            long out_cstep, long out_off) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)cout * M) return;
    const int col = (int)(i / M);
    const long m = i - (long)col * M;
    float v = part[i];
    for (int sp = 1; sp < splits; ++sp) v += part[sp * part_split + i];
    if (bias) v += bias[col];
    const long idx = (long)col * out_cstep + out_off + m;
    if (out_kind == 1)
        ((uint16_t*)out)[idx] = f32_to_bf16(v);
    else if (out_kind == 2)
        ((_Float16*)out)[idx] = f32_to_f16(v);
    else
        ((float*)out)[idx] = v;
}

// ---- at most 8 input channels, 3x3x3, unit strides: the RGB-input conv ----------
//
// The encoder's first conv (3 -> 128 channels) reads little and writes a
// 128-channel bf16 frame per input frame: it is bound by its output bytes,
// which must leave in long runs of one channel plane (stores of 4 pixels of
// 32 channels at a time, as the implicit GEMM's lanes hold them, take more
// than twice as long).  The product is
//   D[x][co] = sum over the 28 window positions (27 and a zero one) and 8
//              staged channels of X[pos][x][c] W[co][pos*8 + c],
// one 32x32x16 MFMA per two positions and 32 pixels, each lane's A operand
// one 16-byte staged pixel (the 8 channels of one position) read from LDS,
// its B operand 8 weights held in registers; a lane then holds 4
// consecutive pixels of one channel per accumulator group, converted and
// written to a [channel][pixel] LDS tile 8 bytes at a time, from which the
// strip rows leave 256 bytes per channel.  A workgroup owns a 128-pixel
// strip of one output frame and a band of rows; per output row a group of
// four waves stages the nine input rows (3 taps x 3 rows) of the strip and
// one pixel each side; wave w of a group computes output channels 32w ..
// 32w + 31.
//
// Waves 0-3 (group 0) take the band's even rows, waves 4-7 (group 1) its odd
// rows, each group with its own LDS halo buffers and output tile.  A row
// takes two phases, each ended by a workgroup barrier:
//   X: the MFMAs on the row's halo, the group's next row's halo (loaded
//      during the previous Y) into the other buffer, the outputs into LDS;
//   Y: the loads of the row after next, the output stores.
// Group 1 runs one phase behind group 0, so that one group's stores drain
// while the other group's MFMAs run.
constexpr int kRgbInHaloW = 130;
constexpr int kRgbInRowBytes = kRgbInHaloW * 16;
constexpr int kRgbInBuf = 9 * kRgbInRowBytes;
constexpr int kRgbInLoads = (9 * kRgbInHaloW + 255) / 256;
constexpr int kRgbInOutPitch = 136;   // bf16 per staged output row (128 pixels + 8)
constexpr int kRgbInOutBytes = 128 * kRgbInOutPitch * 2;
constexpr int kRgbInGroupBytes = 2 * kRgbInBuf + kRgbInOutBytes;

// 16-bit outputs whose rows allow 16-byte stores (VEC8) leave through the
// group's LDS tile: each thread then stores 16-byte runs of 8 pixels of one
// channel, a wave instruction the 256-byte strip rows of 4 channels.
// Otherwise (fp32 outputs, rows not a multiple of 8 pixels) each lane stores
// its accumulators element by element.
template <int OK, bool VEC8>
__global__ __launch_bounds__(512, 1) void conv3d_rgbin_kernel(ConvArgs a, int strips, int bands,
                                                              int band_rows) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2 * kRgbInGroupBytes + 16];
    const int tid = threadIdx.x;
    const int gt = tid & 255;   // thread of the group
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2;
    const int l32 = lane & 31;
    const int khalf = lane >> 5;
    uint8_t* const glds = lds + grp * kRgbInGroupBytes;
    uint16_t* const otile = (uint16_t*)(glds + 2 * kRgbInBuf);
    const uint8_t* const zchunk = lds + 2 * kRgbInGroupBytes;
    // the output as raw bytes (VEC8: below 2 GiB, checked by the launcher)
    const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
        a.out, (short)0, VEC8 ? (int)((long)a.cout * a.out_cstep * 2 < 0x7fffffffL
                                          ? (long)a.cout * a.out_cstep * 2 : 0x7fffffffL)
                              : 0,
        0x00020000);
    int bid = xcd_remap(blockIdx.x, gridDim.x);
    const int strip = bid % strips;
    bid /= strips;
    const int band = bid % bands;
    const int to = bid / bands;
    const int x0 = strip * 128;
    const int y0 = band * band_rows;
    const int y1 = min(a.Ho, y0 + band_rows);
    const int co0 = 32 * (wave & 3);
    const bool active = co0 < a.cout;

    // weights: A operand rows co0 + l32, k = 16 ks + 8 khalf .. + 7 (window
    // position 2 ks + khalf); position 27 and channels past the packed row
    // are zero
    bf16x8 wa[14];
#pragma unroll
    for (int ks = 0; ks < 14; ++ks) {
        uint4 u = make_uint4(0, 0, 0, 0);
        const int k = 16 * ks + 8 * khalf;
        if (active && k + 8 <= 27 * 8)
            u = *reinterpret_cast<const uint4*>(a.packed + (long)(co0 + l32) * a.kp + k);
        wa[ks] = as_bf16x8(u);
    }
    // the output channel of a lane's accumulators
    const int co = co0 + l32;
    const float bv = (active && a.bias) ? a.bias[co] : 0.f;
    // B operand addresses (byte offsets in a halo buffer) of position
    // 2 ks + khalf for pixel column l32 of tile 0; tiles j add 512 bytes
    uint32_t boff[14];
#pragma unroll
    for (int ks = 0; ks < 14; ++ks) {
        const int pos = min(2 * ks + khalf, 26);   // 27 reads the zero chunk instead
        boff[ks] = (uint32_t)((pos / 3) * kRgbInRowBytes + (l32 + pos % 3) * 16);
    }
    if (tid == 0) *reinterpret_cast<uint4*>(lds + 2 * kRgbInGroupBytes) = make_uint4(0, 0, 0, 0);

    const uint32_t pix = 16;
    const uint32_t frame_bytes = (uint32_t)(a.H * a.W) * pix;
    const int tbase = (a.t0 + to) * a.st - a.shift;
    // Staged halo of output row y: item i = (tap * 3 + ky) * 130 + column.
    // Every load is issued, from a clamped address where the pixel lies in
    // the padding (store_rows zeroes those), so that no load sits under a
    // branch.  ok: one bit per load.
    auto load_rows = [&](int y, uint4 (&v)[kRgbInLoads], uint32_t& ok) {
        ok = 0;
#pragma unroll
        for (int k = 0; k < kRgbInLoads; ++k) {
            const int i = min(gt + 256 * k, 9 * kRgbInHaloW - 1);
            const int row = i / kRgbInHaloW, c = i - row * kRgbInHaloW;
            const int tap = row / 3, ky = row - 3 * tap;
            const int yy = y + ky - a.ph, xx = x0 - a.pw + c;
            const int fv = max(tbase + tap * a.dt, 0) - a.fbase;
            uint32_t off = (uint32_t)max(fv, 0) * frame_bytes +
                           (uint32_t)(min(max(yy, 0), a.H - 1) * a.W + min(max(xx, 0), a.W - 1)) * pix;
            const bool in = gt + 256 * k < 9 * kRgbInHaloW && (unsigned)yy < (unsigned)a.H &&
                            (unsigned)xx < (unsigned)a.W && fv >= 0 && off + 16 <= a.staged_bytes;
            off = min(off, a.staged_bytes - 16);
            v[k] = *reinterpret_cast<const uint4*>((const uint8_t*)a.staged + off);
            ok |= (uint32_t)in << k;
        }
    };
    auto store_rows = [&](int buf, const uint4 (&v)[kRgbInLoads], uint32_t ok) {
        // 16-byte output runs: every load and store is unconditional, so the
        // compiler's waits for the loads leave the eight output stores that
        // followed them in flight; otherwise one wait for all
        if constexpr (!VEC8) __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
#pragma unroll
        for (int k = 0; k < kRgbInLoads; ++k) {
            const int i = gt + 256 * k;
            const uint32_t m = 0u - ((ok >> k) & 1);
            if (i < 9 * kRgbInHaloW)
                *reinterpret_cast<uint4*>(glds + buf * kRgbInBuf + i * 16) =
                    make_uint4(v[k].x & m, v[k].y & m, v[k].z & m, v[k].w & m);
        }
    };
    auto barrier = [] {
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
    };

    // the group's rows y0 + grp + 2i, i < rounds (past y1: no MFMAs or
    // stores, the phases and barriers only)
    const int rounds = (y1 - y0 + 1) / 2;
    auto row_of = [&](int i) { return min(y0 + grp + 2 * i, y1 - 1); };
    uint4 pre[kRgbInLoads];
    uint32_t pre_ok = 0;
    if (rounds > 0) {
        load_rows(row_of(0), pre, pre_ok);
        store_rows(0, pre, pre_ok);
        load_rows(row_of(1), pre, pre_ok);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);   // weights and bias on every path
    barrier();
    if (grp == 1) barrier();
    for (int i = 0; i < rounds; ++i) {
        const int y = y0 + grp + 2 * i;
        const bool valid = y < y1;
        const int buf = i & 1;
        // phase X
        f32x16 acc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = f32x16{};
        if (active && valid) {
            // B fragments read one k-step ahead of their MFMAs: in phase X
            // only one wave of each SIMD issues MFMAs, so nothing else hides
            // the LDS latency
            const uint8_t* hb = glds + buf * kRgbInBuf;
            uint4 bf[2][4];
            auto read_b = [&](int ks, uint4 (&b)[4]) {
                // position 27 (lanes 32-63 of the last k-step) reads the zero chunk
                const bool z = ks == 13 && khalf == 1;
                const uint8_t* bp = z ? zchunk : hb + boff[ks];
                const int js = z ? 0 : 512;
#pragma unroll
                for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const uint4*>(bp + js * j);
            };
            read_b(0, bf[0]);
#pragma unroll
            for (int ks = 0; ks < 14; ++ks) {
                __builtin_amdgcn_sched_barrier(0);
                if (ks + 1 < 14) read_b(ks + 1, bf[(ks + 1) & 1]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(bf[ks & 1][j]), wa[ks],
                                                                     acc[j], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // the next row's halo into the other buffer (after the last row the
        // buffer, read by no one any more, takes a row again)
        store_rows(buf ^ 1, pre, pre_ok);
        // D[x][co]: register 4q + e of lane l is pixel 32j + 8q + 4(l/32) + e
        // of tile j, channel co: four consecutive pixels, one 8-byte LDS write
        if constexpr (VEC8) {
            if (active && valid) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float v0 = acc[j][4 * q] + bv, v1 = acc[j][4 * q + 1] + bv;
                        const float v2 = acc[j][4 * q + 2] + bv, v3 = acc[j][4 * q + 3] + bv;
                        const uint2 w = OK == 2 ? make_uint2(pack2_f16_rne(v0, v1), pack2_f16_rne(v2, v3))
                                                : make_uint2(pack2_bf16_rne(v0, v1), pack2_bf16_rne(v2, v3));
                        *reinterpret_cast<uint2*>(otile + co * kRgbInOutPitch + 32 * j + 8 * q + 4 * khalf) = w;
                    }
            }
        }
        barrier();
        // phase Y: the loads of the row after next, then the stores
        load_rows(row_of(i + 2), pre, pre_ok);
        const long rowo = a.out_off + ((long)to * a.Ho + y) * a.Wo;
        if constexpr (VEC8) {
            // 16-byte runs through a buffer descriptor of the output: a run
            // past the channel count or the row (x >= Wo; Wo % 8 == 0), or of
            // a row past the band, takes an offset past the range and is
            // dropped, so every thread issues all eight stores
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int c = gt + 256 * k;
                const int co = c >> 4, x = x0 + 8 * (c & 15);
                const uint4 v = *reinterpret_cast<const uint4*>(otile + co * kRgbInOutPitch + 8 * (c & 15));
                const bool keep = valid && co < a.cout && x < a.Wo;
                const uint32_t off = keep ? (uint32_t)(((long)co * a.out_cstep + rowo + x) * 2) : 0x80000000u;
                __builtin_amdgcn_raw_buffer_store_b128(u32x4{v.x, v.y, v.z, v.w}, ro, off, 0, 2);
            }
        } else if (active && valid) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int x = x0 + 32 * j + 8 * (r >> 2) + 4 * khalf + (r & 3);
                    if (x >= a.Wo) continue;
                    const long idx = (long)co * a.out_cstep + rowo + x;
                    const float v = acc[j][r] + bv;
                    if (OK == 1)
                        ((uint16_t*)a.out)[idx] = f32_to_bf16(v);
                    else if (OK == 2)
                        ((_Float16*)a.out)[idx] = f32_to_f16(v);
                    else
                        ((float*)a.out)[idx] = v;
                }
        }
        barrier();
    }
    if (grp == 0) barrier();
}

bool conv3d_rgbin_ok(const Conv3dShape& s, int mem, int ho, int wo, int h, int w) {
    return s.cpad == 8 && s.kt == 3 && s.kh == 3 && s.kw == 3 && s.st == 1 && s.sh == 1 &&
           s.sw == 1 && s.dt == 1 && s.dh == 1 && s.dw == 1 && s.ph == 1 && s.pw == 1 &&
           s.cout % 32 == 0 && s.cout <= 128 && mem == 0 && ho == h && wo == w;
}

template <int BN, bool SMALL>
void launch_conv3d_kernel(const ConvArgs& a, hipStream_t stream) {
    const dim3 grid((unsigned)(a.mtiles * a.ntiles), a.part ? (unsigned)a.splits : 1u);
    if (a.out_kind == 1)
        conv3d_kernel<BN, 1, SMALL><<<grid, 512, 0, stream>>>(a);
    else if (a.out_kind == 2)
        conv3d_kernel<BN, 2, SMALL><<<grid, 512, 0, stream>>>(a);
    else
        conv3d_kernel<BN, 0, SMALL><<<grid, 512, 0, stream>>>(a);
}

template <int BN>
void launch_conv3d_kernel(const ConvArgs& a, hipStream_t stream) {
    if (a.cpad < 64) {
        launch_conv3d_kernel<BN, true>(a, stream);
    } else if (BN == 256) {
        const dim3 grid((unsigned)(a.mtiles * a.ntiles), a.part ? (unsigned)a.splits : 1u);
        if (a.out_kind == 1)
            conv3d_pp_kernel<1><<<grid, 512, 0, stream>>>(a);
        else if (a.out_kind == 2)
            conv3d_pp_kernel<2><<<grid, 512, 0, stream>>>(a);
        else
            conv3d_pp_kernel<0><<<grid, 512, 0, stream>>>(a);
    } else {
        launch_conv3d_kernel<BN, false>(a, stream);
    }
}

// ---- VAEUpsample3D's depth-to-space shuffle (vae_upsample3d.cpp:270-318) ----
//
// One thread per output element (channel blockIdx.y): output time ot is
// shuffled time st = ot (or ot + 1 past the removed time 1), st = f * tr + z;
// output pixel (y2, x2) = (y * sr + yo, x * sr + xo) reads packed channel
// ((yo * sr + xo) * tr + z) * channels + c.  Writes are contiguous; the two
// (or one) interleaved source planes of a row are each read contiguously.
template <typename T>
__global__ __launch_bounds__(256) void vae_shuffle_kernel(const T* __restrict__ packed,
                                                          long packed_cstep, int channels, int h,
                                                          int w, int tr, int sr, int remove_head,
                                                          int out_t, T* __restrict__ out,
                                                          long out_cstep) {
    const int c = blockIdx.y;
    const int ow = w * sr, oh = h * sr;
    const long plane = (long)oh * ow;
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= plane * out_t) return;
    const int ot = (int)(i / plane);
    const long rem = i - (long)ot * plane;
    const int y2 = (int)(rem / ow), x2 = (int)(rem - (long)y2 * ow);
    const int st = remove_head && ot >= 1 ? ot + 1 : ot;
    const int f = st / tr, z = st - f * tr;
    const int y = y2 / sr, yo = y2 - y * sr;
    const int x = x2 / sr, xo = x2 - x * sr;
    const long pc = (long)((yo * sr + xo) * tr + z) * channels + c;
    out[(long)c * out_cstep + i] = packed[pc * packed_cstep + ((long)f * h + y) * w + x];
}

}  // namespace

hipError_t launch_vae_shuffle(const void* packed, int kind, long packed_cstep, int channels,
                              int frames, int h, int w, int tr, int sr, int remove_head,
                              void* out, long out_cstep, hipStream_t stream) {
    const int out_t = frames * tr - (remove_head ? 1 : 0);
    const long n = (long)out_t * h * sr * w * sr;
    if (n <= 0 || channels <= 0) return hipSuccess;
    if (channels > 65535) return hipErrorInvalidValue;
    const dim3 grid((unsigned)((n + 255) / 256), (unsigned)channels);
    if (kind == 0)
        vae_shuffle_kernel<float><<<grid, 256, 0, stream>>>(
            (const float*)packed, packed_cstep, channels, h, w, tr, sr, remove_head, out_t,
            (float*)out, out_cstep);
    else
        vae_shuffle_kernel<uint16_t><<<grid, 256, 0, stream>>>(
            (const uint16_t*)packed, packed_cstep, channels, h, w, tr, sr, remove_head, out_t,
            (uint16_t*)out, out_cstep);
    return hipGetLastError();
}

template <int P>
static void stage_launch(const void* input, int in_kind, long in_cstep, int cin, long pixels,
                         int cpad, int vec, uint16_t* staged, uint16_t* tail, long tail_q0,
                         hipStream_t stream) {
    const dim3 grid((unsigned)((pixels + P - 1) / P), (unsigned)((cpad + 63) / 64));
    if (in_kind == 1)
        conv3d_stage_kernel<1, P><<<grid, kStageThreads, 0, stream>>>(
            input, in_cstep, cin, pixels, cpad, vec, staged, tail, tail_q0);
    else if (in_kind == 2)
        conv3d_stage_kernel<2, P><<<grid, kStageThreads, 0, stream>>>(
            input, in_cstep, cin, pixels, cpad, vec, staged, tail, tail_q0);
    else
        conv3d_stage_kernel<0, P><<<grid, kStageThreads, 0, stream>>>(
            input, in_cstep, cin, pixels, cpad, vec, staged, tail, tail_q0);
}

hipError_t launch_conv3d_stage(const void* input, int in_kind, long in_cstep, int cin,
                               long pixels, int cpad, uint16_t* staged, uint16_t* tail,
                               long tail_q0, hipStream_t stream) {
    if (pixels <= 0) return hipSuccess;
    // 16-byte runs need 16-byte aligned channel rows
    const int esz = in_kind == 0 ? 4 : 2;
    const int vec = ((uintptr_t)input % 16) == 0 && (in_cstep * esz) % 16 == 0;
    if (cpad >= 64 && cpad % 64 == 0 && vec) {
        const dim3 grid((unsigned)((pixels + 255) / 256), (unsigned)(cpad / 64));
        if (in_kind == 1)
            conv3d_stage_t_kernel<1><<<grid, 256, 0, stream>>>(input, in_cstep, cin, pixels, cpad,
                                                               staged, tail, tail_q0);
        else if (in_kind == 2)
            conv3d_stage_t_kernel<2><<<grid, 256, 0, stream>>>(input, in_cstep, cin, pixels, cpad,
                                                               staged, tail, tail_q0);
        else
            conv3d_stage_t_kernel<0><<<grid, 256, 0, stream>>>(input, in_cstep, cin, pixels, cpad,
                                                               staged, tail, tail_q0);
        return hipGetLastError();
    }
    if (cpad < 64)
        stage_launch<64>(input, in_kind, in_cstep, cin, pixels, cpad, vec, staged, tail, tail_q0,
                         stream);
    else
        stage_launch<128>(input, in_kind, in_cstep, cin, pixels, cpad, vec, staged, tail, tail_q0,
                          stream);
    return hipGetLastError();
}

hipError_t launch_conv3d_pack_weights(const float* weights, const Conv3dShape& s,
                                      uint16_t* packed, hipStream_t stream) {
    const long kp = conv3d_kp(s);
    const long total = (long)s.cout * kp;
    if (total <= 0) return hipSuccess;
    conv3d_pack_kernel<<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(weights, s, kp, total,
                                                                            packed);
    return hipGetLastError();
}

hipError_t launch_conv3d(const Conv3dShape& s, const uint16_t* memory, int mem,
                         size_t memory_bytes, const uint16_t* staged, size_t staged_bytes,
                         int frame_base, int shift, int height, int width, int ho, int wo,
                         int t0, int frames_out, const uint16_t* packed, const float* bias,
                         void* out, int out_kind, long out_cstep, float* part,
                         hipStream_t stream) {
    if (frames_out <= 0) return hipSuccess;
    const long m = (long)frames_out * ho * wo;
    const long kp = conv3d_kp(s);
    const bool small = s.cpad < 64;
    const int tw = conv3d_halo_width(s, wo);
    const bool halo = tw > 0;
    // the implicit-GEMM kernel reads memory frames in place only when each
    // 8-row DMA group lies in one output frame; the halo kernel's tiles
    // always do
    if (m > INT_MAX || staged_bytes >= 0x80000000ull || memory_bytes >= 0x80000000ull ||
        kp * 2 * s.cout >= 0x80000000l || s.cpad != conv3d_cpad(s.cin) || s.kh * s.kw > 32 ||
        (mem > 0 && !halo && (small || ((long)ho * wo) % 8 != 0)))
        return hipErrorInvalidValue;
    ConvArgs a;
    a.staged = staged;
    a.staged_bytes = (uint32_t)staged_bytes;
    a.memory = mem > 0 ? memory : staged;
    a.memory_bytes = mem > 0 ? (uint32_t)memory_bytes : 0u;
    a.mem = mem;
    a.packed = packed;
    a.kp = (int)kp;
    a.bias = bias;
    a.out = out;
    a.out_cstep = out_cstep;
    a.out_off = (long)t0 * ho * wo;
    a.out_kind = out_kind;
    const size_t esz = out_kind == 0 ? 4 : 2;
    a.vec_ok = out_cstep % 4 == 0 && a.out_off % 4 == 0 && ((uintptr_t)out % (4 * esz)) == 0;
    a.H = height;
    a.W = width;
    a.Ho = ho;
    a.Wo = wo;
    a.M = (int)m;
    a.cpad = s.cpad;
    a.cout = s.cout;
    a.kt = s.kt;
    a.kh = s.kh;
    a.kw = s.kw;
    a.st = s.st;
    a.dt = s.dt;
    a.sh = s.sh;
    a.sw = s.sw;
    a.dh = s.dh;
    a.dw = s.dw;
    a.ph = s.ph;
    a.pw = s.pw;
    a.shift = shift;
    a.fbase = frame_base;
    a.t0 = t0;
    a.ytiles = a.xtiles = 0;
    a.part = nullptr;
    a.part_split = 0;
    a.slots = nullptr;
    a.counters = nullptr;
    const int splits = part ? conv3d_k_split(s, m, wo) : 1;
    a.splits = splits;
    if (splits > 1) {
        a.part = part;
        a.part_split = (long)s.cout * m;
    }
    if (!a.part && conv3d_rgbin_ok(s, mem, ho, wo, height, width)) {
        // one band of rows per workgroup, one workgroup per CU
        const int strips = (wo + 127) / 128;
        const int cus = 256;
        const int bands = std::max(1, std::min(ho, cus / std::max(1, strips * frames_out)));
        const int band_rows = (ho + bands - 1) / bands;
        const int nb = (ho + band_rows - 1) / band_rows;
        const long blocks = (long)strips * nb * frames_out;
        if (blocks > INT_MAX) return hipErrorInvalidValue;
        // 16-byte output runs: 8-pixel aligned rows and frames
        const bool vec8 = ((uintptr_t)out % 16) == 0 && out_cstep % 8 == 0 && wo % 8 == 0 &&
                          a.out_off % 8 == 0 && (long)s.cout * out_cstep * 2 < 0x7fffffffL;
        if (out_kind == 1 && vec8)
            conv3d_rgbin_kernel<1, true><<<(unsigned)blocks, 512, 0, stream>>>(a, strips, nb, band_rows);
        else if (out_kind == 2 && vec8)
            conv3d_rgbin_kernel<2, true><<<(unsigned)blocks, 512, 0, stream>>>(a, strips, nb, band_rows);
        else if (out_kind == 1)
            conv3d_rgbin_kernel<1, false><<<(unsigned)blocks, 512, 0, stream>>>(a, strips, nb, band_rows);
        else if (out_kind == 2)
            conv3d_rgbin_kernel<2, false><<<(unsigned)blocks, 512, 0, stream>>>(a, strips, nb, band_rows);
        else
            conv3d_rgbin_kernel<0, false><<<(unsigned)blocks, 512, 0, stream>>>(a, strips, nb, band_rows);
        return hipGetLastError();
    }
    if (halo) {
        const int th = halo_tile_rows(s.cout <= 32 ? 32 : 128, tw);
        a.ytiles = (ho + th - 1) / th;
        a.xtiles = (wo + tw - 1) / tw;
        a.ntiles = s.cout <= 32 ? 1 : (s.cout + 127) / 128;
        const long tiles = (long)frames_out * a.ytiles * a.xtiles * a.ntiles;
        if (tiles > INT_MAX) return hipErrorInvalidValue;
        a.mtiles = (int)tiles;
        a.vec_ok = a.vec_ok && wo % 4 == 0;
        if (s.cout <= 32)
            tw == 128 ? launch_conv3d_halo<32, 128>(a, stream) : launch_conv3d_halo<32, 64>(a, stream);
        else
            tw == 128 ? launch_conv3d_halo<128, 128>(a, stream) : launch_conv3d_halo<128, 64>(a, stream);
        return hipGetLastError();
    }
    if (s.cout <= 32) {
        a.mtiles = (int)((m + 511) / 512);
        a.ntiles = 1;
        launch_conv3d_kernel<32>(a, stream);
    } else if (s.cout <= 128) {
        a.mtiles = (int)((m + 511) / 512);
        a.ntiles = (s.cout + 127) / 128;
        launch_conv3d_kernel<128>(a, stream);
    } else {
        a.mtiles = (int)((m + 255) / 256);
        a.ntiles = (s.cout + 255) / 256;
        if (a.part && !small) {
            // the split-k scratch of the stream (256x256 fp32 slots and
            // counters, one each per CU) when it holds a slot per workgroup;
            // otherwise the partial tiles go to part and a second pass
            size_t bytes = 0;
            void* base = nullptr;
            if (splitk_scratch_bytes(&bytes) == hipSuccess) {
                const size_t slot = (size_t)256 * 256 * sizeof(float);
                const long groups = (long)(bytes / (slot + sizeof(int)));
                if ((long)a.mtiles * a.ntiles * splits <= groups &&
                    stream_scratch(kScratchSplitK, stream, bytes, &base) == hipSuccess) {
                    a.slots = (float*)base;
                    a.counters = (int*)((char*)base + (size_t)groups * slot);
                }
            }
        }
        launch_conv3d_kernel<256>(a, stream);
    }
    if (a.part && !a.slots) {
        const long n = (long)s.cout * m;
        conv3d_reduce_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(
            a.part, splits, a.part_split, s.cout, (int)m, bias, out, out_kind, out_cstep,
            a.out_off);
    }
    return hipGetLastError();
}

}  // namespace s2
