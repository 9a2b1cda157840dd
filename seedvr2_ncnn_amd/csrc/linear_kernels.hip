// gfx950 kernels of the SharedLinear projection (src/seedvr2/shared_linear.cpp:83-96):
// y = act(x W^T + b) for the video and the text stream in one grouped launch.
//
// x [m][k] and W [n][k] are both k-contiguous, which is the natural operand
// layout of v_mfma_f32_32x32x16_bf16 (each lane supplies 8 consecutive k of
// one row of A and one column of B), so both tiles are staged in LDS
// unchanged.  fp32 activations are rounded to bf16 while they are staged.
#include <math.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "awa_index.h"
#include "awa_kernels.h"
#include "s2_device.h"
#include "stream_scratch.h"


namespace s2 {

namespace {

__device__ __forceinline__ uint4 load_chunk(const uint16_t* p) {
    return *reinterpret_cast<const uint4*>(p);
}

__device__ __forceinline__ uint4 load_chunk(const _Float16* p) {
    const uint4 raw = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    uint16_t h[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h[2 * i] = f32_to_bf16((float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xffffu)));
        h[2 * i + 1] = f32_to_bf16((float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16)));
    }
    return pack8_bf16(h);
}

// one output element of type YK (0 fp32, 1 bf16, 2 fp16)
template <int YK>
__device__ __forceinline__ void store1(void* y, long idx, float v) {
    if (YK == 1)
        ((uint16_t*)y)[idx] = f32_to_bf16(v);
    else if (YK == 2)
        ((_Float16*)y)[idx] = f32_to_f16(v);
    else
        ((float*)y)[idx] = v;
}

__device__ __forceinline__ uint4 load_chunk(const float* p) {
    float v[8];
    load8(p, v);
    uint16_t h[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = f32_to_bf16(v[i]);
    return pack8_bf16(h);
}

// erf-GELU, 0.5 x (1 + erf(x / sqrt 2)) = max(x, 0) - |x| Q(|x|) with
// Q(a) = 0.5 erfc(a / sqrt 2): both signs reduce to one fma, and for x < 0
// the result is the product -|x| Q directly, without cancellation.  erfc is
// Abramowitz & Stegun 7.1.26, erfc(z) = (a1 t + ... + a5 t^5) e^(-z^2),
// t = 1 / (1 + p z), |error| <= 1.5e-7; the factor 0.5 is folded into a1..a5
// and e^(-z^2) = 2^(-w^2) with w = z sqrt(log2 e).
__device__ __forceinline__ float gelu(float x) {
    constexpr float kSqrtLog2e = 1.2011224087864498f;
    const float ax = fabsf(x);
    const float w = ax * (0.70710678118654752f * kSqrtLog2e);
    const float t = __builtin_amdgcn_rcpf(fmaf(w, 0.3275911f / kSqrtLog2e, 1.f));
    const float poly =
        t * (0.5f * 0.254829592f +
             t * (0.5f * -0.284496736f +
                  t * (0.5f * 1.421413741f + t * (0.5f * -1.453152027f + t * (0.5f * 1.061405429f)))));
    const float q = poly * __builtin_amdgcn_exp2f(-w * w);   // Q(|x|)
    return fmaf(-ax, q, fmaxf(x, 0.f));
}

}  // namespace

// Block tile 128x128, k-step 64, four waves in a 2x2 grid of 64x64 wave tiles
// (2x2 MFMA 32x32 accumulators per wave).  LDS double buffered, rows padded
// by 16 bytes against bank conflicts.
template <typename TX, int YK, int ACT>
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
                if (ACT == S2_ACT_GELU) v = gelu(v);
                store1<YK>(y, (long)row * n + col, v);
            }
    }
}

// ---------------------------------------------------------------------------
// Large-tile path for bf16 activations with k % 64 == 0.
//
// Block tile 256x256 with eight waves, two per SIMD, in a 2 (m) x 4 (n) grid
// of 128x64 wave tiles (4x2 MFMA 32x32x16 accumulators = 128 fp32 per lane).
// The two waves of a SIMD ping-pong: one issues a whole 64-k step of MFMAs
// from fragment registers while the other reads its next step's fragments
// from LDS (the main loop below).  The operands stream through two 64-k LDS
// stages (64 KB each) filled by buffer_load_dwordx4 ... lds (global -> LDS,
// no VGPR staging).  The buffer descriptors bound each tile to its valid
// rows, so ragged m and n read zeros.  LDS rows are 128 bytes; 16-byte chunk
// c of row r is stored at position c ^ (((r >> 1) ^ ((r & 1) << 2)) & 7), so
// the rows one ds_read_b128 phase touches land on distinct banks.  The bf16
// epilogue adds the bias and activation in fp32, converts with
// v_cvt_pk_bf16_f32, assembles the 256x256 tile in LDS and writes it out as
// 16-byte row chunks.
//
// Tail balancing.  When the tile count leaves the last wave of workgroups
// partly idle, the tiles of that wave are not given one workgroup each:
// their 64-k iterations are dealt out evenly to sk_groups workgroups, each
// taking one contiguous range of (tile, k-iteration) pairs (with sk_groups
// a multiple of the tile count, every range lies inside one tile).  A tile finished by one workgroup takes the normal epilogue; a tile
// split between workgroups has every part store its fp32 accumulators to a
// per-workgroup slot and bump the tile's arrival counter, and the last part
// to arrive sums all the slots in workgroup order (so the result does not
// depend on which part arrives last), runs the epilogue and resets the
// counter.  No workgroup waits on another.
namespace {

__device__ __forceinline__ int lds_swizzle(int r) { return ((r >> 1) ^ ((r & 1) << 2)) & 7; }

// Sum over aligned groups of N lanes (N = 8 or 16) by DPP lane moves: quad
// permutations [1,0,3,2] and [2,3,0,1], then the half-row and row mirrors.
// Each step adds the value of a lane of the other half of the group, which
// after the previous steps holds the same partial sum as lane ^ (N/2), so
// the result equals the shuffle-xor reduction over masks 1, 2, 4, 8 bit for
// bit (and needs no LDS round trip).
template <int N>
__device__ __forceinline__ float row_sum(float x) {
    static_assert(N == 8 || N == 16, "row_sum over 8 or 16 lanes");
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, false));
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x141, 0xF, 0xF, false));
    if (N == 16) x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x140, 0xF, 0xF, false));
    return x;
}

constexpr int kSlotFloats = 128 * 512;   // one workgroup's accumulators

// Cache policy of the slot stores and loads: sc0 sc1, coherent across the
// XCDs' L2s (stores write through, loads do not hit a stale L2 line), so the
// parts of a tile can meet without cache-wide writeback or invalidation.
constexpr int kCoherent = 1 | 16;
// nt: a streaming store, not kept in the L2
constexpr int kNonTemporal = 2;
// word 3 of a raw (untyped, stride 0) buffer descriptor
constexpr int kRawBufferFormat = 0x00020000;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

}  // namespace

struct SkTail {
    int dp_tiles;      // tiles [0, dp_tiles): one workgroup each
    int sk_tiles;      // tiles [dp_tiles, dp_tiles + sk_tiles): shared out along k
    int sk_groups;     // workgroups sharing them: a multiple of sk_tiles, so that
                       // each workgroup's k range lies inside one tile
    float* slots;      // [sk_groups][kSlotFloats] partial accumulators
    int* counters;     // [sk_tiles] arrivals; zero between launches
};

// The fused QKV projection of the attention layer (AWA = head dim): the
// tile rows are the plan's QKV row space (video tokens in window order, then
// the text tokens), gathered from the source-ordered activations, and the
// epilogue writes the attention workspace directly: RMS-normalised and
// rotated Q and K rows [head][seg_total][D] and V transposed [head][D][seg_total]
// (adaptive_window_attention.cpp:886-927), text tokens to their staging rows.
struct AwaQkvArgs {
    const QkvRow* row_table;  // the plan's rows, [mtiles * 256]
    int inner;                // heads * head_dim
    long seg_total;           // row pitch of Q, K and V^T
    long seg_text;            // first text staging row
    const float* norm;        // [4][D]: video q, video k, text q, text k
    const float2* rope;       // (cos, sin) [position][pairs]
    int pairs;
    float eps;
    int official_bf16;
    uint16_t* q;
    uint16_t* k;
    uint16_t* vt;
};

template <int YK, int ACT, int AWA = 0, int RES = 0>
__global__ __launch_bounds__(512, 1) void shared_linear_256_kernel(
    const uint16_t* __restrict__ x0, int m0, const uint16_t* __restrict__ x1, int m1,
    const uint16_t* __restrict__ wgt, const float* __restrict__ bias, int n, int k,
    void* __restrict__ y0, void* __restrict__ y1, int mv, int mtiles, int ntiles, SkTail sk,
    AwaQkvArgs awa, LinearResidual res) {
    constexpr int BM = 256, BN = 256, BK = 64;
    constexpr int TB = BM * BK * 2;   // 32 KB per operand per stage
    constexpr int SB = 2 * TB;        // 64 KB per stage
    constexpr int RB = BK * 2;        // LDS row bytes
    constexpr int EP = BN * 2 + 16;   // epilogue LDS row pitch (bytes)
    constexpr int LDS_BYTES = 2 * SB > BM * EP ? 2 * SB : BM * EP;
    constexpr int GROUP = 4;   // row-tiles per raster group (4 measured 1-3% faster than 8 or 16)
    __shared__ __attribute__((aligned(1024))) uint8_t lds[LDS_BYTES];
    __shared__ int arrival;
    __shared__ QkvRow qrows[AWA ? BM : 1];
    // fused QKV: byte offsets of the gathered A rows of every lane of the
    // four A-loading waves, eight per lane (read back at each DMA issue:
    // the main loop has no registers to spare for them)
    __shared__ uint4 goff_lds[AWA ? 4 * 64 * 2 : 1];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
    const int l32 = lane & 31;
    const int g = lane >> 5;
    const int wm = wave >> 2;
    const int wn = wave & 3;
    const int nk = k / BK;
    const int sw = lds_swizzle(l32);   // fragment rows differ from l32 by multiples of 32
    const uint32_t lds_base = (uint32_t)(uintptr_t)lds;

    // The two token streams share one row space: video row r is row r, text
    // row r is row mv + r (mv = m0 rounded up to a multiple of 8), so the
    // tile holding the video tail also holds the first text rows.  Every
    // 8-row DMA group lies in one stream.
    int row0, col0;   // the current tile
    auto set_tile = [&](int t) {
        // grouped raster: GROUP m-tiles share each sweep over the n-tiles
        const int group_size = GROUP * ntiles;
        const int first_m = (t / group_size) * GROUP;
        const int gm = min(mtiles - first_m, GROUP);
        const int mt = first_m + (t % group_size) % gm;
        const int nt = (t % group_size) / gm;
        row0 = mt * BM;
        col0 = nt * BN;
    };
    // output row of tile row rl, or null past either stream
    // output row pitch: n, or n / 2 for SwiGLU, whose weight has a gate and
    // an up row per output column
    const int ny = ACT == S2_ACT_SWIGLU ? n / 2 : n;
    auto out_row = [&](int rl) -> void* {
        const int r = row0 + rl;
        if (r < m0) return (char*)y0 + (long)r * ny * (YK ? 2 : 4);
        if (r >= mv && r < mv + m1) return (char*)y1 + (long)(r - mv) * ny * (YK ? 2 : 4);
        return nullptr;
    };

    // Fused QKV projection: the current tile's rows of the plan's row table
    // (one row per thread of the first four waves).
    auto build_rows = [&]() {
        if constexpr (AWA != 0) {
            if (tid < BM) qrows[tid] = awa.row_table[row0 + tid];
        }
    };

    f32x16 acc[4][2];

    // Thread coordinates for the epilogues, derived from an opaque copy of
    // the thread index: addresses computed from them are not hoisted above
    // the main loop, where every register is taken and hoisted values would
    // be spilled and reloaded one scratch round trip at a time.
    struct EpiIds {
        int tid, l32, g, wm, wn;
    };
    auto epi_ids = [&]() {
        EpiIds e;
        int t = tid;
        asm volatile("" : "+v"(t));
        const int w = __builtin_amdgcn_readfirstlane(t >> 6);
        e.tid = t;
        e.l32 = t & 31;
        e.g = (t >> 5) & 1;
        e.wm = w >> 2;
        e.wn = w & 3;
        return e;
    };

    // acc + bias (and the activation) of this wave's rows of the tile, as
    // 16-bit values in the LDS staging rows (pitch EP); the 16-bit outputs
    // of the plain epilogue
    auto stage_own_rows = [&]() {
        if constexpr (YK != 0 && AWA == 0 && ACT != S2_ACT_SWIGLU) {
            const EpiIds ei = epi_ids();
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int cl = ei.wn * 64 + 32 * j + ei.l32;
                const float bv = (bias && col0 + cl < n) ? bias[col0 + cl] : 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        float v = acc[i][j][r] + bv;
                        if (ACT == S2_ACT_GELU) v = gelu(v);
                        const int rl = ei.wm * 128 + 32 * i + 8 * (r >> 2) + 4 * ei.g + (r & 3);
                        if (YK == 2)
                            *(_Float16*)(lds + rl * EP + cl * 2) = f32_to_f16(v);
                        else
                            *(__bf16*)(lds + rl * EP + cl * 2) = (__bf16)v;
                    }
            }
        }
    };

    // acc = sum over 64-k iterations [kb, ke) of the current tile.
    //
    // Ping-pong main loop.  The two waves of each SIMD (wave w and w + 4:
    // group 0 owns tile rows 0-127, group 1 rows 128-255) take turns: one
    // issues the 32 MFMAs of a whole 64-k step from fragment registers while
    // the other reads its fragments of the next step from LDS, so the matrix
    // core never waits on an LDS read.  Every phase ends at a workgroup
    // barrier; group 1 runs one phase behind group 0.  The DMA of a step is
    // split between the groups: group 1 loads the B rows into the stage it
    // has just finished reading (it is that stage's last reader), group 0 the
    // A rows one phase later; each waits for its DMA two phases after issuing
    // it, before the barrier that opens the stage to its first reader.
    //
    //   phase     2s                        2s + 1
    //   group 0   DMA A of step s + 1,      MFMAs of step s,
    //             read step s               wait for its DMA
    //   group 1   MFMAs of step s - 1       read step s, wait for its DMA of
    //                                       step s + 1, DMA B of step s + 2
    auto mainloop = [&](int kb, int ke, bool early) {
        const int grp = wave >> 2;
        const int wq = wave & 3;
        // plain: the tile's rows of each stream; fused QKV: whole streams,
        // each DMA lane addressing its gathered row
        const i32x4 rav = AWA ? wave_uniform(buffer_rsrc(x0, (uint32_t)((long)m0 * k * 2)))
                              : wave_uniform(buffer_rsrc(
                                    x0 + (long)row0 * k, (uint32_t)(max(min(m0 - row0, BM), 0) * k * 2)));
        const i32x4 rat =
            AWA ? wave_uniform(buffer_rsrc(x1, (uint32_t)((long)m1 * k * 2)))
                : wave_uniform(buffer_rsrc(x1 + (long)(row0 - mv) * k,
                                           (uint32_t)(row0 + BM > mv ? min(mv + m1 - row0, BM) * k * 2 : 0)));
        const int wrow = __builtin_amdgcn_readfirstlane(row0 + wq * 64);
        const i32x4 rb =
            wave_uniform(buffer_rsrc(wgt + (long)col0 * k, (uint32_t)(min(n - col0, BN) * k * 2)));
        // Wave wq of a group fills LDS rows 64 wq .. 64 wq + 63 of its operand
        // (group 0: A, group 1: B) with 8 DMA instructions of 8 rows.  Row
        // r + 8j has the swizzle of row r with bit 2 flipped for odd j, so two
        // offsets serve all eight.
        const int row_a = wq * 64 + (lane >> 3);
        const uint32_t vrow = (uint32_t)(row_a * k * 2);
        const uint32_t voff_even = vrow + (((lane & 7) ^ lds_swizzle(row_a)) * 16);
        const uint32_t voff_odd = vrow + (((lane & 7) ^ lds_swizzle(row_a) ^ 4) * 16);
        // fused QKV: byte offsets of this lane's eight gathered A rows (a gap
        // or padding row points one row past its stream: the DMA reads zeros)
        if constexpr (AWA != 0) {
            if (grp == 0) {
                uint32_t go[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int src = qrows[row_a + 8 * j].src;
                    const int rr = src >= 0 ? src : (wrow + j * 8 < mv ? m0 : m1);
                    go[j] = (uint32_t)rr * (uint32_t)(k * 2) +
                            (uint32_t)((((lane & 7) ^ lds_swizzle(row_a) ^ ((j & 1) << 2))) * 16);
                }
                // lanes 16 bytes apart in each half, so a 16-lane read
                // phase covers all banks once
                goff_lds[wq * 64 + lane] = make_uint4(go[0], go[1], go[2], go[3]);
                goff_lds[256 + wq * 64 + lane] = make_uint4(go[4], go[5], go[6], go[7]);
            }
        }
        auto issue = [&](int stage, int kt, int operand) {
            const uint32_t soff = __builtin_amdgcn_readfirstlane((uint32_t)(kt * BK * 2));
            const uint32_t st = lds_base + stage * SB + operand * TB + wq * 8 * 1024;
            uint32_t go[8];
            if constexpr (AWA != 0) {
                if (!operand) {
                    const uint4 g0 = goff_lds[wq * 64 + lane];
                    const uint4 g1 = goff_lds[256 + wq * 64 + lane];
                    go[0] = g0.x; go[1] = g0.y; go[2] = g0.z; go[3] = g0.w;
                    go[4] = g1.x; go[5] = g1.y; go[6] = g1.z; go[7] = g1.w;
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                uint32_t vo = ((j & 1) ? voff_odd : voff_even) + (uint32_t)(j * 8 * k * 2);
                if constexpr (AWA != 0)
                    if (!operand) vo = go[j];
                lds_dma16(operand ? rb : (wrow + j * 8 < mv ? rav : rat),
                          __builtin_amdgcn_readfirstlane(st + j * 1024), vo, soff);
            }
        };
        bf16x8 fa[4][4], fb[4][2];
        auto read_step = [&](int stage) {
            const uint8_t* st = lds + stage * SB;
#pragma unroll
            for (int kk = 0; kk < BK / 16; ++kk) {
                const int pc = ((2 * kk + g) ^ sw) * 16;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    fa[kk][i] = as_bf16x8(*(const uint4*)(st + (wm * 128 + 32 * i + l32) * RB + pc));
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    fb[kk][j] =
                        as_bf16x8(*(const uint4*)(st + TB + (wn * 64 + 32 * j + l32) * RB + pc));
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
        const int steps = ke - kb;
        // steps 0 and 1: group 0 loads A, group 1 B
        issue(0, kb, grp);
        if (steps > 1) issue(1, kb + 1, grp);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        barrier();
        if (grp == 1) barrier();
#pragma unroll 1
        for (int s = 0; s < steps; ++s) {
            // memory phase
            if (grp == 0 && s >= 1 && s + 1 < steps) issue((s + 1) & 1, kb + s + 1, 0);
            read_step(s & 1);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (grp == 1) {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // B of step s + 1
                if (s + 2 < steps) issue(s & 1, kb + s + 2, 1);
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
            if (grp == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // A of step s + 1
            barrier();
        }
        // group 0's barrier matching group 1's last MFMA phase; with an early
        // epilogue group 0 stages its rows first (epilogue)
        if (grp == 0 && !early) barrier();
    };

    // Fused QKV epilogue.  The tile's 256 columns lie in one of q, k, v
    // (inner is a multiple of 256) and cover 256 / D heads from hbase.  The
    // tile is first rounded to bf16 (acc + bias, nearest even: the values a
    // bf16 QKV blob would hold) and staged in LDS, so that every value the
    // attention then reads is bit-identical to what the separate projection
    // and the attention prologue (awa_prologue_kernel) produce.
    //   q, k: row-major staging; D/8 threads per (row, head) hold 8
    //     channels each, reduce the sum of squares with DPP lane moves, apply
    //     rms_norm (:510-519) with the video or text weights, then
    //     apply_mm_rope (:521-543) at the row's position, in the prologue's
    //     fp32 operation order, and store 16 bytes of the head's row.
    //   v: transposed staging (channel rows of the 256 tile rows); every
    //     thread then stores 4-byte key pairs of V^T.  Window runs and the
    //     text rows start at even rows of the row space and segments at
    //     even workspace rows, so each pair of tile rows is one aligned pair
    //     of workspace keys.
    auto awa_epilogue = [&]() {
        if constexpr (AWA != 0) {
#pragma clang fp contract(off)
            constexpr int D = AWA;
            constexpr int SP = BN * 2 + 16;   // bytes per staged row
            // transposed (v) staging: 8-byte writes of 32 lanes to 32 rows;
            // a pitch of 130 dwords puts them on distinct bank pairs
            constexpr int SPV = BN * 2 + 8;
            // an opaque copy of the thread index: nothing the epilogue derives
            // from it is hoisted above the main loop, where every register is
            // taken
            const EpiIds ei = epi_ids();
            const int etid = ei.tid;
            const int part = col0 / awa.inner;   // 0 q, 1 k, 2 v
            const int hbase = (col0 - part * awa.inner) / D;
            __syncthreads();   // every wave is done reading the last stage
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int cl = ei.wn * 64 + 32 * j + ei.l32;
                const float bv = bias ? bias[col0 + cl] : 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int q4 = 0; q4 < 4; ++q4) {
                        // registers 4 q4 .. 4 q4 + 3: rows rl .. rl + 3 of column cl
                        const int rl = ei.wm * 128 + 32 * i + 8 * q4 + 4 * ei.g;
                        uint16_t hv[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            hv[e] = __builtin_bit_cast(uint16_t, (__bf16)(acc[i][j][4 * q4 + e] + bv));
                        if (part < 2) {
#pragma unroll
                            for (int e = 0; e < 4; ++e) *(uint16_t*)(lds + (rl + e) * SP + cl * 2) = hv[e];
                        } else {
                            *(uint2*)(lds + cl * SPV + rl * 2) =
                                make_uint2(hv[0] | ((uint32_t)hv[1] << 16), hv[2] | ((uint32_t)hv[3] << 16));
                        }
                    }
            }
            __syncthreads();
            if (part < 2) {
                constexpr int TPR = D / 8;        // threads per (row, head)
                uint16_t* dst = part == 0 ? awa.q : awa.k;
                const int ch = etid & 31;          // 8-channel chunk of the 256 columns
                const int hl = ch * 8 / D;
                const int d0 = ch * 8 - hl * D;
                float wv[8], wt[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    wv[i] = awa.norm[part * D + d0 + i];
                    wt[i] = awa.norm[(2 + part) * D + d0 + i];
                }
                // RoPE slots of this thread's four channel pairs: pair
                // (2p, 2p+1) of axis a lies in [a*2P, (a+1)*2P); 6P <= D.
                // The four pairs are consecutive, so they lie on axis axA
                // from pair pairA on, then (pairs split.. of a chunk that
                // crosses an axis boundary) on axis axA + 1 from pair 0.  A
                // row's position on axis a is bits [16(a & 1), +16) of
                // position word a / 2.
                const int P = awa.pairs;
                bool rot[4];
#pragma unroll
                for (int pp = 0; pp < 4; ++pp) rot[pp] = d0 + 2 * pp < 6 * P;
                const int axA = P > 0 ? min(d0 / (2 * P), 2) : 0;
                const int pairA = rot[0] ? (d0 - axA * 2 * P) >> 1 : 0;
                const int split = rot[0] ? min(P - pairA, 4) : 4;
                const int axB = min(axA + 1, 2);
                // (cos, sin) of the four pairs at a row's position, without
                // branches (so that the wait for these loads is exact): gap
                // rows hold position 0, and a pair past the rotated width
                // reads an entry at most three past its row's (the table has
                // kRopePad entries of slack) and does not use it.  The loads
                // of pass p + 1 are issued before pass p computes.
                const char* rope_b = reinterpret_cast<const char*>(awa.rope);
                auto rope_load = [&](const QkvRow& ri, float2 (&cs)[4]) {
                    const uint32_t wa = axA == 2 ? ri.pos2 : ri.pos01;
                    const uint32_t wb = axB == 2 ? ri.pos2 : ri.pos01;
                    const uint32_t posA = (wa >> (16 * (axA & 1))) & 0xffff;
                    const uint32_t posB = (wb >> (16 * (axB & 1))) & 0xffff;
                    // byte offsets of pair 0 of the chunk on each axis
                    const uint32_t offA = (__umul24(posA, (uint32_t)P) + pairA) * 8;
                    const uint32_t offB = __umul24(posB, (uint32_t)P) * 8 - split * 8;
#pragma unroll
                    for (int pp = 0; pp < 4; ++pp) {
                        const uint32_t off = (pp < split ? offA : offB) + 8 * pp;
                        cs[pp] = *reinterpret_cast<const float2*>(rope_b + off);
                    }
                };
                // The results of all passes stay in registers (the
                // accumulators are dead by now) and are stored after the
                // loop, so the loop holds loads only and each pass waits for
                // its own loads, not for earlier stores.
                constexpr int PASSES = BM / 16;
                uint4 res[PASSES];
                // Only the tile holding the first text row (the row space is
                // the video rows in window order, then the text rows) selects
                // between the video and text weights per row.
                auto passes = [&](auto text_tag) {
                constexpr bool TEXT = decltype(text_tag)::value;
                QkvRow ri_next = qrows[etid >> 5];
                float2 cs_next[4];
                rope_load(ri_next, cs_next);
#pragma unroll
                for (int pass = 0; pass < PASSES; ++pass) {
                    const int rl = pass * 16 + (etid >> 5);
                    const QkvRow ri = ri_next;
                    float2 cs[4];
#pragma unroll
                    for (int pp = 0; pp < 4; ++pp) cs[pp] = cs_next[pp];
                    if (pass + 1 < PASSES) {
                        ri_next = qrows[rl + 16];
                        rope_load(ri_next, cs_next);
                    }
                    const int kind = ri.pos2 >> 16;
                    const uint4 raw = *(const uint4*)(lds + rl * SP + ch * 16);
                    const uint32_t wd[4] = {raw.x, raw.y, raw.z, raw.w};
                    float x[8];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        x[2 * i] = __uint_as_float(wd[i] << 16);
                        x[2 * i + 1] = __uint_as_float(wd[i] & 0xffff0000u);
                    }
                    float ss = x[0] * x[0];
#pragma unroll
                    for (int i = 1; i < 8; ++i) ss = fmaf(x[i], x[i], ss);
                    ss = row_sum<TPR>(ss);
                    const float inv = __builtin_amdgcn_rsqf(ss / (float)D + awa.eps);
                    const bool video = !TEXT || kind == 1;
#pragma unroll
                    for (int i = 0; i < 8; ++i) x[i] = x[i] * inv * (video ? wv[i] : wt[i]);
#pragma unroll
                    for (int pp = 0; pp < 4; ++pp) {
                        if (rot[pp]) {
                            const float a0 = x[2 * pp], a1 = x[2 * pp + 1];
                            x[2 * pp] = fmaf(a0, cs[pp].x, -(a1 * cs[pp].y));
                            x[2 * pp + 1] = fmaf(a0, cs[pp].y, a1 * cs[pp].x);
                        }
                    }
                    if (awa.official_bf16) {
                        uint16_t hb[8];
#pragma unroll
                        for (int i = 0; i < 8; ++i) hb[i] = round_bf16_ref_bits(x[i]);
                        res[pass] = pack8_bf16(hb);
                    } else {
                        res[pass] = cvt8_bf16(x);
                    }
                }
                };
                if (row0 + BM > mv)
                    passes(std::true_type{});
                else
                    passes(std::false_type{});
#pragma unroll
                for (int pass = 0; pass < PASSES; ++pass) {
                    const QkvRow ri = qrows[pass * 16 + (etid >> 5)];
                    if (ri.pos2 >> 16)
                        __builtin_nontemporal_store(
                            __builtin_bit_cast(u32x4, res[pass]),
                            (u32x4*)(dst + ((long)(hbase + hl) * awa.seg_total + ri.dest) * D + d0));
                }
            } else {
                // thread t stores key pair t % 128 (tile rows 2q, 2q + 1) of
                // channels t / 128 + 4c
                const int qp = etid & 127;
                const QkvRow ri = qrows[2 * qp];
                if (ri.pos2 >> 16) {
                    uint16_t* base = awa.vt + (long)hbase * D * awa.seg_total + ri.dest;
#pragma unroll 8
                    for (int c = 0; c < 64; ++c) {
                        const int cl = (etid >> 7) + 4 * c;
                        const uint32_t v = *(const uint32_t*)(lds + cl * SPV + qp * 4);
                        __builtin_nontemporal_store(v, (uint32_t*)(base + (long)cl * awa.seg_total));
                    }
                }
            }
        }
    };

    // SwiGLU: the weight's rows come in blocks of 256, the first 128 gate
    // rows and the next 128 up rows of the same 128 output columns, so a
    // tile's columns 0-127 are gates and 128-255 ups of output columns
    // col0/2 .. col0/2 + 127.  acc + bias is staged as fp32 in two halves of
    // 128 rows; each thread then forms silu(g) * u for 4 columns of a row.
    auto swiglu_epilogue = [&]() {
        if constexpr (ACT == S2_ACT_SWIGLU) {
            const EpiIds ei = epi_ids();
            constexpr int EF = BN * 4 + 16;   // fp32 row pitch (bytes)
            const int oc0 = col0 / 2;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                __syncthreads();   // the stage (h = 0) or the previous half is no longer read
                if (ei.wm == h) {
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const int cl = ei.wn * 64 + 32 * j + ei.l32;
                        const float bv = bias ? bias[col0 + cl] : 0.f;
#pragma unroll
                        for (int i = 0; i < 4; ++i)
#pragma unroll
                            for (int r = 0; r < 16; ++r) {
                                const int rl = 32 * i + 8 * (r >> 2) + 4 * ei.g + (r & 3);
                                *(float*)(lds + rl * EF + cl * 4) = acc[i][j][r] + bv;
                            }
                    }
                }
                __syncthreads();
#pragma unroll 2
                for (int it = 0; it < 8; ++it) {
                    const int idx = it * 512 + ei.tid;
                    const int rl = idx >> 5;
                    const int c4 = (idx & 31) * 4;
                    const f32x4 gv = *(const f32x4*)(lds + rl * EF + c4 * 4);
                    const f32x4 uv = *(const f32x4*)(lds + rl * EF + (c4 + 128) * 4);
                    float o[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        // silu(g) = g / (1 + e^-g), e^-g = 2^(-g log2 e)
                        const float gg = gv[e];
                        const float sig = __builtin_amdgcn_rcpf(
                            1.f + __builtin_amdgcn_exp2f(-gg * 1.4426950408889634f));
                        o[e] = gg * sig * uv[e];
                    }
                    void* yr = out_row(h * 128 + rl);
                    const int col = oc0 + c4;
                    if (!yr || col >= ny) continue;
                    if (YK == 0) {
                        const f32x4 ov = {o[0], o[1], o[2], o[3]};
                        __builtin_nontemporal_store(ov, (f32x4*)((float*)yr + col));
                    } else {
                        uint16_t hb[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            hb[e] = YK == 2 ? __builtin_bit_cast(uint16_t, f32_to_f16(o[e]))
                                            : __builtin_bit_cast(uint16_t, (__bf16)o[e]);
                        typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
                        const u32x2 hv = {hb[0] | ((uint32_t)hb[1] << 16),
                                          hb[2] | ((uint32_t)hb[3] << 16)};
                        __builtin_nontemporal_store(hv, (u32x2*)((uint16_t*)yr + col));
                    }
                }
            }
        }
    };

    // Residual epilogue: thread (sub, ch) holds the bf16 projection of
    // columns col0 + 8 ch .. + 7 of tile rows sub + 16 c; all residual loads
    // go out before the first store.  out may be x: each element is read and
    // written by one thread.
    auto residual_store = [&](const u32x4 (&sv)[16], int sub, int ch) {
        if constexpr (RES != 0) {
#pragma clang fp contract(off)
            const int col = col0 + ch * 8;
            if (col >= n) return;
            int cur = -1;
            float g[8];
            // two halves of eight rows: the half's residual loads (raw, two
            // 16-byte chunks for fp32, one for 16-bit types) go out first
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                int loc[8];   // stream << 30 | row within the stream; -1: no row
                u32x4 raw[8][2];
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const int r = row0 + 16 * (8 * h + c) + sub;
                    const int st = r < m0 ? 0 : (r >= mv && r < mv + m1 ? 1 : -1);
                    const int local = st == 0 ? r : r - mv;
                    loc[c] = st < 0 ? -1 : (st << 30) | local;
                    if (st < 0) continue;
                    const long e = (long)local * n + col;
                    const void* xs = st ? res.x[1] : res.x[0];
                    if (res.x_kind == 0) {
                        raw[c][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>((const float*)xs + e));
                        raw[c][1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>((const float*)xs + e + 4));
                    } else {
                        raw[c][0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>((const uint16_t*)xs + e));
                    }
                }
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    if (loc[c] < 0) continue;
                    const int st = loc[c] >> 30;
                    const int local = loc[c] & 0x3fffffff;
                    // the row's sample: the number of its stream's row ends
                    // at or below it (the ends are read with uniform indices)
                    int b = 0;
                    for (int j = 0; j + 1 < res.rows.batch; ++j) {
                        const int e = st ? res.rows.end[kAdaMaxBatch + j] : res.rows.end[j];
                        if (local >= e) b = j + 1;
                    }
                    const int key = st * kAdaMaxBatch + b;
                    if (key != cur) {
                        cur = key;
                        const float* ga = res.gate + (long)b * n + col;
                        const float* gs = st ? res.gate_s[1] : res.gate_s[0];
#pragma unroll
                        for (int i = 0; i < 8; ++i) g[i] = gs ? ga[i] + gs[col + i] : ga[i];
                    }
                    float xv[8];
                    if (res.x_kind == 0) {
#pragma unroll
                        for (int i = 0; i < 8; ++i) xv[i] = __uint_as_float(raw[c][i >> 2][i & 3]);
                    } else {
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            const uint16_t hv = (uint16_t)(raw[c][0][i >> 1] >> (16 * (i & 1)));
                            xv[i] = res.x_kind == 1 ? bf16_to_f32(hv)
                                                    : (float)__builtin_bit_cast(_Float16, hv);
                        }
                    }
                    const u32x4 yw = sv[8 * h + c];
                    float o[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const uint32_t w = yw[i >> 1];
                        const float y = __uint_as_float(i & 1 ? (w & 0xffff0000u) : (w << 16));
                        const float p = y * g[i];
                        o[i] = xv[i] + p;
                    }
                    const long e = (long)local * n + col;
                    void* os = st ? res.out[1] : res.out[0];
                    if (res.x_kind == 0) {
                        u32x4 a, b2;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            a[i] = __float_as_uint(o[i]);
                            b2[i] = __float_as_uint(o[4 + i]);
                        }
                        __builtin_nontemporal_store(a, reinterpret_cast<u32x4*>((float*)os + e));
                        __builtin_nontemporal_store(b2, reinterpret_cast<u32x4*>((float*)os + e + 4));
                    } else {
                        store4(os, e, o[0], o[1], o[2], o[3], res.x_kind);
                        store4(os, e + 4, o[4], o[5], o[6], o[7], res.x_kind);
                    }
                }
            }
        }
    };

    // y tile = act(acc + bias)
    auto epilogue = [&](bool early) {
        if constexpr (AWA != 0) {
            awa_epilogue();
            return;
        }
        if constexpr (ACT == S2_ACT_SWIGLU) {
            swiglu_epilogue();
            return;
        }
        const EpiIds ei = epi_ids();
        if (YK && (n & 7) == 0) {
            if constexpr (RES == 0) {
                // Thread t of group g (waves 4g .. 4g + 3) stores 16-byte
                // chunk t%32 of rows 128g + t/32 + 8c, all sixteen LDS reads
                // before the first store.  Each stream's rows of the tile go
                // through a buffer descriptor bounded by those rows, so the
                // range check drops a row past its stream, and a chunk past
                // n (an offset with bit 31 set: offsets are below 2^31, the
                // launcher checks 256 rows of output), without a branch per
                // store; a wave's two rows lie in one 8-row group, hence in
                // one stream.  The output is not read again by this launch:
                // the stores are non-temporal, leaving the L2 to the operand
                // tiles.
                //
                // Early schedule (a whole tile): group 1's last MFMA phase
                // reads no stage (its fragments are in registers, no DMA is
                // in flight), so group 0 stages its rows 0-127 meanwhile and
                // meets group 1 at the end of that phase (mainloop left that
                // barrier to here); then group 0 stores while group 1 stages
                // rows 128-255, and group 1 stores last.  Otherwise both
                // groups stage, then store.  The barriers are plain s_barrier:
                // group 0's stores need no wait before group 1 goes on.
                const int pitch = ny * 2;
                const __amdgpu_buffer_rsrc_t rs0 = __builtin_amdgcn_make_buffer_rsrc(
                    (char*)y0 + (long)row0 * pitch, (short)0, max(min(m0 - row0, BM), 0) * pitch,
                    kRawBufferFormat);
                const __amdgpu_buffer_rsrc_t rs1 = __builtin_amdgcn_make_buffer_rsrc(
                    (char*)y1 + (long)(row0 - mv) * pitch, (short)0,
                    row0 + BM > mv ? min(mv + m1 - row0, BM) * pitch : 0, kRawBufferFormat);
                const int g0 = ei.wm;
                const int t = ei.tid - 256 * g0;
                const int ch = t & 31;
                const int sub = t >> 5;
                const int lw = ei.wn;   // wave within the group
                const uint32_t drop = col0 + ch * 8 < n ? 0u : 0x80000000u;
                auto store_rows = [&]() {
                    u32x4 sv[16];
#pragma unroll
                    for (int c = 0; c < 16; ++c)
                        sv[c] = *(const u32x4*)(lds + (128 * g0 + 8 * c + sub) * EP + ch * 16);
#pragma unroll
                    for (int c = 0; c < 16; ++c) {
                        const int rl = 128 * g0 + 8 * c + sub;
                        const uint32_t off = (uint32_t)(rl * pitch + col0 * 2 + ch * 16) | drop;
                        if (row0 + 128 * g0 + 8 * c + 2 * lw < mv)
                            __builtin_amdgcn_raw_buffer_store_b128(sv[c], rs0, off, 0, kNonTemporal);
                        else
                            __builtin_amdgcn_raw_buffer_store_b128(sv[c], rs1, off, 0, kNonTemporal);
                    }
                };
                auto plain_barrier = [] {
                    __builtin_amdgcn_sched_barrier(0);
                    asm volatile("s_barrier" ::: "memory");
                    __builtin_amdgcn_sched_barrier(0);
                };
                const bool first_half = early && g0 == 0;
                if (!early) plain_barrier();   // every wave is done reading the last stage
                stage_own_rows();
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                if (first_half) {
                    plain_barrier();
                    store_rows();
                }
                plain_barrier();
                if (!first_half) store_rows();
            } else {
                // the residual epilogue: thread t holds 16-byte chunk t%32 of
                // tile rows t/32 + 16c
                __syncthreads();   // every wave is done reading the last stage
                stage_own_rows();
                __syncthreads();
                const int ch = ei.tid & 31;
                const int sub = ei.tid >> 5;
                u32x4 sv[16];
#pragma unroll
                for (int c = 0; c < 16; ++c)
                    sv[c] = *(const u32x4*)(lds + (16 * c + sub) * EP + ch * 16);
                residual_store(sv, sub, ch);
            }
            return;
        }
        if (!YK && (n & 3) == 0) {
            // fp32: the same LDS staging in two halves of 128 rows (1 KB
            // rows); the waves of row half h (wm == h) fill it, then all
            // store 16-byte row chunks
            constexpr int EF = BN * 4 + 16;   // fp32 row pitch (bytes)
            static_assert(128 * EF <= LDS_BYTES, "fp32 half tile exceeds the LDS");
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                __syncthreads();   // the stage (h = 0) or the previous half is no longer read
                if (ei.wm == h) {
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const int cl = ei.wn * 64 + 32 * j + ei.l32;
                        const float bv = (bias && col0 + cl < n) ? bias[col0 + cl] : 0.f;
#pragma unroll
                        for (int i = 0; i < 4; ++i)
#pragma unroll
                            for (int r = 0; r < 16; ++r) {
                                float v = acc[i][j][r] + bv;
                                if (ACT == S2_ACT_GELU) v = gelu(v);
                                const int rl = 32 * i + 8 * (r >> 2) + 4 * ei.g + (r & 3);
                                *(float*)(lds + rl * EF + cl * 4) = v;
                            }
                    }
                }
                __syncthreads();
                // 128 rows x 1024 bytes: thread t stores chunk t%64 of rows
                // t/64 + 8c
#pragma unroll 4
                for (int c = 0; c < 16; ++c) {
                    const int rl = (ei.tid >> 6) + 8 * c;
                    const int ch = ei.tid & 63;
                    const int col = col0 + ch * 4;
                    float* yr = (float*)out_row(h * 128 + rl);
                    if (yr && col < n)
                        __builtin_nontemporal_store(*(const u32x4*)(lds + rl * EF + ch * 16),
                                                    (u32x4*)(yr + col));
                }
            }
            return;
        }
        // ragged n: direct stores, register r of a 32x32 accumulator is row
        // 8(r/4) + 4g + r%4, column l32
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = col0 + ei.wn * 64 + 32 * j + ei.l32;
            if (col >= n) continue;
            const float bv = bias ? bias[col] : 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    void* yr = out_row(ei.wm * 128 + 32 * i + 8 * (r >> 2) + 4 * ei.g + (r & 3));
                    if (!yr) continue;
                    float v = acc[i][j][r] + bv;
                    if (ACT == S2_ACT_GELU) v = gelu(v);
                    store1<YK>(yr, col, v);
                }
        }
    };

    // Work of this workgroup as segments (tile, k-iterations [kb, ke)).  A
    // data-parallel workgroup has one whole tile.  Stream-K workgroup s owns
    // iterations [bound(s), bound(s + 1)) of the split tiles, iteration i
    // being k-step i % nk of split tile i / nk.
    const bool split = (int)blockIdx.x >= sk.dp_tiles;
    // consecutive ranges (neighbouring tiles of the raster) on one XCD, so
    // that they share A and B panels in its L2 (dp_tiles is a multiple of 8)
    const int s = split ? xcd_remap(blockIdx.x - sk.dp_tiles, sk.sk_groups) : 0;
    const long total = (long)sk.sk_tiles * nk;
    auto bound = [&](long q) { return q * total / sk.sk_groups; };
    // the stream-K workgroup whose range holds iteration i
    auto owner = [&](long i) { return (int)(((i + 1) * sk.sk_groups - 1) / total); };
    long i = split ? bound(s) : 0;
    const long iend = split ? bound(s + 1) : nk;
    bool first = true;
#pragma unroll 1
    while (i < iend) {
        int t, kb, ke;
        if (split) {
            t = (int)(i / nk);
            kb = (int)(i - (long)t * nk);
            ke = (int)min((long)nk, kb + (iend - i));
            set_tile(sk.dp_tiles + t);
        } else {
            t = 0;
            kb = 0;
            ke = nk;
            set_tile(xcd_remap(blockIdx.x, sk.dp_tiles));
        }
        if (!first) __syncthreads();   // the previous segment's LDS is no longer read
        if constexpr (AWA != 0) {
            build_rows();
            __syncthreads();
        }
        bool finish = kb == 0 && ke == nk;
        // the plain 16-bit epilogue of a whole tile without an activation runs
        // early (see epilogue); with GELU the early schedule would serialise
        // the two groups' VALU work, which otherwise shares the SIMDs
        const bool early = AWA == 0 && RES == 0 && ACT == S2_ACT_NONE && YK != 0 &&
                           (n & 7) == 0 && finish;
        mainloop(kb, ke, early);
        if (!finish) {
            // slot layout: float4 c (4 accumulator registers) of thread tid
            // at byte (c * 512 + tid) * 16; the chunk index goes in soffset
            const __amdgpu_buffer_rsrc_t mine = __builtin_amdgcn_make_buffer_rsrc(
                sk.slots + (long)s * kSlotFloats, (short)0, kSlotFloats * 4, kRawBufferFormat);
#pragma unroll
            for (int ii = 0; ii < 4; ++ii)
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        f32x4 v = {acc[ii][j][4 * c], acc[ii][j][4 * c + 1], acc[ii][j][4 * c + 2],
                                   acc[ii][j][4 * c + 3]};
                        __builtin_amdgcn_raw_buffer_store_b128(
                            __builtin_bit_cast(u32x4, v), mine, tid * 16,
                            ((ii * 2 + j) * 4 + c) * 512 * 16, kCoherent);
                    }
            // The slot stores write through to memory; every wave waits for
            // its own before the workgroup barrier.  The arrival is an
            // agent-scope acquire-release read-modify-write: it releases this
            // part's slot (ordered after the barrier) and, for the last part,
            // acquires every earlier part's, which the second barrier passes
            // on to the other waves of the workgroup.
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (tid == 0)
                arrival = __hip_atomic_fetch_add(&sk.counters[t], 1, __ATOMIC_ACQ_REL,
                                                 __HIP_MEMORY_SCOPE_AGENT);
            __syncthreads();
            const int lo = owner((long)t * nk);
            const int hi = owner((long)t * nk + nk - 1);
            if (arrival == hi - lo) {
                // sum every part, this one's included, in workgroup order so
                // that the result does not depend on the order of arrival
#pragma unroll
                for (int ii = 0; ii < 4; ++ii)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[ii][j][r] = 0.f;
#pragma unroll 1
                for (int q = lo; q <= hi; ++q) {
                    const __amdgpu_buffer_rsrc_t other = __builtin_amdgcn_make_buffer_rsrc(
                        sk.slots + (long)q * kSlotFloats, (short)0, kSlotFloats * 4, kRawBufferFormat);
                    // sixteen 16-byte loads in flight per batch (four
                    // accumulators; the fragment registers are free here)
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
                                                   other, tid * 16,
                                                   (((2 * h + iq) * 2 + j) * 4 + c) * 512 * 16,
                                                   kCoherent));
#pragma unroll
                        for (int iq = 0; iq < 2; ++iq)
#pragma unroll
                            for (int j = 0; j < 2; ++j)
#pragma unroll
                                for (int c = 0; c < 4; ++c) {
                                    f32x16& d = acc[2 * h + iq][j];
                                    d[4 * c] += v[iq][j][c].x;
                                    d[4 * c + 1] += v[iq][j][c].y;
                                    d[4 * c + 2] += v[iq][j][c].z;
                                    d[4 * c + 3] += v[iq][j][c].w;
                                }
                    }
                }
                if (tid == 0)
                    __hip_atomic_store(&sk.counters[t], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                finish = true;
            }
        }
        if (finish) epilogue(early);
        // every memory operation of this segment is complete: a real
        // s_waitcnt (not asm) lets the compiler's wait insertion know, so
        // it adds no vmcnt wait of its own inside the next main loop
        __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
        first = false;
        i += ke - kb;
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

// Elementwise erf-GELU (the epilogue's gelu) over fp32, bf16 or fp16 values,
// four per thread.
template <typename T>
__global__ void gelu_kernel(const T* x, T* y, size_t n) {
    const size_t i0 = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const size_t i = i0 + j;
        if (i >= n) return;
        if constexpr (std::is_same<T, float>::value)
            y[i] = gelu(x[i]);
        else if constexpr (std::is_same<T, uint16_t>::value)
            y[i] = __builtin_bit_cast(uint16_t, (__bf16)gelu(bf16_to_f32(x[i])));
        else
            y[i] = f32_to_f16(gelu((float)x[i]));
    }
}

hipError_t launch_gelu(const void* x, void* y, size_t n, int kind, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    const unsigned blocks = (unsigned)((n + 1023) / 1024);
    if (kind == 1)
        gelu_kernel<uint16_t><<<blocks, 256, 0, stream>>>((const uint16_t*)x, (uint16_t*)y, n);
    else if (kind == 2)
        gelu_kernel<_Float16><<<blocks, 256, 0, stream>>>((const _Float16*)x, (_Float16*)y, n);
    else
        gelu_kernel<float><<<blocks, 256, 0, stream>>>((const float*)x, (float*)y, n);
    return hipGetLastError();
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

// Scratch of the split-k tail: one partial-accumulator slot per workgroup
// that shares a tile (at most one per CU), then one arrival counter per
// shared tile (fewer than the CUs).
namespace {

constexpr int kMaxDevices = 64;

// Compute units of the current device (the workgroups of one wave of tiles).
hipError_t device_cus(int* cus) {
    static int g_cus[kMaxDevices];
    static std::once_flag g_once[kMaxDevices];
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::call_once(g_once[dev], [dev] {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            n = 0;
        g_cus[dev] = n > 0 ? n : 256;
    });
    *cus = g_cus[dev];
    return hipSuccess;
}

size_t sk_scratch_bytes(int groups) {
    return (size_t)groups * kSlotFloats * sizeof(float) + (size_t)groups * sizeof(int);
}

}  // namespace

// Split-k scratch of a stream on the current device: a slot per compute unit.
hipError_t splitk_scratch_bytes(size_t* bytes) {
    int G = 0;
    const hipError_t e = device_cus(&G);
    if (e == hipSuccess) *bytes = sk_scratch_bytes(G);
    return e;
}

namespace {

// The no-allocation entry point's scratch: slots and counters for up to
// kNoallocGroups sharing workgroups (the split of a 256-CU device), about
// 64 MB that every GPU the library runs on holds until the process ends.
constexpr int kNoallocGroups = 256;
constexpr size_t kNoallocBytes = (size_t)kNoallocGroups * kSlotFloats * sizeof(float) +
                                 (size_t)kNoallocGroups * sizeof(int);
static __device__ __align__(256) unsigned char scratch[kNoallocBytes];

// Device address of `scratch` on the current device.  The host-side name is
// only a stand-in for the symbol: kernels get this address instead.
hipError_t noalloc_scratch(void** out) {
    static void* g_ptr[kMaxDevices];
    static hipError_t g_err[kMaxDevices];
    static std::once_flag g_once[kMaxDevices];
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::call_once(g_once[dev], [dev] {
        void* p = nullptr;
        g_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_ptr[dev] = p;
    });
    if (g_err[dev] != hipSuccess) return g_err[dev];
    *out = g_ptr[dev];
    return hipSuccess;
}

__global__ void zero_counters_kernel(int* counters, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) counters[i] = 0;
}

}  // namespace

// Where the split-k tail keeps its partial tiles: the calling stream's own
// allocation (stream_scratch), or, for the no-allocation entry point, the
// static `scratch` array (whose counters are cleared before every launch
// that uses them, since a call keeps whatever the last one left).
enum class SkSource { kStream, kStatic };

// Split-k tail of a launch of `tiles` 256x256 tiles with nk 64-k steps:
// when the last wave of tiles would leave more than 3% of the workgroup
// slots idle, each tile of that wave is split along k into P equal parts on
// P workgroups (P <= 4, at least 8 k-iterations a part): the wave then takes
// about 1/P of a tile's time plus the reduction of P partial tiles.
static hipError_t plan_sk_tail(long tiles, int nk, SkSource source, hipStream_t stream, SkTail* out) {
    int G = 0;
    hipError_t e = device_cus(&G);
    if (e != hipSuccess) return e;
    SkTail sk{(int)tiles, 0, 0, nullptr, nullptr};
    const long waves = (tiles + G - 1) / G;
    const long rem = tiles % G == 0 ? G : tiles % G;
    if ((double)tiles / (double)(waves * G) < 0.97) {
        const long parts = std::min<long>(4, std::min<long>(G / rem, nk / 8));
        if (parts >= 2) {
            sk.dp_tiles = (int)(tiles - rem);
            sk.sk_tiles = (int)rem;
            sk.sk_groups = (int)(rem * parts);
        }
    }
    if (sk.sk_groups > 0) {
        void* base = nullptr;
        if (source == SkSource::kStatic) {
            // (hipErrorNotSupported: the caller reports a size beyond the
            // static scratch)
            if (sk.sk_groups > kNoallocGroups) return hipErrorNotSupported;
            e = noalloc_scratch(&base);
            if (e != hipSuccess) return e;
            sk.slots = (float*)base;
            sk.counters = (int*)((char*)base + (size_t)kNoallocGroups * kSlotFloats * 4);
            zero_counters_kernel<<<1, 256, 0, stream>>>(sk.counters, sk.sk_tiles);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
        } else {
            e = stream_scratch(kScratchSplitK, stream, sk_scratch_bytes(G), &base);
            if (e != hipSuccess) return e;
            sk.slots = (float*)base;
            sk.counters = (int*)((char*)base + (size_t)G * kSlotFloats * 4);
        }
    }
    *out = sk;
    return hipSuccess;
}

template <typename TX, int YK, int ACT>
static hipError_t linear_impl(const void* x0, int m0, const void* x1, int m1, const uint16_t* w,
                              const float* bias, int n, int k, void* y0, void* y1,
                              hipStream_t stream, SkSource source) {
    // bf16 activations (the operand type of the MFMAs) go straight to LDS;
    // fp32 and fp16 ones are rounded to bf16 while staged by the 128 kernel
    if (std::is_same<TX, uint16_t>::value && k % 64 == 0 &&
        (long)256 * k * 2 <= 0x7fffffffL &&   // buffer offsets are 32-bit
        (long)256 * n * 4 <= 0x7fffffffL) {
        const int mv = (m0 + 7) / 8 * 8;   // first text row in the joint row space
        const int ntiles = (n + 255) / 256;
        const int mtiles = (mv + m1 + 255) / 256;
        const long tiles = (long)mtiles * ntiles;
        if (tiles == 0) return hipSuccess;
        SkTail sk;
        hipError_t e = plan_sk_tail(tiles, k / 64, source, stream, &sk);
        if (e != hipSuccess) return e;
        const long blocks = (long)sk.dp_tiles + sk.sk_groups;
        shared_linear_256_kernel<YK, ACT><<<(unsigned)blocks, 512, 0, stream>>>(
            (const uint16_t*)x0, m0, (const uint16_t*)x1, m1, w, bias, n, k, y0, y1, mv, mtiles,
            ntiles, sk, AwaQkvArgs{}, LinearResidual{});
        return hipGetLastError();
    }
    const int mt0 = (m0 + 127) / 128;
    const int mt1 = (m1 + 127) / 128;
    const int ntiles = (n + 127) / 128;
    const int mtiles = mt0 + mt1;
    const long blocks = (long)mtiles * ntiles;
    if (blocks == 0) return hipSuccess;
    shared_linear_kernel<TX, YK, ACT><<<(unsigned)blocks, 256, 0, stream>>>(
        (const TX*)x0, m0, (const TX*)x1, m1, w, bias, n, k, y0, y1, mt0, mtiles, ntiles);
    return hipGetLastError();
}

template <typename TX, int YK>
static hipError_t linear_act(int act, const void* x0, int m0, const void* x1, int m1,
                             const uint16_t* w, const float* bias, int n, int k, void* y0,
                             void* y1, hipStream_t stream, SkSource src) {
    if (act == S2_ACT_SWIGLU) {
        // bf16 activations on the 256-tile path only (the caller checks);
        // n is the output width, the weight has 2n interleaved rows
        if constexpr (std::is_same<TX, uint16_t>::value) {
            if (k % 64 != 0 || n % 128 != 0 || (long)256 * k * 2 > 0x7fffffffL)
                return hipErrorInvalidValue;
            return linear_impl<TX, YK, S2_ACT_SWIGLU>(x0, m0, x1, m1, w, bias, 2 * n, k, y0, y1,
                                                      stream, src);
        }
        return hipErrorInvalidValue;
    }
    if (act == S2_ACT_GELU)
        return linear_impl<TX, YK, S2_ACT_GELU>(x0, m0, x1, m1, w, bias, n, k, y0, y1, stream, src);
    return linear_impl<TX, YK, S2_ACT_NONE>(x0, m0, x1, m1, w, bias, n, k, y0, y1, stream, src);
}

template <typename TX>
static hipError_t linear_out(int y_kind, int act, const void* x0, int m0, const void* x1, int m1,
                             const uint16_t* w, const float* bias, int n, int k, void* y0,
                             void* y1, hipStream_t stream, SkSource src) {
    if (y_kind == 1)
        return linear_act<TX, 1>(act, x0, m0, x1, m1, w, bias, n, k, y0, y1, stream, src);
    if (y_kind == 2)
        return linear_act<TX, 2>(act, x0, m0, x1, m1, w, bias, n, k, y0, y1, stream, src);
    return linear_act<TX, 0>(act, x0, m0, x1, m1, w, bias, n, k, y0, y1, stream, src);
}

static hipError_t linear_dispatch(const void* x0, int m0, const void* x1, int m1, int x_kind,
                                  const uint16_t* w, const float* bias, int n, int k, int act,
                                  void* y0, void* y1, int y_kind, hipStream_t stream,
                                  SkSource src) {
    if (x_kind == 1)
        return linear_out<uint16_t>(y_kind, act, x0, m0, x1, m1, w, bias, n, k, y0, y1, stream, src);
    if (x_kind == 2)
        return linear_out<_Float16>(y_kind, act, x0, m0, x1, m1, w, bias, n, k, y0, y1, stream, src);
    return linear_out<float>(y_kind, act, x0, m0, x1, m1, w, bias, n, k, y0, y1, stream, src);
}

hipError_t launch_shared_linear(const void* x0, int m0, const void* x1, int m1, int x_kind,
                                const uint16_t* w, const float* bias, int n, int k, int act,
                                void* y0, void* y1, int y_kind, hipStream_t stream) {
    return linear_dispatch(x0, m0, x1, m1, x_kind, w, bias, n, k, act, y0, y1, y_kind, stream,
                           SkSource::kStream);
}

hipError_t launch_shared_linear_noalloc(const void* x0, int m0, const void* x1, int m1,
                                        int x_kind, const uint16_t* w, const float* bias, int n,
                                        int k, int act, void* y0, void* y1, int y_kind,
                                        hipStream_t stream) {
    return linear_dispatch(x0, m0, x1, m1, x_kind, w, bias, n, k, act, y0, y1, y_kind, stream,
                           SkSource::kStatic);
}

hipError_t launch_shared_linear_residual(const uint16_t* x0, int m0, const uint16_t* x1, int m1,
                                         const uint16_t* w, const float* bias, int n, int k,
                                         const LinearResidual& res, hipStream_t stream) {
    if (k % 64 != 0 || n % 8 != 0 || (long)256 * k * 2 > 0x7fffffffL ||
        (long)256 * n * 4 > 0x7fffffffL)
        return hipErrorInvalidValue;
    const int mv = (m0 + 7) / 8 * 8;
    const int ntiles = (n + 255) / 256;
    const int mtiles = (mv + m1 + 255) / 256;
    const long tiles = (long)mtiles * ntiles;
    if (tiles == 0) return hipSuccess;
    SkTail sk;
    hipError_t e = plan_sk_tail(tiles, k / 64, SkSource::kStream, stream, &sk);
    if (e != hipSuccess) return e;
    const long blocks = (long)sk.dp_tiles + sk.sk_groups;
    shared_linear_256_kernel<1, S2_ACT_NONE, 0, 1><<<(unsigned)blocks, 512, 0, stream>>>(
        x0, m0, x1, m1, w, bias, n, k, nullptr, nullptr, mv, mtiles, ntiles, sk, AwaQkvArgs{},
        res);
    return hipGetLastError();
}

hipError_t launch_awa_qkv(const s2_awa_plan& plan, const uint16_t* x_video, const uint16_t* x_text,
                          int k, const uint16_t* w, const float* bias, const float* norm,
                          const float2* rope, uint16_t* q, uint16_t* kk, uint16_t* vt,
                          hipStream_t stream) {
    const int d = plan.config.head_dim;
    const int inner = plan.config.heads * d;
    if ((d != 64 && d != 128) || inner % 256 != 0 || k % 64 != 0 ||
        (long)(plan.video_tokens + 1) * k * 2 > 0x7fffffffL ||
        (long)(plan.text_tokens + 1) * k * 2 > 0x7fffffffL)
        return hipErrorInvalidValue;
    const int n = 3 * inner;
    const int ntiles = n / 256;
    const int mtiles = (plan.qkv_rows + 255) / 256;
    const long tiles = (long)mtiles * ntiles;
    if (tiles == 0) return hipSuccess;
    SkTail sk;
    hipError_t e = plan_sk_tail(tiles, k / 64, SkSource::kStream, stream, &sk);
    if (e != hipSuccess) return e;
    AwaQkvArgs a;
    a.row_table = plan.d_qkv_rows;
    a.inner = inner;
    a.seg_total = plan.seg_total;
    a.seg_text = plan.seg_text;
    a.norm = norm;
    a.rope = rope;
    a.pairs = plan.config.rope_pairs_per_axis;
    a.eps = plan.config.epsilon;
    a.official_bf16 = plan.config.official_bf16_attention;
    a.q = q;
    a.k = kk;
    a.vt = vt;
    const long blocks = (long)sk.dp_tiles + sk.sk_groups;
    if (d == 128)
        shared_linear_256_kernel<1, S2_ACT_NONE, 128><<<(unsigned)blocks, 512, 0, stream>>>(
            x_video, plan.video_tokens, x_text, plan.text_tokens, w, bias, n, k, nullptr, nullptr,
            plan.qkv_text_row, mtiles, ntiles, sk, a, LinearResidual{});
    else
        shared_linear_256_kernel<1, S2_ACT_NONE, 64><<<(unsigned)blocks, 512, 0, stream>>>(
            x_video, plan.video_tokens, x_text, plan.text_tokens, w, bias, n, k, nullptr, nullptr,
            plan.qkv_text_row, mtiles, ntiles, sk, a, LinearResidual{});
    return hipGetLastError();
}

}  // namespace s2
