// gfx950 kernels of the AdaptiveWindowAttention forward.
//
//   rope_table     cos/sin of pos*freq for every position the plan can hold
//   awa_prologue   per (window, 64-row chunk, head): gather the window's video
//                  rows by plan index math and the sample's text rows, RMSNorm
//                  q and k, 3-axis RoPE, round to bf16, write window-ordered
//                  Q and K rows and V transposed (keys contiguous per channel)
//   awa_attention  per (window, 128-query tile, head): softmax(q k^T/sqrt d) v
//                  over the window's video+text keys on bf16 MFMA 32x32x16
//                  with an online softmax; video rows are scattered straight
//                  to source order, text rows go to per-window partials
//   awa_text_pool  deterministic mean of the text partials over the sample's
//                  windows, in window order
//   awa_plan_tables  video_indices / inverse / local_positions on the device
//
// Reference: src/seedvr2/adaptive_window_attention.cpp:764-978 (CPU forward)
// and the Vulkan path :1059-1270 with its shaders :21-409.
#include <math.h>

#include <type_traits>

#include "awa_index.h"
#include "awa_kernels.h"
#include "s2_device.h"

namespace s2 {

// ---------------------------------------------------------------------------
// cos/sin table: table[pos * pairs + p] = (cos(pos*f[p]), sin(pos*f[p])), the
// angle formed in fp32 as apply_mm_rope does (:534-536).
__global__ void rope_table_kernel(const float* __restrict__ freqs, int pairs, int positions,
                                  float2* __restrict__ table) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= pairs * positions) return;
    const int pos = i / pairs;
    const int p = i - pos * pairs;
    const float angle = (float)pos * freqs[p];
    table[i] = make_float2(cosf(angle), sinf(angle));
}

// ---------------------------------------------------------------------------
// Eight consecutive input channels held as loaded (bf16, fp16 or fp32),
// converted to fp32 when used.
template <typename T>
struct type_tag {
    using type = T;
};

template <typename T>
struct Raw8;

template <>
struct Raw8<uint16_t> {
    uint4 v;
    __device__ __forceinline__ void load(const uint16_t* p) { v = *reinterpret_cast<const uint4*>(p); }
    __device__ __forceinline__ void to_float(float (&f)[8]) const {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = __uint_as_float(w[i] << 16);
            f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
};

template <>
struct Raw8<_Float16> {
    uint4 v;
    __device__ __forceinline__ void load(const _Float16* p) { v = *reinterpret_cast<const uint4*>(p); }
    __device__ __forceinline__ void to_float(float (&f)[8]) const {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xffffu));
            f[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
        }
    }
};

template <>
struct Raw8<float> {
    float4 a, b;
    __device__ __forceinline__ void load(const float* p) {
        a = *reinterpret_cast<const float4*>(p);
        b = *reinterpret_cast<const float4*>(p + 4);
    }
    __device__ __forceinline__ void to_float(float (&f)[8]) const {
        f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
        f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    }
};

// ---------------------------------------------------------------------------
// Prologue.  256 threads; each row of D channels is handled by D/8 threads
// holding 8 consecutive channels (RoPE pairs never straddle threads).
template <int D, typename TIn>
__global__ __launch_bounds__(256) void awa_prologue_kernel(
    const WinMeta* __restrict__ wins, const ChunkRef* __restrict__ chunks,
    const TIn* __restrict__ vq, const TIn* __restrict__ vk, const TIn* __restrict__ vv,
    long vstride, const TIn* __restrict__ tq, const TIn* __restrict__ tk,
    const TIn* __restrict__ tv, long tstride, const float* __restrict__ norm,
    const float2* __restrict__ rope, int pairs, float eps, int official_bf16,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_out, uint16_t* __restrict__ vt_out,
    long seg_total) {
#pragma clang fp contract(off)
    constexpr int TPR = D / 8;         // threads per row
    constexpr int RPP = 256 / TPR;     // rows per pass
    constexpr int CHUNK = kSegAlign;   // rows per workgroup
    constexpr int VTP = CHUNK;         // LDS pitch of the V^T tile (one 128-byte row per channel)
    __shared__ __attribute__((aligned(16))) uint16_t vt_lds[D * VTP];

    const ChunkRef ch = chunks[blockIdx.y];
    const WinMeta w = wins[ch.window];
    const int head = blockIdx.x;
    const int tid = threadIdx.x;
    const int d0 = (tid % TPR) * 8;
    const int rot_width = pairs * 6;
    // a video chunk writes the window's segment, a text chunk (row0 >=
    // n_video) its sample's staging rows; rows past lim are padding
    const bool text_chunk = ch.row0 >= w.n_video;
    const int lim = text_chunk ? w.seq : w.n_video;
    const long base_row = text_chunk ? (long)w.ts_row - w.n_video : (long)w.seg_off;
    const long head_rows = (long)head * seg_total + base_row;

    constexpr int NP = CHUNK / RPP;      // rows per thread
    // Every row's q, k and v loads are issued before any of them is used, so
    // a thread keeps 3 * NP loads in flight; rows past the sequence (padding)
    // read video row 0 and are zeroed afterwards.
    Raw8<TIn> rq[NP], rk[NP], rv[NP];
    float2 cs[NP][4];   // RoPE (cos, sin) of this thread's four channel pairs
    // norm weights of this thread's 8 channels: video q, video k, text q, text k
    float nw[4][8];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 8; ++i) nw[t][i] = norm[t * D + d0 + i];
#pragma unroll
    for (int pass = 0; pass < NP; ++pass) {
        const int r = ch.row0 + pass * RPP + tid / TPR;   // row within the window sequence
        const bool video = r < w.n_video;
        const TokenCoord tc = window_token(w, video ? r : 0);
        // window-local video position, temporal axis offset by the text
        // length (:901-902); text position (i,i,i) (:915)
        const int tt = r - w.n_video;
        const int pos[3] = {video ? tc.lt + w.text_len : tt, video ? tc.lh : tt, video ? tc.lw : tt};
#pragma unroll
        for (int pp = 0; pp < 4; ++pp) {
            // pair (2p, 2p+1) of axis a is rotated by pos[a] * f[p]; pairs
            // past the rotated width are left unrotated
            const int d = d0 + 2 * pp;
            const int axis = d / (2 * pairs > 0 ? 2 * pairs : 1);
            const int pair = (d - axis * 2 * pairs) >> 1;
            const bool rot = d < rot_width && r < lim;
            cs[pass][pp] = rot ? rope[pos[axis < 3 ? axis : 0] * pairs + pair] : make_float2(1.f, 0.f);
        }
        const long src = video ? tc.src : (long)w.text_off + tt;
        const bool ok = r < lim;
        const TIn* bq = video || !ok ? vq : tq;
        const TIn* bk = video || !ok ? vk : tk;
        const TIn* bv = video || !ok ? vv : tv;
        const long row = ok ? src : 0;
        const long stride = video || !ok ? vstride : tstride;
        const int col = head * D + d0;
        rq[pass].load(bq + row * stride + col);
        rk[pass].load(bk + row * stride + col);
        rv[pass].load(bv + row * stride + col);
    }
#pragma unroll
    for (int pass = 0; pass < NP; ++pass) {
        const int rl = pass * RPP + tid / TPR;   // row within the chunk
        const int r = ch.row0 + rl;               // row within the window sequence
        uint16_t qb[8], kb[8], vb[8];
        if (r < lim) {
            const bool video = r < w.n_video;
            float q[8], k[8], v[8];
            rq[pass].to_float(q);
            rk[pass].to_float(k);
            rv[pass].to_float(v);
            // sums of squares as one fma chain per row (the fused QKV
            // epilogue takes the same operation order)
            float sq2 = q[0] * q[0], sk2 = k[0] * k[0];
#pragma unroll
            for (int i = 1; i < 8; ++i) {
                sq2 = fmaf(q[i], q[i], sq2);
                sk2 = fmaf(k[i], k[i], sk2);
            }
#pragma unroll
            for (int off = 1; off < TPR; off <<= 1) {
                sq2 += __shfl_xor(sq2, off);
                sk2 += __shfl_xor(sk2, off);
            }
            // rms_norm (:510-519): x * (1 / sqrt(sum/size + eps)) * w, the
            // reciprocal square root by v_rsq_f32 (within 1 ulp)
            const float inv_q = __builtin_amdgcn_rsqf(sq2 / (float)D + eps);
            const float inv_k = __builtin_amdgcn_rsqf(sk2 / (float)D + eps);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                q[i] = q[i] * inv_q * (video ? nw[0][i] : nw[2][i]);
                k[i] = k[i] * inv_k * (video ? nw[1][i] : nw[3][i]);
            }
            // apply_mm_rope (:521-543): pair (2p, 2p+1) of axis a rotated by pos[a]*f[p]
#pragma unroll
            for (int pp = 0; pp < 4; ++pp) {
                if (d0 + 2 * pp < rot_width) {
                    const float2 c = cs[pass][pp];
                    const float q0 = q[2 * pp], q1 = q[2 * pp + 1];
                    const float k0 = k[2 * pp], k1 = k[2 * pp + 1];
                    q[2 * pp] = fmaf(q0, c.x, -(q1 * c.y));
                    q[2 * pp + 1] = fmaf(q0, c.y, q1 * c.x);
                    k[2 * pp] = fmaf(k0, c.x, -(k1 * c.y));
                    k[2 * pp + 1] = fmaf(k0, c.y, k1 * c.x);
                }
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (official_bf16) {
                    qb[i] = round_bf16_ref_bits(q[i]);
                    kb[i] = round_bf16_ref_bits(k[i]);
                    vb[i] = round_bf16_ref_bits(v[i]);
                } else {   // v_cvt_pk_bf16_f32: round to nearest even
                    qb[i] = __builtin_bit_cast(uint16_t, (__bf16)q[i]);
                    kb[i] = __builtin_bit_cast(uint16_t, (__bf16)k[i]);
                    vb[i] = __builtin_bit_cast(uint16_t, (__bf16)v[i]);
                }
            }
        } else {
            // padding rows (the attention masks them as keys in any case)
#pragma unroll
            for (int i = 0; i < 8; ++i) qb[i] = kb[i] = vb[i] = 0;
        }
        const long orow = (head_rows + r) * D + d0;
        *reinterpret_cast<uint4*>(q_out + orow) = pack8_bf16(qb);
        *reinterpret_cast<uint4*>(k_out + orow) = pack8_bf16(kb);
        // channel d0+i, key rl: 16-byte key chunk rl/8 stored at position
        // (rl/8) ^ (channel/8 & 7), which spreads the 16 channels one store
        // instruction writes over 8 bank groups
#pragma unroll
        for (int i = 0; i < 8; ++i)
            vt_lds[(d0 + i) * VTP + ((((rl >> 3) ^ (d0 >> 3)) & 7) << 3) + (rl & 7)] = vb[i];
    }
    __syncthreads();
    // V^T rows: channel-major, the chunk's 64 keys contiguous (128 bytes).
    for (int idx = tid; idx < D * (CHUNK / 8); idx += 256) {
        const int d = idx / (CHUNK / 8);
        const int c8 = idx - d * (CHUNK / 8);
        const uint4 val =
            *reinterpret_cast<const uint4*>(&vt_lds[d * VTP + (((c8 ^ (d >> 3)) & 7) << 3)]);
        *reinterpret_cast<uint4*>(vt_out + ((long)head * D + d) * seg_total + base_row + ch.row0 +
                                  c8 * 8) = val;
    }
}

// v_permlane32_swap with the same value in both operands leaves, in every
// lane, the pair {x[lane], x[lane ^ 32]} in its two results (a VALU op, no
// LDS round trip as with a shuffle).
// Maxima of attention scores with the NaN-propagating maximum (v_maximum3 on
// gfx950), which needs no quieting of its operands first, unlike fmaxf
__device__ __forceinline__ float max3_scores(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

__device__ __forceinline__ float max_with_lane_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __builtin_elementwise_maximum(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float sum_with_lane_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ---------------------------------------------------------------------------
// Flash window attention.
//
// Four waves; wave j owns query rows q_row0 + 32j .. +31.  Keys stream in
// tiles of 32 through a ring of three LDS stages, each holding the tile's K
// rows and its V^T rows, filled by buffer_load_dwordx4 ... lds (global ->
// LDS without VGPR staging) two tiles ahead.  At about 140 VGPRs three
// workgroups share a CU, so three waves per SIMD hide the MFMA dependency
// chains and the softmax VALU work of one another.
//
// The score tile is computed transposed, S^T = K Q^T, so that each lane owns
// one query column; the probabilities then feed O^T += V^T P^T directly from
// the accumulator registers.  For that the A-operand row R of the S^T MFMA
// loads key pi(R) = R with bits 2 and 3 swapped: accumulator register
// i = 8s+j of lane group g then holds key 16s + 8g + j, which is exactly the
// B-operand slot 8g+j of the 16-key PV step s.
//
// Softmax in the log2 domain.  When the norm weights bound every exponent
// (|s| * log2(e) / sqrt(D) <= B <= 60, see the score bound below) the
// exponentials are taken relative to the fixed reference B: no row maximum,
// rescale or wave vote per tile.  Otherwise it is an online softmax with a
// lazily updated row max: the running max only moves when a tile's max
// exceeds it by more than 8, so un-normalised probabilities stay below 2^8
// and the accumulator rescale is skipped for the many tiles that do not
// raise any row max of the wave.  Either way the result is the same softmax;
// only the reference point of the exponentials changes.
//
// LDS swizzles (16-byte chunk c of row r stored at position c ^ f(r)) keep
// the rows one ds_read_b128 phase reads on distinct banks:
//   K rows (D*2 bytes):  f(r) = r with bits 2 and 3 swapped, its low three
//     bits for D = 64.  A ds_read_b128 phase covers 8 lanes; the A-operand
//     row of lane l32 is l32 with bits 2 and 3 swapped, so f of its row is
//     l32 & 15, and the 8 lanes of a phase read 8 distinct chunk positions.
//   V^T rows (64 bytes): f(r) = (r >> 2) & 3.  Rows four apart share
//     their banks; the fragment read of a 16-lane group covers rows r..r+15,
//     so rows r, r+4, r+8, r+12 must take distinct chunk positions.  (The
//     LDS conflict counter reads 4 cycles per ds_read_b128 for
//     ((r >> 1) ^ (r >> 3)) & 3, 12 without a swizzle, 0 for this one.)
template <int D>
__device__ __forceinline__ int k_swizzle(int r) {
    const int f = (r & 3) | ((r >> 1) & 4) | ((r << 1) & 8);
    return D == 128 ? f : (f & 7);
}
__device__ __forceinline__ int vt_swizzle(int r) { return (r >> 2) & 3; }

template <int D>
__global__ __launch_bounds__(256, 3) void awa_attention_kernel(
    const WinMeta* __restrict__ wins, const AttnItem* __restrict__ items, int slots_per_xcd,
    const uint16_t* __restrict__ q_in, const uint16_t* __restrict__ k_in,
    const uint16_t* __restrict__ vt_in, long seg_total, float scale_log2, int official_bf16,
    void* __restrict__ out_video, int out_kind, int inner, float* __restrict__ text_partial,
    const float* __restrict__ norm) {
    constexpr int KT = 32;                  // keys per tile
    constexpr int STAGES = 3;
    constexpr int KB = KT * D * 2;          // K tile bytes
    constexpr int VB = D * KT * 2;          // V^T tile bytes
    constexpr int SB = KB + VB;             // stage bytes
    constexpr int NKK = D / 16;             // MFMA k-steps over the head dim
    constexpr int NDT = D / 32;             // 32-channel output tiles
    constexpr int KCH = D / 8;              // 16-byte chunks per K row
    constexpr int KRI = 1024 / (D * 2);     // K rows per DMA instruction
    constexpr int KI_W = KB / 1024 / 4;     // K DMA instructions per wave per tile
    constexpr int VI_W = VB / 1024 / 4;     // V^T DMA instructions per wave per tile
    constexpr int DMA_W = KI_W + VI_W;
    constexpr float kLazy = 8.f;            // max growth (log2) tolerated before rescaling
    constexpr float kFixedMax = 60.f;       // largest score bound taken as the fixed reference
    __shared__ __attribute__((aligned(1024))) uint8_t lds[STAGES * SB];
    __shared__ float wmax[4];

    const int bid = blockIdx.x;
    const AttnItem it = items[(bid % kNumXcd) * slots_per_xcd + bid / kNumXcd];
    if (it.window < 0) return;
    const WinMeta w = wins[it.window];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int l32 = lane & 31;
    const int g = lane >> 5;
    // The window's sequence is its video rows (segment rows seg_off ..) then
    // its sample's text rows (staging rows ts_row ..), each padded to whole
    // key tiles: nvt video tiles, then the text tiles.
    const long head_k = (long)it.head * seg_total;   // the head's row 0 of Q and K
    const int nvt = (w.n_video + KT - 1) / KT;
    const int nkt = nvt + (w.text_len + KT - 1) / KT;

    // this thread's norm weights for the score bound below (their latency
    // overlaps that of the Q loads and the first DMAs)
    const float nw0 = norm[tid];
    const float nw1 = D == 128 ? norm[256 + tid] : 0.f;

    // Q fragment (B operand of S^T = K Q^T): query row l32 of this wave,
    // channels 16kk + 8g .. +7.
    const int qrow = it.q_row0 + wave * 32 + l32;
    const bool wave_active = it.q_row0 + wave * 32 < w.seq;
    bf16x8 qf[NKK];
    {
        const bool valid = qrow < w.seq;
        const long row = qrow < w.n_video ? (long)w.seg_off + qrow : (long)w.ts_row + qrow - w.n_video;
        const uint16_t* qp = q_in + (head_k + row) * D + 8 * g;
#pragma unroll
        for (int kk = 0; kk < NKK; ++kk) {
            uint4 raw = make_uint4(0, 0, 0, 0);
            if (valid) raw = *reinterpret_cast<const uint4*>(qp + 16 * kk);
            qf[kk] = as_bf16x8(raw);
        }
    }

    // DMA sources: the head's K rows [seg_total][D] and V^T rows
    // [D][seg_total]; a tile's first key row goes in the scalar offset.
    const i32x4 rk = buffer_rsrc(k_in + head_k * D, (uint32_t)(seg_total * D * 2));
    const i32x4 rv = buffer_rsrc(vt_in + head_k * D, (uint32_t)(seg_total * D * 2));
    uint32_t koff[KI_W], voff[VI_W];
#pragma unroll
    for (int j = 0; j < KI_W; ++j) {
        const int row = (wave * KI_W + j) * KRI + lane / KCH;
        const int c = (lane % KCH) ^ k_swizzle<D>(row);
        koff[j] = (uint32_t)((row * D + c * 8) * 2);
    }
#pragma unroll
    for (int j = 0; j < VI_W; ++j) {
        const int d = (wave * VI_W + j) * 16 + (lane >> 2);
        const int c = (lane & 3) ^ vt_swizzle(d);
        voff[j] = (uint32_t)(((long)d * seg_total + c * 8) * 2);
    }
    const uint32_t lds_base = (uint32_t)(uintptr_t)lds;
    // first key row of tile kt, and the number of its keys that are real
    // (KT or more but in the last tile of either part)
    auto tile_row = [&](int kt) {
        return kt < nvt ? w.seg_off + kt * KT : w.ts_row + (kt - nvt) * KT;
    };
    auto tile_keys = [&](int kt) {
        return kt < nvt ? w.n_video - kt * KT : w.text_len - (kt - nvt) * KT;
    };
    auto issue = [&](int stage, int kt) {
        const uint32_t st = lds_base + stage * SB;
        const uint32_t key0 = (uint32_t)__builtin_amdgcn_readfirstlane(tile_row(kt));
#pragma unroll
        for (int j = 0; j < KI_W; ++j)
            lds_dma16(rk, __builtin_amdgcn_readfirstlane(st + (wave * KI_W + j) * 1024), koff[j],
                      key0 * (D * 2));
#pragma unroll
        for (int j = 0; j < VI_W; ++j)
            lds_dma16(rv, __builtin_amdgcn_readfirstlane(st + KB + (wave * VI_W + j) * 1024),
                      voff[j], key0 * 2);
    };

    f32x16 o[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
    float m_run = -INFINITY;   // running max (log2 domain), same in lanes l and l^32
    float l_run = 0.f;         // this lane's share of the running sum

    // S^T A-operand row l32 loads key krow; its swizzle and the V^T row
    // swizzle depend on l32 only
    const int krow = (l32 & 0x13) | ((l32 & 4) << 1) | ((l32 & 8) >> 1);
    const int kswz = k_swizzle<D>(krow);
    const int vswz = vt_swizzle(l32);

    issue(0, 0);
    if (nkt > 1) issue(1, 1);
    // The Q loads must be complete before the loop in a way the compiler
    // sees: its wait insertion does not track the DMA asm, and with Q loads
    // possibly outstanding at the loop header it would put a vmcnt(0) before
    // the first MFMA of every tile, which also waits for the DMA issued two
    // tiles ahead.  The first tile needs its DMA anyway.
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    // Score bound.  q and k rows are RMS-normalised (norm <= sqrt(D)),
    // scaled by the norm weights, rotated and rounded to bf16, so
    // |q.k| <= D * Wq * Wk * (1 + 2^-7) with Wq (Wk) the largest |weight| of
    // the video and text q (k) norms, and every exponent s * scale_log2 lies
    // within +-B, B = sqrt(D) log2(e) Wq Wk (1 + 2^-6).  For B <= kFixedMax the
    // softmax is taken relative to the fixed reference B instead of a running
    // row maximum: every exponential lies in [2^-2B, 1] (normal floats, also
    // as bf16), so no maximum, rescale or vote is needed.  A NaN weight gives
    // a NaN bound and the running-maximum path.
    {
        // wave maximum of |weight|: DPP within rows of 16 lanes, then the
        // four row results (NaN-propagating throughout)
        float a = D == 128 ? __builtin_elementwise_maximum(fabsf(nw0), fabsf(nw1)) : fabsf(nw0);
        a = __builtin_elementwise_maximum(
            a, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(a), 0xB1, 0xF, 0xF, false)));
        a = __builtin_elementwise_maximum(
            a, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(a), 0x4E, 0xF, 0xF, false)));
        a = __builtin_elementwise_maximum(
            a, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(a), 0x141, 0xF, 0xF, false)));
        a = __builtin_elementwise_maximum(
            a, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(a), 0x140, 0xF, 0xF, false)));
        const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 0));
        const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 16));
        const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 32));
        const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), 48));
        if (lane == 0)
            wmax[wave] = __builtin_elementwise_maximum(__builtin_elementwise_maximum(r0, r1),
                                                       __builtin_elementwise_maximum(r2, r3));
    }
    __syncthreads();
    // [vq | vk | tq | tk]: D = 128, waves 0-1 hold q weights, 2-3 k weights;
    // D = 64, waves 0 and 2 q, 1 and 3 k
    const float wq = D == 128 ? __builtin_elementwise_maximum(wmax[0], wmax[1])
                              : __builtin_elementwise_maximum(wmax[0], wmax[2]);
    const float wk = D == 128 ? __builtin_elementwise_maximum(wmax[2], wmax[3])
                              : __builtin_elementwise_maximum(wmax[1], wmax[3]);
    const float bound = sqrtf((float)D) * 1.4426950408889634f * 1.015625f * wq * wk;
    const bool fixed_ref = bound <= kFixedMax;   // false for a NaN bound
    if (fixed_ref) m_run = bound;
    // The tile loop is unrolled by the stage count so that every LDS
    // address is a loop-invariant register plus a constant stage offset.
    auto tiles = [&](auto fixed_tag) {
    constexpr bool FIXED = decltype(fixed_tag)::value;
#pragma unroll 1
    for (int kt0 = 0; kt0 < nkt; kt0 += STAGES) {
#pragma unroll
        for (int u = 0; u < STAGES; ++u) {
            const int kt = kt0 + u;
            if (kt >= nkt) break;
            if (kt + 1 < nkt) {   // stage kt+1 may stay in flight
                if constexpr (DMA_W == 4)
                    asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
                else
                    asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
            } else {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
            __syncthreads();   // tile kt visible to all waves; tile kt-1 no longer read
            if (kt + 2 < nkt) issue((u + 2) % STAGES, kt + 2);
            const uint8_t* st = lds + u * SB;
            // The last tile of either part holds nkeys < KT real keys; the
            // rest of its rows are padding with whatever the workspace holds
            // there.  Their scores are masked below, and their V^T entries
            // are zeroed here (probability 0 times a NaN would reach the
            // sum): the tile's D x 4 key chunks of 8, one or two a thread, by
            // all waves, active or not, before one more barrier.
            const int nkeys = tile_keys(kt);
            const bool partial = nkeys < KT;
            if (partial) {
                // an opaque copy of the thread index: the chunk addresses stay
                // in this branch instead of being hoisted, per stage, into
                // registers the tile loop needs
                int t0 = tid;
                asm volatile("" : "+v"(t0));
#pragma unroll
                for (int idx = t0; idx < D * 4; idx += 256) {
                    const int r = idx >> 2, c = idx & 3;
                    uint8_t* chunk = lds + u * SB + KB + r * (KT * 2) + ((c ^ vt_swizzle(r)) * 16);
                    if (8 * c >= nkeys) {
                        *(uint4*)chunk = make_uint4(0, 0, 0, 0);
                    } else if (8 * c + 8 > nkeys) {
                        for (int e = nkeys - 8 * c; e < 8; ++e) ((uint16_t*)chunk)[e] = 0;
                    }
                }
                __syncthreads();
            }

            // S^T = K Q^T
            // a wave whose 32 query rows all lie past the sequence (the last
            // q-tile of a window) only takes part in the DMA and barriers
            if (!wave_active) continue;
            f32x16 s;
            const uint8_t* kp = st + krow * (D * 2);
            auto kfrag = [&](int kk) {
                return as_bf16x8(*(const uint4*)(kp + (((2 * kk + g) ^ kswz) * 16)));
            };
            // K fragments are read two slices ahead of their MFMA (the
            // scheduling barriers keep the compiler from sinking each read
            // next to its use, which would expose the LDS latency per slice)
            bf16x8 kf[NKK];
            kf[0] = kfrag(0);
            kf[1] = kfrag(1);
#pragma unroll
            for (int kk = 0; kk < NKK; ++kk) {
                __builtin_amdgcn_sched_barrier(0);
                if (kk + 2 < NKK) kf[kk + 2] = kfrag(kk + 2);
                __builtin_amdgcn_sched_barrier(0);
                // one accumulation chain: back-to-back dependent MFMAs of
                // the same shape accumulate without extra wait states
                if (kk == 0)
                    s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[0], qf[0], f32x16{}, 0, 0, 0);
                else
                    s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[kk], qf[kk], s, 0, 0, 0);
            }
            // scores of the padding keys are masked
            if (partial) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    // register i of lane group g holds key 16*(i/8) + 8g + (i%8)
                    const int key = 16 * (i >> 3) + 8 * g + (i & 7);
                    if (key >= nkeys) s[i] = -INFINITY;
                }
            }
            float alpha = 1.f;
            if constexpr (!FIXED) {
                float mx = max3_scores(s[0], s[1], s[2]);
#pragma unroll
                for (int i = 3; i < 15; i += 2) mx = max3_scores(mx, s[i], s[i + 1]);
                mx = max3_scores(mx, mx, s[15]);
                mx = max_with_lane_xor32(mx) * scale_log2;
                if (mx > m_run + kLazy) {
                    alpha = __builtin_amdgcn_exp2f(m_run - mx);   // 0 on the first tile
                    m_run = mx;
                }
            }
            float p[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) p[i] = __builtin_amdgcn_exp2f(fmaf(s[i], scale_log2, -m_run));
            bf16x8 pb[2];
#pragma unroll
            for (int half = 0; half < 2; ++half)
#pragma unroll
                for (int j = 0; j < 8; ++j) pb[half][j] = (__bf16)p[8 * half + j];
            // pairwise sum: a dependency depth of 4 instead of 16
#pragma unroll
            for (int w2 = 8; w2 >= 1; w2 >>= 1)
#pragma unroll
                for (int i = 0; i < w2; ++i) p[i] += p[i + w2];
            if constexpr (FIXED) {
                l_run += p[0];
            } else {
                l_run = l_run * alpha + p[0];
                if (__any(alpha != 1.f)) {
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                        for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
                }
            }
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                const uint8_t* vp = st + KB + (32 * dt + l32) * (KT * 2);
#pragma unroll
                for (int ps = 0; ps < 2; ++ps) {
                    const bf16x8 a = as_bf16x8(*(const uint4*)(vp + (((2 * ps + g) ^ vswz) * 16)));
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb[ps], o[dt], 0, 0, 0);
                }
            }
        }
    }
    };
    if (fixed_ref)
        tiles(std::true_type{});
    else
        tiles(std::false_type{});

    const float l_tot = sum_with_lane_xor32(l_run);
    const float inv_l = 1.f / l_tot;
    if (qrow >= w.seq) return;
    // O^T register i of tile dt: channel 32dt + 8(i/4) + 4g + (i%4), query l32
    if (qrow < w.n_video) {
        const TokenCoord c = window_token(w, qrow);
        const long obase = c.src * inner + (long)it.head * D;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const int ch = 32 * dt + 8 * a + 4 * g;
                float vals[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float x = o[dt][4 * a + e] * inv_l;
                    if (official_bf16) x = bf16_to_f32(round_bf16_ref_bits(x));
                    vals[e] = x;
                }
                store4(out_video, obase + ch, vals[0], vals[1], vals[2], vals[3], out_kind);
            }
    } else {
        const long obase = (long)(w.tpart_off + qrow - w.n_video) * inner + (long)it.head * D;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const int ch = 32 * dt + 8 * a + 4 * g;
                float vals[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float x = o[dt][4 * a + e] * inv_l;
                    if (official_bf16) x = bf16_to_f32(round_bf16_ref_bits(x));
                    vals[e] = x;
                }
                *reinterpret_cast<float4*>(text_partial + obase + ch) =
                    make_float4(vals[0], vals[1], vals[2], vals[3]);
            }
    }
}

// ---------------------------------------------------------------------------
// Text mean-pool (:963-974): out = sum over the sample's windows, in plan
// order, of partial * (1/num_windows), accumulated in fp32 from zero.
__global__ void awa_text_pool_kernel(const SampleMeta* __restrict__ samples,
                                     const int* __restrict__ text_sample,
                                     const WinMeta* __restrict__ wins,
                                     const float* __restrict__ partial, int text_tokens,
                                     int inner, void* __restrict__ out, int out_kind) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;   // float4 index
    const int q4 = inner / 4;
    if (i >= (long)text_tokens * q4) return;
    const int row = (int)(i / q4);
    const int c = (int)(i - (long)row * q4) * 4;
    const SampleMeta sm = samples[text_sample[row]];
    const int tt = row - sm.text_off;
    // the sample's windows hold consecutive partial blocks of text_len rows
    const float* p = partial + ((long)wins[sm.first_window].tpart_off + tt) * inner + c;
    const long step = (long)sm.text_len * inner;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
    for (int k = 0; k < sm.num_windows; ++k) {
        const float4 x = *reinterpret_cast<const float4*>(p + k * step);
        acc.x += x.x * sm.pool_scale;
        acc.y += x.y * sm.pool_scale;
        acc.z += x.z * sm.pool_scale;
        acc.w += x.w * sm.pool_scale;
    }
    store4(out, (long)row * inner + c, acc.x, acc.y, acc.z, acc.w, out_kind);
}

// ---------------------------------------------------------------------------
// Plan tables (AdaptiveWindowPlan's per-token arrays) from the same index math.
__global__ void awa_plan_tables_kernel(const WinMeta* __restrict__ wins, int* __restrict__ indices,
                                       int* __restrict__ inverse, int* __restrict__ positions) {
    const WinMeta w = wins[blockIdx.y];
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= w.n_video) return;
    const TokenCoord c = window_token(w, r);
    const int p = w.part_off + r;
    if (indices) indices[p] = (int)c.src;
    if (inverse) inverse[c.src] = p;
    if (positions) {
        positions[3 * p + 0] = c.lt;
        positions[3 * p + 1] = c.lh;
        positions[3 * p + 2] = c.lw;
    }
}

// ---------------------------------------------------------------------------
// Launchers

hipError_t launch_rope_table(const float* freqs, int pairs, int positions, float2* table,
                             hipStream_t stream) {
    const int n = pairs * positions;
    if (n <= 0) return hipSuccess;
    rope_table_kernel<<<(n + 255) / 256, 256, 0, stream>>>(freqs, pairs, positions, table);
    return hipGetLastError();
}

template <int D, typename TIn>
static hipError_t prologue_impl(const s2_awa_plan& plan, const void* vq, const void* vk,
                                const void* vv, long vstride, const void* tq, const void* tk,
                                const void* tv, long tstride, const float* norm,
                                const float2* rope, uint16_t* q_out, uint16_t* k_out,
                                uint16_t* vt_out, hipStream_t stream) {
    // heads vary fastest: concurrently running workgroups gather the same
    // token rows (different head slices), which keeps DRAM rows and L2 lines hot
    dim3 grid(plan.config.heads, plan.num_chunks);
    awa_prologue_kernel<D, TIn><<<grid, 256, 0, stream>>>(
        plan.d_wins, plan.d_chunks, (const TIn*)vq, (const TIn*)vk, (const TIn*)vv, vstride,
        (const TIn*)tq, (const TIn*)tk, (const TIn*)tv, tstride, norm, rope,
        plan.config.rope_pairs_per_axis, plan.config.epsilon, plan.config.official_bf16_attention,
        q_out, k_out, vt_out, plan.seg_total);
    return hipGetLastError();
}

hipError_t launch_awa_prologue(const s2_awa_plan& plan, const void* vq, const void* vk,
                               const void* vv, long vstride, const void* tq, const void* tk,
                               const void* tv, long tstride, int in_kind, const float* norm,
                               const float2* rope, uint16_t* q_out, uint16_t* k_out,
                               uint16_t* vt_out, hipStream_t stream) {
    const int d = plan.config.head_dim;
    auto run = [&](auto dtag, auto ttag) {
        constexpr int DD = decltype(dtag)::value;
        using T = typename decltype(ttag)::type;
        return prologue_impl<DD, T>(plan, vq, vk, vv, vstride, tq, tk, tv, tstride, norm, rope,
                                    q_out, k_out, vt_out, stream);
    };
    auto by_type = [&](auto dtag) {
        if (in_kind == 1) return run(dtag, type_tag<uint16_t>{});
        if (in_kind == 2) return run(dtag, type_tag<_Float16>{});
        return run(dtag, type_tag<float>{});
    };
    if (d == 128) return by_type(std::integral_constant<int, 128>{});
    if (d == 64) return by_type(std::integral_constant<int, 64>{});
    return hipErrorInvalidValue;
}

hipError_t launch_awa_attention(const s2_awa_plan& plan, const uint16_t* q, const uint16_t* k,
                                const uint16_t* vt, void* out_video, int out_kind,
                                float* text_partial, const float* norm, hipStream_t stream) {
    const int d = plan.config.head_dim;
    const int inner = plan.config.heads * d;
    const float scale_log2 = 1.4426950408889634f / sqrtf((float)d);
    const int grid = plan.slots_per_xcd * kNumXcd;
    if (grid == 0) return hipSuccess;
    if (d == 128)
        awa_attention_kernel<128><<<grid, 256, 0, stream>>>(
            plan.d_wins, plan.d_items, plan.slots_per_xcd, q, k, vt, plan.seg_total, scale_log2,
            plan.config.official_bf16_attention, out_video, out_kind, inner, text_partial, norm);
    else if (d == 64)
        awa_attention_kernel<64><<<grid, 256, 0, stream>>>(
            plan.d_wins, plan.d_items, plan.slots_per_xcd, q, k, vt, plan.seg_total, scale_log2,
            plan.config.official_bf16_attention, out_video, out_kind, inner, text_partial, norm);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_awa_text_pool(const s2_awa_plan& plan, const float* partial, void* out_text,
                                int out_kind, hipStream_t stream) {
    const int inner = plan.config.heads * plan.config.head_dim;
    const long n = (long)plan.text_tokens * (inner / 4);
    if (n == 0) return hipSuccess;
    awa_text_pool_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(
        plan.d_samples, plan.d_text_sample, plan.d_wins, partial, plan.text_tokens, inner,
        out_text, out_kind);
    return hipGetLastError();
}


hipError_t launch_awa_plan_tables(const s2_awa_plan& plan, int* indices, int* inverse,
                                  int* positions, hipStream_t stream) {
    if (plan.num_windows == 0 || plan.max_window_tokens == 0) return hipSuccess;
    dim3 grid((plan.max_window_tokens + 255) / 256, plan.num_windows);
    awa_plan_tables_kernel<<<grid, 256, 0, stream>>>(plan.d_wins, indices, inverse, positions);
    return hipGetLastError();
}

}  // namespace s2
