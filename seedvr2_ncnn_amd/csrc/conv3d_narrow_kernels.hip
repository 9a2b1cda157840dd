// DecomposedConv3D (src/seedvr2/decomposed_conv3d.cpp:605-755) for layers
// with at most three output channels: the VAE decoder's RGB output conv,
// 128 -> 3 channels, 3x3x3, unit strides, one pixel of spatial padding.
//
// As an implicit GEMM with the output channels as its columns such a layer
// leaves 29 of every 32 MFMA columns empty, and it re-reads each input pixel
// for every window position.  Here the window positions become the columns
// instead: for one input row of one padded frame,
//   D[x][(tap, ky, co)] = sum_kx sum_ci X[ci][x + kx - 1] W[tap][co][ci][ky][kx]
// is one MFMA product (x: 128 output columns of a strip, 27 of 32 columns
// used, k = ci, the three kx as three passes over the same staged row shifted
// by one pixel), and output (t, y, x, co) is the sum of D over the (tap, ky)
// pairs with t = p - tap, y = row - ky + 1, p the padded frame of the row.
// Every input row is read from HBM once per workgroup (plus one row above
// and below the workgroup's band), straight from the planar blob: the
// layer is bound by the bytes of its 128-channel input.
//
// The temporal memory holds, instead of the last two padded frames of 128
// channels, the partial sums those frames contribute to the next forward's
// first two output frames ([2][cout][H][W] fp32): the next forward adds them
// where it would have read the frames.
#include <limits.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "conv3d_kernels.h"
#include "s2_device.h"

namespace s2 {
namespace {

constexpr int kPx = 128;               // output columns of a strip
constexpr int kXPitch = 136;           // bf16 per staged pixel: 128 channels + 8 (bank spread)
constexpr int kXBytes = (kPx + 2) * kXPitch * 2;
constexpr int kDCols = 27;             // (tap, ky, co) product columns
// accumulator rows (slot, row, channel) of 128 pixels: an odd pitch puts the
// rows the 27 columns of an MFMA tile add to in distinct banks
constexpr int kAccPitch = kPx + 1;
constexpr int kAccBytes = kNarrowSlots * 3 * 3 * kAccPitch * 4;
// LDS of a workgroup with nb staged-row buffers
constexpr int lds_bytes(int nb) { return nb * kXBytes + kAccBytes; }
static_assert(lds_bytes(2) <= 160 * 1024, "narrow conv LDS exceeds the CU's 160 KB");
static_assert(2 * lds_bytes(1) <= 160 * 1024, "two narrow conv workgroups exceed the CU's LDS");

// 16-bit blobs: two workgroups per CU, one staged-row buffer each (the
// workgroups' phases overlap); fp32 blobs, whose row loads take twice the
// registers: one workgroup with two buffers.
template <int KIND>
constexpr int buffers() { return KIND == 0 ? 2 : 1; }

struct NarrowArgs {
    const void* in;
    long in_cstep;
    int vec;            // rows allow 16-byte loads of 8-pixel runs
    int cin, cout, cpad, H, W;
    int prefix;         // padded frames before input frame 0
    int p_first;        // first padded frame read (the memory frames are in mem_in)
    int padded;         // padded frames
    int out_frames;
    const uint16_t* w;  // packed [cout][kp]
    long kp;
    const float* bias;
    void* out;
    long out_cstep;
    int out_kind;
    const float* mem_in;   // [2][cout][H][W] or null
    float* mem_out;        // [2][cout][H][W] or null
    int slots;             // output frames accumulated: out_frames (+ 2 with mem_out)
    int strips, bands, band_rows;
};

// One thread's share of a staged row: channels 8h..8h+7 at pixels
// x0 + 8g .. + 7 (16-bit blobs: one 16-byte run per channel; fp32: two),
// and one pixel of the halo.
template <int KIND>
struct RowLoad {
    uint4 v[KIND == 0 ? 16 : 8];
    uint32_t halo;
};

template <int KIND>
__device__ __forceinline__ float elem(const void* p, long i) {
    if (KIND == 1) return __uint_as_float((uint32_t)((const uint16_t*)p)[i] << 16);
    if (KIND == 2) return (float)((const _Float16*)p)[i];
    return ((const float*)p)[i];
}

template <int KIND>
__device__ __forceinline__ uint32_t elem_bits(const void* p, long i) {
    if (KIND == 0) return __float_as_uint(((const float*)p)[i]);
    return ((const uint16_t*)p)[i];
}

// 16-bit value of an element as staged (bf16)
template <int KIND>
__device__ __forceinline__ uint16_t to_bf16_bits(uint32_t raw) {
    if (KIND == 1) return (uint16_t)raw;
    if (KIND == 2) return __builtin_bit_cast(uint16_t, (__bf16)(float)__builtin_bit_cast(_Float16, (uint16_t)raw));
    return __builtin_bit_cast(uint16_t, (__bf16)__uint_as_float(raw));
}

template <int KIND, bool VEC>
__global__ __launch_bounds__(256, 3 - buffers<KIND>()) void conv3d_narrow_kernel(NarrowArgs a) {
    // one staged row of loads in flight (issued a step ahead; two rows ahead
    // measured no faster)
    constexpr int DIST = 1;
    constexpr int NB = buffers<KIND>();
    __shared__ __attribute__((aligned(16))) uint8_t lds[lds_bytes(NB)];
    uint16_t* const xs0 = (uint16_t*)lds;
    float* const acc = (float*)(lds + NB * kXBytes);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    // consecutive logical workgroups (the strips of a band, then the next
    // band) run on one XCD, so the halo pixels and rows a workgroup reads of
    // its neighbours' strips and bands come from that XCD's L2
    int bid = xcd_remap(blockIdx.x, gridDim.x);
    const int strip = bid % a.strips;
    bid /= a.strips;
    const int band = bid % a.bands;
    const int group = bid / a.bands;
    const int x0 = strip * kPx;
    const int y0 = band * a.band_rows;
    const int y1 = min(a.H, y0 + a.band_rows);
    const int s_lo = group * kNarrowSlots;
    const int s_hi = min(a.slots, s_lo + kNarrowSlots);
    const int ns = s_hi - s_lo;
    // padded frames that reach the slots: p = t + tap, tap 0..2
    const int p_lo = max(a.p_first, s_lo);
    const int p_hi = min(a.padded, s_hi + 2);
    const int nf = p_hi - p_lo;
    const int r_lo = max(y0 - 1, 0);
    const int r_hi = min(y1, a.H - 1);
    const int nsteps = nf > 0 ? (r_hi - r_lo + 1) * nf : 0;

    // weights of product column n = (tap * 3 + ky) * 3 + co at kx, k-step ks:
    // the MFMA B operand (8 consecutive channels of one column per lane)
    const int n = lane & 31;
    const int khalf = lane >> 5;
    const int col_co = n % 3, col_tap = n / 9, col_ky = (n / 3) % 3;
    const bool col_ok = n < kDCols && col_co < a.cout;
    bf16x8 wf[3][8];
    {
        const int co = n % 3, tk = n / 3;
#pragma unroll
        for (int kx = 0; kx < 3; ++kx)
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                uint4 u = make_uint4(0, 0, 0, 0);
                if (n < kDCols && co < a.cout && 16 * ks < a.cin)
                    u = *reinterpret_cast<const uint4*>(a.w + co * a.kp + (tk * 3 + kx) * a.cpad +
                                                        16 * ks + 8 * khalf);
                wf[kx][ks] = __builtin_bit_cast(bf16x8, u);
            }
    }

    // ---- loads of one staged row (step sp) into registers ----
    // Eight consecutive lanes hold eight channel groups of one pixel run and
    // the next eight the same groups of the next run: a load instruction
    // reads 128 contiguous bytes of each channel row (eight runs), and the
    // 16-byte LDS writes of sixteen lanes are two 128-byte halves of staged
    // pixels 8 apart, which fall in opposite halves of the banks.
    const int h = (tid & 7) + 8 * (tid >> 7);   // channels 8h .. 8h + 7
    const int g = (tid >> 3) & 15;              // pixels 8g .. 8g + 7 of the strip
    const int xg = x0 + 8 * g;
    const bool hvalid = 8 * h < a.cin;   // cin % 16 == 0: all eight channels or none
    // halo pixel of this thread (threads below 2 cin): channel tid / 2 at x0 - 1
    // or x0 + 128
    const int hx = (tid & 1) ? x0 + kPx : x0 - 1;
    const bool halo_ok = tid < 2 * a.cin && hx >= 0 && hx < a.W;
    const long halo_off = (long)min(tid >> 1, a.cin - 1) * a.in_cstep + min(max(hx, 0), a.W - 1);
    // byte offsets of this thread's loads from the start of a row (clamped
    // into the blob where the channel or the pixel run lies outside it)
    constexpr int kEsz = KIND == 0 ? 4 : 2;
    uint32_t voff[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        voff[i] = (uint32_t)(((long)min(8 * h + i, a.cin - 1) * a.in_cstep +
                              min(xg, a.W - (KIND == 0 ? 4 : 8))) * kEsz);
    // fp32: the second 16-byte run (pixels 4..7), relative to the first
    const uint32_t voff_hi = (uint32_t)((min(xg + 4, a.W - 4) - min(xg, a.W - 4)) * kEsz);
    const uint32_t halo_voff = (uint32_t)(halo_off * kEsz);
    auto issue = [&](int sp, RowLoad<KIND>& L) {
        if (VEC) {
            // Every load is issued, from a clamped address where the pixel
            // run or the channel lies outside the blob (stage zeroes those),
            // so that no load sits under a branch: the wait before a row is
            // staged then leaves the loads of the rows after it in flight.
            // Steps past the last reload the last row.
            // the row's base address is wave-uniform, the thread's channel
            // and pixel offset a 32-bit constant (the blob is below 4 GiB)
            const int spc = min(sp, nsteps - 1);
            const int yy = r_lo + spc / nf;
            const int pp = p_lo + spc % nf;
            const long row = ((long)max(pp - a.prefix, 0) * a.H + yy) * a.W;
            const char* rb = (const char*)a.in + row * (KIND == 0 ? 4 : 2);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (KIND == 0) {
                    L.v[2 * i] = *reinterpret_cast<const uint4*>(rb + voff[i]);
                    L.v[2 * i + 1] = *reinterpret_cast<const uint4*>(rb + voff[i] + voff_hi);
                } else {
                    L.v[i] = *reinterpret_cast<const uint4*>(rb + voff[i]);
                }
            }
            L.halo = KIND == 0 ? *reinterpret_cast<const uint32_t*>(rb + halo_voff)
                               : (uint32_t)*reinterpret_cast<const uint16_t*>(rb + halo_voff);
            return;
        }
        if (sp >= nsteps) return;
        const int yy = r_lo + sp / nf;
        const int pp = p_lo + sp % nf;
        const long row = ((long)max(pp - a.prefix, 0) * a.H + yy) * a.W;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int c = 8 * h + i;
            const long base = (long)c * a.in_cstep + row + xg;
            uint32_t e[8];
#pragma unroll
            for (int q = 0; q < 8; ++q)
                e[q] = c < a.cin && xg + q < a.W ? elem_bits<KIND>(a.in, base + q) : 0u;
            if (KIND == 0) {
                L.v[2 * i] = make_uint4(e[0], e[1], e[2], e[3]);
                L.v[2 * i + 1] = make_uint4(e[4], e[5], e[6], e[7]);
            } else {
                L.v[i] = make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16),
                                    e[6] | (e[7] << 16));
            }
        }
        L.halo = halo_ok ? elem_bits<KIND>(a.in, halo_off + row) : 0u;
    };
    // registers -> staged row buffer [pixel + 1][channel] bf16 (transposed)
    auto stage = [&](int sp, const RowLoad<KIND>& L, uint16_t* xs) {
        if (sp >= nsteps) return;
        if (hvalid) {
            // pixel runs past the frame's right edge are zeros
            const uint4 z = make_uint4(0, 0, 0, 0);
            const bool lo_ok = xg < a.W, hi_ok = KIND == 0 ? xg + 4 < a.W : lo_ok;
            uint32_t w[8][4];   // channel i, pixel pair d (bf16 pairs)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (KIND == 0) {
                    const uint4 lo = lo_ok ? L.v[2 * i] : z, hi = hi_ok ? L.v[2 * i + 1] : z;
                    w[i][0] = pack2_bf16_rne(__uint_as_float(lo.x), __uint_as_float(lo.y));
                    w[i][1] = pack2_bf16_rne(__uint_as_float(lo.z), __uint_as_float(lo.w));
                    w[i][2] = pack2_bf16_rne(__uint_as_float(hi.x), __uint_as_float(hi.y));
                    w[i][3] = pack2_bf16_rne(__uint_as_float(hi.z), __uint_as_float(hi.w));
                } else {
                    const uint4 v = lo_ok ? L.v[i] : z;
                    const uint32_t r[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        if (KIND == 2)
                            w[i][d] = (uint32_t)to_bf16_bits<2>(r[d] & 0xffffu) |
                                      ((uint32_t)to_bf16_bits<2>(r[d] >> 16) << 16);
                        else
                            w[i][d] = r[d];
                    }
                }
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                uint32_t o[4];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const uint32_t lo = w[2 * d][q >> 1], hi = w[2 * d + 1][q >> 1];
                    o[d] = (q & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
                }
                *reinterpret_cast<uint4*>(xs + (1 + 8 * g + q) * kXPitch + 8 * h) =
                    make_uint4(o[0], o[1], o[2], o[3]);
            }
        }
        if (tid < 2 * a.cin)
            xs[((tid & 1) ? kPx + 1 : 0) * kXPitch + (tid >> 1)] =
                halo_ok ? to_bf16_bits<KIND>(L.halo) : (uint16_t)0;
    };

    // ---- accumulator rows: slot (t - s_lo), row y % 3, channel, pixel ----
    // Item u + lane of a wave (u a multiple of 64, wave-uniform) has slot
    // u / 384, channel (u / 128) % 3 and pixel u % 128 + lane: the index
    // arithmetic runs on the scalar unit.
    const int wbase = __builtin_amdgcn_readfirstlane(tid & ~63);
    auto acc_at = [&](int ts, int y, int co) { return acc + ((ts * 3 + y % 3) * 3 + co) * kAccPitch; };
    float bias_r[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) bias_r[c] = a.bias && c < a.cout ? a.bias[c] : 0.f;
    // The memory's partial sums of output row y (slots 0 and 1, group 0):
    // element k of a thread is item wbase + 256 k + lane.  Loaded one step
    // before the row is initialised, ahead of that step's row loads, so that
    // waiting for them leaves those in flight.
    const bool has_mem = a.mem_in != nullptr && s_lo == 0;
    auto load_mem = [&](int y, float (&mv)[3]) {
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const int u = wbase + 256 * k;
            const int t = u / (3 * kPx), co = (u / kPx) % 3, x = x0 + u % kPx + lane;
            mv[k] = 0.f;
            if (has_mem && y < y1 && t < ns && co < a.cout && x < a.W)
                mv[k] = a.mem_in[((long)(t * a.cout + co) * a.H + y) * a.W + x];
        }
    };
    auto init_row = [&](int y, const float (&mv)[3]) {
        if (y >= y1) return;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const int u = wbase + 256 * k;
            if (u < ns * 3 * kPx) acc_at(u / (3 * kPx), y, (u / kPx) % 3)[u % kPx + lane] = mv[k];
        }
        for (int u = wbase + 768; u < ns * 3 * kPx; u += 256)
            acc_at(u / (3 * kPx), y, (u / kPx) % 3)[u % kPx + lane] = 0.f;
    };
    auto emit_row = [&](int y) {
        for (int u = wbase; u < ns * 3 * kPx; u += 256) {
            const int ts = u / (3 * kPx), co = (u / kPx) % 3, px = u % kPx + lane;
            const int t = s_lo + ts, x = x0 + px;
            if (co >= a.cout) continue;
            const float v = acc_at(ts, y, co)[px];
            if (x >= a.W) continue;
            if (t < a.out_frames) {
                const long o = (long)co * a.out_cstep + ((long)t * a.H + y) * a.W + x;
                const float r = v + (co == 0 ? bias_r[0] : co == 1 ? bias_r[1] : bias_r[2]);
                if (a.out_kind == 1)
                    ((uint16_t*)a.out)[o] = f32_to_bf16(r);
                else if (a.out_kind == 2)
                    ((_Float16*)a.out)[o] = f32_to_f16(r);
                else
                    ((float*)a.out)[o] = r;
            } else if (a.mem_out) {
                a.mem_out[((long)((t - a.out_frames) * a.cout + co) * a.H + y) * a.W + x] = v;
            }
        }
    };

    // staged channels at and above cin stay zero (the MFMAs read all 128)
    for (int i = tid; i < NB * kXBytes / 16; i += 256)
        reinterpret_cast<uint4*>(lds)[i] = make_uint4(0, 0, 0, 0);
    __syncthreads();
    for (int y = y0; y < min(y0 + 3, y1); ++y) {
        float mv[3];
        load_mem(y, mv);
        init_row(y, mv);
    }
    RowLoad<KIND> ring[DIST];
    issue(0, ring[0]);
    stage(0, ring[0], xs0);
#pragma unroll
    for (int d = 1; d <= DIST - 1; ++d) issue(d, ring[d % DIST]);
    __syncthreads();

    auto step = [&](int s, auto par) {
        constexpr int P = decltype(par)::value;
        const int yy = r_lo + s / nf;
        const int pp = p_lo + s % nf;
        // the last step of input row yy completes output row yy - 1, whose
        // accumulators then start output row yy + 2
        const bool row_end = s % nf == nf - 1 && yy - 1 >= y0 && yy - 1 < y1;
        float mv[3] = {0.f, 0.f, 0.f};
        if (row_end) load_mem(yy + 2, mv);
        // the loads of step s + depth go to the set step s's data came from
        issue(s + DIST, ring[(P + DIST) % DIST]);
        const uint16_t* xs = xs0 + (P % NB) * (kXBytes / 2);
        // all 128 staged channels (those at and above cin are zeros, with
        // zero weights): two accumulators, so that consecutive MFMAs do not
        // wait on each other
        f32x16 d0 = {}, d1 = {};
#pragma unroll
        for (int kx = 0; kx < 3; ++kx)
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                const uint4 u = *reinterpret_cast<const uint4*>(
                    xs + (32 * wave + (lane & 31) + kx) * kXPitch + 16 * ks + 8 * khalf);
                if (ks & 1)
                    d1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, u),
                                                                 wf[kx][ks], d1, 0, 0, 0);
                else
                    d0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, u),
                                                                 wf[kx][ks], d0, 0, 0, 0);
            }
        const f32x16 d = d0 + d1;
        // out(t, y', x, co) += D[x][(tap, ky, co)], t = p - tap, y' = row - ky + 1.
        // Lane l holds column l % 32 of pixels 32 wave + 8(r/4) + 4(l/32) + r%4
        // (register r) and adds them to its target row in LDS: within a step
        // the columns' targets are distinct and the waves' pixels disjoint, so
        // no two lanes read or write one element.
        {
            const int t = pp - col_tap, yo = yy - col_ky + 1;
            if (col_ok && t >= s_lo && t < s_hi && yo >= y0 && yo < y1) {
                float* dst = acc_at(t - s_lo, yo, col_co) + 32 * wave + 4 * khalf;
                float v[16];
#pragma unroll
                for (int r = 0; r < 16; ++r) v[r] = dst[8 * (r >> 2) + (r & 3)];
#pragma unroll
                for (int r = 0; r < 16; ++r) dst[8 * (r >> 2) + (r & 3)] = v[r] + d[r];
            }
        }
        // one buffer: every wave is done with the staged row before the next
        // one overwrites it
        if (NB == 1) __syncthreads();
        stage(s + 1, ring[(P + 1) % DIST], xs0 + ((P + 1) % NB) * (kXBytes / 2));
        __syncthreads();
        if (row_end) {
            // every add of the row is in (the barrier above)
            emit_row(yy - 1);
            init_row(yy + 2, mv);
            __syncthreads();
        }
    };
    for (int s = 0; s < nsteps; s += 2) {
        step(s, std::integral_constant<int, 0>{});
        if (s + 1 < nsteps) step(s + 1, std::integral_constant<int, 1>{});
    }
    __syncthreads();
    // rows whose last input row is the frame's last row
    for (int e = max(y0, r_hi); e < y1; ++e) emit_row(e);
}

int narrow_cus() {
    static std::mutex mu;
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if (!cus[dev] &&
        hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus[dev] = 256;
    return cus[dev];
}

}  // namespace

hipError_t launch_conv3d_narrow(const Conv3dShape& s, const void* input, int in_kind,
                                long in_cstep, int frames, int height, int width, int prefix,
                                int mem, int out_frames, const uint16_t* packed, const float* bias,
                                void* out, int out_kind, long out_cstep, const float* mem_in,
                                float* mem_out, hipStream_t stream) {
    if (!conv3d_narrow(s) || frames <= 0 || height <= 0 || width <= 0 || out_frames <= 0 ||
        (mem != 0 && mem != 2) || (mem && !mem_in))
        return hipErrorInvalidValue;
    NarrowArgs a;
    a.in = input;
    a.in_cstep = in_cstep;
    const size_t esz = in_kind == 0 ? 4 : 2;
    a.vec = (uintptr_t)input % 16 == 0 && in_cstep % (16 / esz) == 0 && width % (16 / esz) == 0;
    a.cin = s.cin;
    a.cout = s.cout;
    a.cpad = s.cpad;
    a.H = height;
    a.W = width;
    a.prefix = prefix;
    a.p_first = mem;
    a.padded = frames + prefix;
    a.out_frames = out_frames;
    a.w = packed;
    a.kp = conv3d_kp(s);
    a.bias = bias;
    a.out = out;
    a.out_cstep = out_cstep;
    a.out_kind = out_kind;
    a.mem_in = mem ? mem_in : nullptr;
    a.mem_out = mem_out;
    a.slots = out_frames + (mem_out ? 2 : 0);
    if (a.padded != out_frames + 2) return hipErrorInvalidValue;
    a.strips = (width + kPx - 1) / kPx;
    const int groups = (a.slots + kNarrowSlots - 1) / kNarrowSlots;
    // about as many workgroups as fit on the chip at once (two a CU for
    // 16-bit blobs): bands of rows, each read with one row of halo above and
    // below
    const int cus = narrow_cus() * (in_kind == 0 ? 1 : 2);
    const int bands = std::max(1, std::min(height, cus / std::max(1, a.strips * groups)));
    a.band_rows = (height + bands - 1) / bands;
    a.bands = (height + a.band_rows - 1) / a.band_rows;
    const long blocks = (long)a.strips * a.bands * groups;
    if (blocks > INT_MAX) return hipErrorInvalidValue;
    const dim3 grid((unsigned)blocks);
    if (in_kind == 1)
        a.vec ? conv3d_narrow_kernel<1, true><<<grid, 256, 0, stream>>>(a)
              : conv3d_narrow_kernel<1, false><<<grid, 256, 0, stream>>>(a);
    else if (in_kind == 2)
        a.vec ? conv3d_narrow_kernel<2, true><<<grid, 256, 0, stream>>>(a)
              : conv3d_narrow_kernel<2, false><<<grid, 256, 0, stream>>>(a);
    else
        a.vec ? conv3d_narrow_kernel<0, true><<<grid, 256, 0, stream>>>(a)
              : conv3d_narrow_kernel<0, false><<<grid, 256, 0, stream>>>(a);
    return hipGetLastError();
}

}  // namespace s2
