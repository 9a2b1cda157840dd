// Host launchers of the DecomposedConv3D kernels (conv3d_kernels.hip).
//
// The convolution runs as an implicit GEMM over a staged copy of its input:
// the temporally padded frames in channel-last bf16, [frame][y][x][cpad]
// (conv3d_cpad: zero channels above num_input).  Weights are packed once to
// bf16 [num_output][kp], k = window position * cpad + channel, the same k
// order, so both MFMA operands are k-contiguous.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace s2 {

struct Conv3dShape {
    int cin, cout, cpad;
    int kt, kh, kw;
    int st, sh, sw;
    int dt, dh, dw;
    int ph, pw;
};

// Channels per staged pixel: 8, 16 or 32 for layers of at most 32 input
// channels (a 64-wide k-step then spans several window positions), else
// num_input rounded up to 64.
inline int conv3d_cpad(int cin) {
    return cin <= 8 ? 8 : cin <= 16 ? 16 : cin <= 32 ? 32 : (cin + 63) / 64 * 64;
}
// The halo kernel takes layers with a 3x3 spatial window of unit stride and
// dilation and at least 16 input channels, in tiles 128 or 64 output columns
// wide, whichever the output width fills to at least 93% (128 first): below
// that, enough MFMA work falls past the frame that the implicit-GEMM kernel
// is faster.  Returns the tile width, or 0 for the implicit-GEMM kernel.
inline int conv3d_halo_width(const Conv3dShape& s, int wo) {
    if (s.kh != 3 || s.kw != 3 || s.sh != 1 || s.sw != 1 || s.dh != 1 || s.dw != 1 ||
        s.cpad % 16 != 0 || wo <= 0)
        return 0;
    for (int tw = 128; tw >= 64; tw /= 2)
        if ((long)(wo + tw - 1) / tw * tw * 100 <= (long)wo * 107) return tw;
    return 0;
}
inline bool conv3d_halo_ok(const Conv3dShape& s, int wo) { return conv3d_halo_width(s, wo) > 0; }
// Output tiles of the implicit-GEMM kernel for m output pixels.
inline long conv3d_gemm_tiles(const Conv3dShape& s, long m) {
    if (s.cout <= 128) return (m + 511) / 512 * ((s.cout + 127) / 128);
    return (m + 255) / 256 * ((s.cout + 255) / 256);
}
// Ranges the implicit-GEMM kernel splits its k loop into (one workgroup per
// range and tile, partial tiles summed by a second pass) when its tiles
// would leave most of the chip idle: layers of at least 64 input channels
// with fewer tiles than the CUs (256 on MI355X).  The count of the fewest
// rounds of workgroups per k-step: s ranges of a tiles-tile layer take
// ceil(tiles * s / 256) rounds of 1/s of the loop; the smallest such s up to
// 8 (more partial tiles cost more than they fill).  1: no split.
inline int conv3d_k_split(const Conv3dShape& s, long m, int wo) {
    if (s.cpad < 64 || conv3d_halo_width(s, wo) > 0) return 1;
    const long tiles = conv3d_gemm_tiles(s, m);
    if (tiles >= 256) return 1;
    const long steps = (long)s.kt * s.kh * s.kw * (s.cpad / 64);
    int best = 1;
    double best_t = 1.0;
    for (int sp = 2; sp <= 8 && sp <= steps; ++sp) {
        const double t = (double)((tiles * sp + 255) / 256) / sp;
        if (t < best_t - 1e-9) {
            best = sp;
            best_t = t;
        }
    }
    return best;
}
// Packed weight row length: window positions x cpad, rounded up to 64.
inline long conv3d_kp(const Conv3dShape& s) {
    return ((long)s.kt * s.kh * s.kw * s.cpad + 63) / 64 * 64;
}

// planar input [cin][frames*H*W] (channel stride in_cstep; element type
// in_kind: 0 fp32, 1 bf16, 2 fp16) -> staged [frames*H*W][cpad] bf16.  When
// tail is non-null, pixels tail_q0.. are also written to tail (the next
// temporal memory).
hipError_t launch_conv3d_stage(const void* input, int in_kind, long in_cstep, int cin,
                               long pixels, int cpad, uint16_t* staged, uint16_t* tail,
                               long tail_q0, hipStream_t stream);
// fp32 [kt][cout][cin][kh][kw] -> bf16 [cout][kp] (conv3d_kp)
hipError_t launch_conv3d_pack_weights(const float* weights, const Conv3dShape& s,
                                      uint16_t* packed, hipStream_t stream);
// Output frames [t0, t0 + frames_out) of the convolution.  Padded frame p
// (p = t*st + tap*dt) is frame v = max(p - shift, 0) of [memory | input]:
// memory frame v when v < mem (memory holds mem frames, memory_bytes), else
// input frame v - mem, at frame v - mem - frame_base of `staged` (which must
// hold every input frame these outputs read).  Both buffers < 2 GiB; mem > 0
// needs ho*wo % 8 == 0.  out: planar [cout][...], element (co, t, y, x) at
// co*out_cstep + (t*Ho + y)*Wo + x, type out_kind; bias fp32 [cout] or null.
// part: fp32 scratch of conv3d_k_split(s, frames_out*ho*wo, wo) x cout x
// frames_out*ho*wo floats for the split k loop, or null (no split).
hipError_t launch_conv3d(const Conv3dShape& s, const uint16_t* memory, int mem,
                         size_t memory_bytes, const uint16_t* staged, size_t staged_bytes,
                         int frame_base, int shift, int height, int width, int ho, int wo,
                         int t0, int frames_out, const uint16_t* packed, const float* bias,
                         void* out, int out_kind, long out_cstep, float* part,
                         hipStream_t stream);

// Layers of at most 3 output channels with a 3x3x3 window, unit strides and
// dilations, one pixel of spatial padding and 16..128 input channels (a
// multiple of 16) run conv3d_narrow_kernels.hip: the window positions are the
// MFMA columns and the temporal memory holds partial sums of the next
// forward's first two output frames, [2][cout][H][W] fp32, instead of input
// frames.
inline bool conv3d_narrow(const Conv3dShape& s) {
    return s.cout <= 3 && s.cin >= 16 && s.cin <= 128 && s.cin % 16 == 0 && s.kt == 3 &&
           s.kh == 3 && s.kw == 3 && s.st == 1 && s.sh == 1 && s.sw == 1 && s.dt == 1 &&
           s.dh == 1 && s.dw == 1 && s.ph == 1 && s.pw == 1;
}
// output frames one narrow-conv workgroup accumulates (more: several groups)
constexpr int kNarrowSlots = 6;
// Narrow conv over `frames` planar input frames (channel stride in_cstep,
// type in_kind) of height x width: padded frame p is input frame
// max(p - prefix, 0); mem = 2 with mem_in the previous forward's partial sums
// (prefix 2, the memory frames not read), mem = 0 without (prefix =
// head_frames).  out_frames = frames + prefix - 2.  mem_out (or null)
// receives the partial sums for the next forward; it must not be mem_in when
// out_frames + 2 > kNarrowSlots (workgroups of different output frames read
// and write the memory concurrently).
hipError_t launch_conv3d_narrow(const Conv3dShape& s, const void* input, int in_kind,
                                long in_cstep, int frames, int height, int width, int prefix,
                                int mem, int out_frames, const uint16_t* packed, const float* bias,
                                void* out, int out_kind, long out_cstep, const float* mem_in,
                                float* mem_out, hipStream_t stream);

// VAEUpsample3D's shuffle: packed [channels*tr*sr*sr][frames][h][w] (channel
// stride packed_cstep) -> out [channels][frames*tr - remove_head][h*sr][w*sr]
// (channel stride out_cstep), elements of type kind (0 fp32; 1, 2 16-bit)
hipError_t launch_vae_shuffle(const void* packed, int kind, long packed_cstep, int channels,
                              int frames, int h, int w, int tr, int sr, int remove_head,
                              void* out, long out_cstep, hipStream_t stream);

}  // namespace s2
