// The fused DiT block graph on MI355X: an ncnn::Net (ncnn/net.h) with the
// SeedVR2 custom layers registered, run on device-resident blobs.
//
// The reference's BlockGraph (src/seedvr2/seedvr2_dit.cpp:603-633) registers
// AdaptiveWindowAttention with a runtime-state userdata and SharedLinear,
// loads blocks/seedvr2_blocks.ncnn.param/.bin, and for each denoising step
// sets the runtime state's shapes, feeds in0 (video), in1 (text), in2
// (video_shape), in3 (text_length) and in4..in9 (the six modulation vectors)
// to an extractor, and extracts out0/out1 and, optionally, the video and text
// boundary blobs of chosen blocks (:722-833).  This class does the same with
// its own HipDeviceAllocator as the extractor's blob allocator, so every
// blob between two layers stays in HBM and only in0..in9 are uploaded when
// they are host Mats (in2 / in3 stay on the host).  Device inputs of another
// HipDeviceAllocator may come from another stream: the graph's stream waits
// for that stream's work enqueued before run(), and every layer runs on the
// graph's stream.  Outputs are ready once the graph's stream has run.  It
// also registers the block's norm/modulation layers (DiTAdaIn, DiTAdaOut,
// DiTAdaOutIn, dit_block_ops.h) with the same runtime state, and folds
// SharedLinear -> GELU pairs into the GEMM epilogue.
#ifndef SEEDVR2_DIT_BLOCK_GRAPH_H
#define SEEDVR2_DIT_BLOCK_GRAPH_H

#include <array>
#include <string>
#include <vector>

#include <net.h>

#include "adaptive_window_attention.h"
#include "hip_allocator.h"

namespace seedvr2 {

class DiTBlockGraph
{
public:
    // stream: the hipStream_t (as void*) every layer of the graph runs on.
    explicit DiTBlockGraph(void* stream = 0);
    ~DiTBlockGraph();

    // Registers the layers and loads the graph; the 16-bit storage option
    // (bf16 blobs between the GEMMs and the attention) is on unless
    // fp32_blobs.  fuse_gelu folds SharedLinear -> GELU pairs; fuse_qkv (bf16
    // blobs only) folds each QKV SharedLinear into the attention layer it
    // feeds (ncnn::Net::fuse_qkv_attention), and the split q / k / v
    // projections of v3 graphs likewise (fuse_split_qkv_attention), so the
    // QKV blobs cannot be extracted as checkpoints; with bf16 blobs
    // fuse_gelu also folds gate / up / Swish / mul chains into one SwiGLU
    // projection (fuse_swiglu); fold_modulation folds norm / modulation /
    // residual chains written with ncnn built-ins (dit_block_fold.h).
    // Returns 0 or the first failing code of load_param / load_model.
    int load(const char* param_path, const char* model_path, bool fp32_blobs = false,
             bool fuse_gelu = true, bool fuse_qkv = true, bool fold_modulation = true);
    int load_mem(const char* param_text, const unsigned char* model, size_t model_bytes,
                 bool fp32_blobs = false, bool fuse_gelu = true, bool fuse_qkv = true,
                 bool fold_modulation = true);

    // One pass of the graph.  inputs[0..9] are in0..in9 (host or device
    // Mats); out_video / out_text receive out0 / out1 as device blobs of this
    // graph's allocator, valid until the next run() or clear_blobs().
    // checkpoints (optional): names of further blobs to extract, returned in
    // checkpoint_blobs in the same order.
    int run(const std::vector<std::array<int, 3> >& video_shapes,
            const std::vector<int>& text_lengths, const ncnn::Mat inputs[10],
            ncnn::Mat& out_video, ncnn::Mat& out_text,
            const std::vector<std::string>* checkpoints = 0,
            std::vector<ncnn::Mat>* checkpoint_blobs = 0);

    // Frees every device blob the graph's allocator holds.
    void clear_blobs();

    int fused_gelu_count() const { return fused_gelu; }
    int fused_qkv_count() const { return fused_qkv; }
    int folded_modulation_count() const { return folded_modulation; }
    int fused_swiglu_count() const { return fused_swiglu; }
    HipDeviceAllocator& allocator() { return alloc; }
    ncnn::Net net;
    AdaptiveWindowRuntimeState runtime_state;

private:
    int register_layers();

    HipDeviceAllocator alloc;
    int fused_gelu;
    int fused_qkv;
    int folded_modulation;
    int fused_swiglu;
    int finish_load(int ret, bool fp32_blobs, bool fuse_gelu, bool fuse_qkv, bool fold_modulation);
    std::vector<void*> last_blocks;   // uploads and outputs of the last run
};

}  // namespace seedvr2

#endif  // SEEDVR2_DIT_BLOCK_GRAPH_H
