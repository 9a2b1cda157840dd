// The DiT block's norm and AdaSingle modulation as ncnn layers over the
// s2_dit_ada_* C-ABI, for block graphs run by ncnn::Net (ncnn/net.h).
//
// In the reference these operations are ncnn built-ins inside the exported
// seedvr2_blocks .param (not in the reference repository); the block graph
// takes their six per-sample vectors as inputs in4..in9, [batch][hidden]
// fp32 (src/seedvr2/seedvr2_dit.cpp:441-448, 734-738).  Here each of the
// three fused passes is one layer:
//
//   DiTAdaIn     bottoms x_video, x_text, shift, scale      tops h_video, h_text
//                h = rmsnorm(x) * (scale[b] + scale_s) + (shift[b] + shift_s)
//   DiTAdaOut    bottoms x_video, x_text, y_video, y_text, gate
//                tops    out_video, out_text
//                out = x + y * (gate[b] + gate_s)
//   DiTAdaOutIn  bottoms x_video, x_text, y_video, y_text, gate, shift, scale
//                tops    out_video, out_text, h_video, h_text
//                DiTAdaOut, then DiTAdaIn on its output, in one pass
//
// Params: 0 hidden, 1 epsilon (default 1e-5), 2 stream vectors (0 none, 1:
// the block's own [hidden] per-stream vectors follow in the .bin as raw fp32,
// DiTAdaIn: video_shift, video_scale, text_shift, text_scale; DiTAdaOut:
// video_gate, text_gate; DiTAdaOutIn: the gates then the four of DiTAdaIn).
// Rows per sample come from the AdaptiveWindowRuntimeState the creator takes
// as userdata (t*h*w video and text_length rows of each sample), the state
// the graph's AdaptiveWindowAttention layers read.  Blobs are device blobs
// (HipDeviceAllocator): x and out in their element type, h in 16 bits under
// use_bf16_storage / use_fp16_storage and fp32 otherwise.  Return codes are
// the reference layers' 0 / -1 / -100.
#ifndef SEEDVR2_DIT_BLOCK_OPS_H
#define SEEDVR2_DIT_BLOCK_OPS_H

#include <mutex>
#include <vector>

#include <layer.h>

#include "adaptive_window_attention.h"
#include "hip_allocator.h"

namespace seedvr2 {

class DiTBlockOp : public ncnn::Layer
{
public:
    // kind: 0 DiTAdaIn, 1 DiTAdaOut, 2 DiTAdaOutIn
    DiTBlockOp(int kind, const AdaptiveWindowRuntimeState* state);
    virtual ~DiTBlockOp();

    virtual int load_param(const ncnn::ParamDict& pd);
    virtual int load_model(const ncnn::ModelBin& mb);
    virtual int create_pipeline(const ncnn::Option& opt);
    virtual int destroy_pipeline(const ncnn::Option& opt);
    virtual int forward(const std::vector<ncnn::Mat>& bottom_blobs,
                        std::vector<ncnn::Mat>& top_blobs,
                        const ncnn::Option& opt) const;

private:
    int upload_locked() const;

    int kind;
    const AdaptiveWindowRuntimeState* state;
    int hidden;
    float epsilon;
    int stream_vectors;
    std::vector<ncnn::Mat> vectors;   // host copies, in .bin order

    mutable std::mutex mutex;
    mutable DeviceBuffer vectors_gpu;   // the same, fp32 [count][hidden]
    mutable bool dirty;
};

// One token stream's pass, made by the graph fold (dit_block_fold.h) from
// a chain of ncnn built-ins:
//   kind 0 ada_in      bottoms x, shift, scale           top  h
//   kind 1 ada_out     bottoms x, y, gate                top  out
//   kind 2 ada_out_in  bottoms x, y, gate, shift, scale  tops out, h
// with the arithmetic of DiTBlockOp.  stream 0 is the video stream, 1 the
// text stream: its rows per sample come from the runtime state.  hidden is
// the width of x.  The block's own [hidden] vectors of the stream (gate,
// shift, scale; empty Mats for none) come from the chain's MemoryData.
class DiTStreamOp : public ncnn::Layer
{
public:
    DiTStreamOp(int kind, int stream, const AdaptiveWindowRuntimeState* state, float epsilon,
                const ncnn::Mat& gate, const ncnn::Mat& shift, const ncnn::Mat& scale);
    virtual ~DiTStreamOp();

    virtual int create_pipeline(const ncnn::Option& opt);
    virtual int destroy_pipeline(const ncnn::Option& opt);
    virtual int forward(const std::vector<ncnn::Mat>& bottom_blobs,
                        std::vector<ncnn::Mat>& top_blobs,
                        const ncnn::Option& opt) const;

    int kind_of() const { return kind; }
    int stream_of() const { return stream; }
    float epsilon_of() const { return epsilon; }
    const ncnn::Mat& vector(int i) const { return vectors[i]; }   // 0 gate, 1 shift, 2 scale

private:
    int upload_locked() const;

    int kind;
    int stream;
    const AdaptiveWindowRuntimeState* state;
    float epsilon;
    ncnn::Mat vectors[3];

    mutable std::mutex mutex;
    mutable DeviceBuffer vectors_gpu;   // [3][hidden] fp32, a slot per present vector
    mutable bool dirty;
};

ncnn::Layer* dit_ada_in_layer_creator(void* userdata);
ncnn::Layer* dit_ada_out_layer_creator(void* userdata);
ncnn::Layer* dit_ada_out_in_layer_creator(void* userdata);
void dit_block_op_layer_destroyer(ncnn::Layer* layer, void* userdata);

}  // namespace seedvr2

#endif  // SEEDVR2_DIT_BLOCK_OPS_H
