// The fused DiT block graph on MI355X (dit_block_graph.h).
#include "dit_block_graph.h"

#include <stdio.h>

#include "dit_block_fold.h"
#include "dit_block_ops.h"
#include "seedvr2_hip.h"
#include "shared_linear.h"

namespace seedvr2 {

DiTBlockGraph::DiTBlockGraph(void* stream)
    : alloc(stream), fused_gelu(0), fused_qkv(0), folded_modulation(0), fused_swiglu(0)
{
}

DiTBlockGraph::~DiTBlockGraph()
{
    net.clear();
    alloc.clear();
}

// The registrations of seedvr2_dit.cpp:614-618, plus the block's
// norm/modulation layers, all sharing the runtime state.
int DiTBlockGraph::register_layers()
{
    int ret = net.register_custom_layer("AdaptiveWindowAttention",
                                        adaptive_window_attention_layer_creator,
                                        adaptive_window_attention_layer_destroyer, &runtime_state);
    if (ret == 0)
        ret = net.register_custom_layer("SharedLinear", shared_linear_layer_creator,
                                        shared_linear_layer_destroyer);
    if (ret == 0)
        ret = net.register_custom_layer("DiTAdaIn", dit_ada_in_layer_creator,
                                        dit_block_op_layer_destroyer, &runtime_state);
    if (ret == 0)
        ret = net.register_custom_layer("DiTAdaOut", dit_ada_out_layer_creator,
                                        dit_block_op_layer_destroyer, &runtime_state);
    if (ret == 0)
        ret = net.register_custom_layer("DiTAdaOutIn", dit_ada_out_in_layer_creator,
                                        dit_block_op_layer_destroyer, &runtime_state);
    return ret;
}

int DiTBlockGraph::load(const char* param_path, const char* model_path, bool fp32_blobs,
                        bool fuse_gelu, bool fuse_qkv, bool fold_modulation)
{
    net.clear();
    net.opt.use_bf16_storage = !fp32_blobs;
    net.opt.use_fp16_storage = false;
    int ret = register_layers();
    if (ret == 0)
        ret = net.load_param(param_path);
    if (ret == 0)
        ret = net.load_model(model_path);
    return finish_load(ret, fp32_blobs, fuse_gelu, fuse_qkv, fold_modulation);
}

int DiTBlockGraph::load_mem(const char* param_text, const unsigned char* model,
                            size_t model_bytes, bool fp32_blobs, bool fuse_gelu, bool fuse_qkv,
                            bool fold_modulation)
{
    net.clear();
    net.opt.use_bf16_storage = !fp32_blobs;
    net.opt.use_fp16_storage = false;
    int ret = register_layers();
    if (ret == 0)
        ret = net.load_param_mem(param_text);
    if (ret == 0)
        ret = net.load_model(model, model_bytes);
    return finish_load(ret, fp32_blobs, fuse_gelu, fuse_qkv, fold_modulation);
}

// The graph folds, in an order where none hides another's pattern.
int DiTBlockGraph::finish_load(int ret, bool fp32_blobs, bool fuse_gelu, bool fuse_qkv,
                               bool fold_modulation)
{
    fused_gelu = fused_qkv = folded_modulation = fused_swiglu = 0;
    if (ret != 0)
        return ret;
    if (fuse_gelu)
        fused_gelu = net.fuse_shared_linear_gelu();
    if (fuse_gelu && !fp32_blobs)   // the SwiGLU epilogue takes bf16 activations
        fused_swiglu = net.fuse_swiglu();
    if (fold_modulation)
        folded_modulation = fold_dit_modulation(net, &runtime_state);
    if (fuse_qkv && !fp32_blobs)
        fused_qkv = net.fuse_qkv_attention() + net.fuse_split_qkv_attention();
    return 0;
}

// The extractor sequence of seedvr2_dit.cpp:722-833 on device blobs.
int DiTBlockGraph::run(const std::vector<std::array<int, 3> >& video_shapes,
                       const std::vector<int>& text_lengths, const ncnn::Mat inputs[10],
                       ncnn::Mat& out_video, ncnn::Mat& out_text,
                       const std::vector<std::string>* checkpoints,
                       std::vector<ncnn::Mat>* checkpoint_blobs)
{
    // The previous run's outputs go back to the pool (the kernels that will
    // reuse them run after that run's, on the same stream), except those fed
    // back as inputs of this run (a denoising loop's out0 -> in0): they are
    // released after the run that reads them.
    std::vector<void*> still_read;
    for (size_t i = 0; i < last_blocks.size(); i++)
    {
        bool input = false;
        for (int j = 0; j < 10; j++)
            input = input || inputs[j].data == last_blocks[i];
        if (input)
            still_read.push_back(last_blocks[i]);
        else
            alloc.release_blob(last_blocks[i]);
    }
    last_blocks.swap(still_read);
    runtime_state.video_shapes = video_shapes;
    runtime_state.text_lengths = text_lengths;
    ncnn::Extractor ex = net.create_extractor();
    ex.set_light_mode(true);
    ex.set_blob_allocator(&alloc);
    ex.set_workspace_allocator(&alloc);
    // Host inputs are uploaded once by the extractor on this graph's stream,
    // except in2 / in3 (video_shape, text_length), which the attention layers
    // read on the host; device inputs of another allocator are ordered
    // behind that allocator's stream (ncnn::Extractor::input).
    int ret = 0;
    for (int i = 0; ret == 0 && i < 10; i++)
    {
        char name[8];
        snprintf(name, sizeof(name), "in%d", i);
        ret = ex.input(name, inputs[i]);
    }
    if (ret == 0 && checkpoints)
    {
        checkpoint_blobs->assign(checkpoints->size(), ncnn::Mat());
        for (size_t i = 0; ret == 0 && i < checkpoints->size(); i++)
            ret = ex.extract((*checkpoints)[i].c_str(), (*checkpoint_blobs)[i]);
    }
    if (ret == 0)
        ret = ex.extract("out0", out_video);
    if (ret == 0)
        ret = ex.extract("out1", out_text);
    if (ret == 0)
    {
        last_blocks.push_back(out_video.data);
        last_blocks.push_back(out_text.data);
        for (size_t i = 0; checkpoint_blobs && i < checkpoint_blobs->size(); i++)
            last_blocks.push_back((*checkpoint_blobs)[i].data);
    }
    return ret;
}

void DiTBlockGraph::clear_blobs()
{
    last_blocks.clear();
    alloc.clear();
}

}  // namespace seedvr2
