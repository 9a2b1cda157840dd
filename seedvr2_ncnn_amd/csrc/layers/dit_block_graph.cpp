// The fused DiT block graph on MI355X (dit_block_graph.h).
#include "dit_block_graph.h"

#include <stdio.h>

#include "dit_block_ops.h"
#include "seedvr2_hip.h"
#include "shared_linear.h"

namespace seedvr2 {

DiTBlockGraph::DiTBlockGraph(void* stream) : alloc(stream), fused_gelu(0), fused_qkv(0) {}

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
                        bool fuse_gelu, bool fuse_qkv)
{
    net.clear();
    net.opt.use_bf16_storage = !fp32_blobs;
    net.opt.use_fp16_storage = false;
    int ret = register_layers();
    if (ret == 0)
        ret = net.load_param(param_path);
    if (ret == 0)
        ret = net.load_model(model_path);
    fused_gelu = (ret == 0 && fuse_gelu) ? net.fuse_shared_linear_gelu() : 0;
    fused_qkv = (ret == 0 && fuse_qkv && !fp32_blobs) ? net.fuse_qkv_attention() : 0;
    return ret;
}

int DiTBlockGraph::load_mem(const char* param_text, const unsigned char* model,
                            size_t model_bytes, bool fp32_blobs, bool fuse_gelu, bool fuse_qkv)
{
    net.clear();
    net.opt.use_bf16_storage = !fp32_blobs;
    net.opt.use_fp16_storage = false;
    int ret = register_layers();
    if (ret == 0)
        ret = net.load_param_mem(param_text);
    if (ret == 0)
        ret = net.load_model(model, model_bytes);
    fused_gelu = (ret == 0 && fuse_gelu) ? net.fuse_shared_linear_gelu() : 0;
    fused_qkv = (ret == 0 && fuse_qkv && !fp32_blobs) ? net.fuse_qkv_attention() : 0;
    return ret;
}

// The extractor sequence of seedvr2_dit.cpp:722-833 on device blobs.
int DiTBlockGraph::run(const std::vector<std::array<int, 3> >& video_shapes,
                       const std::vector<int>& text_lengths, const ncnn::Mat inputs[10],
                       ncnn::Mat& out_video, ncnn::Mat& out_text,
                       const std::vector<std::string>* checkpoints,
                       std::vector<ncnn::Mat>* checkpoint_blobs)
{
    // the previous run's uploads and outputs go back to the pool (the
    // kernels that will reuse them run after that run's, on the same stream)
    for (size_t i = 0; i < last_blocks.size(); i++)
        alloc.release_blob(last_blocks[i]);
    last_blocks.clear();
    runtime_state.video_shapes = video_shapes;
    runtime_state.text_lengths = text_lengths;
    ncnn::Extractor ex = net.create_extractor();
    ex.set_light_mode(true);
    ex.set_blob_allocator(&alloc);
    ex.set_workspace_allocator(&alloc);
    int ret = 0;
    for (int i = 0; ret == 0 && i < 10; i++)
    {
        char name[8];
        snprintf(name, sizeof(name), "in%d", i);
        ncnn::Mat m = inputs[i];
        // in2 / in3 (video_shape, text_length) stay where they are: the
        // attention layers read host shape blobs on the host
        if (i != 2 && i != 3 && !device_allocator_of(m) && m.dims == 2 && !m.empty() &&
            (m.elemsize == 4 || m.elemsize == 2))
        {
            // a host blob: one upload on the graph's stream
            m = alloc.create_blob(m.w, m.h, m.elemsize);
            if (m.empty())
                return -100;
            last_blocks.push_back(m.data);
            ret = s2_memcpy_h2d(m.data, inputs[i].data, (size_t)m.w * m.h * m.elemsize,
                                alloc.stream());
            if (ret != 0)
                return layer_status(ret);
        }
        ret = ex.input(name, m);
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
