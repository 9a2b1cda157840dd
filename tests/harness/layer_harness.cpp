// Test harness: drives the ncnn-surface layers (AdaptiveWindowAttention,
// SharedLinear, DecomposedConv3D, VAEChunkedMHA) the way an ncnn Net does -- creator, load_param from a .param
// field string, load_model from raw weight bytes, create_pipeline, forward --
// and exposes that to the Python tests through a few extern "C" calls.
// Test infrastructure only; built into tests/harness/liblayer_harness.so.
#include <string.h>

#include <array>
#include <string>
#include <vector>

#include <layer.h>
#include <net.h>
#include <modelbin.h>
#include <paramdict.h>

#include "adaptive_window_attention.h"
#include "decomposed_conv3d.h"
#include "dit_block_graph.h"
#include "hip_allocator.h"
#include "seedvr2_hip.h"
#include "shared_linear.h"
#include "vae_chunked_mha.h"
#include "vae_resample3d.h"

namespace {

seedvr2::HipDeviceAllocator& device_allocator() {
    static seedvr2::HipDeviceAllocator alloc(0);
    return alloc;
}

struct Handle {
    ncnn::Layer* layer;
    ncnn::layer_destroyer_func destroyer;
    seedvr2::AdaptiveWindowRuntimeState state;
    ncnn::Option opt;
};

}  // namespace

extern "C" {

typedef struct h_blob {
    int dims;       // 0 = empty blob, 1 or 2
    int w, h;
    int elemsize;   // 4 fp32 / int32, 2 bf16 or fp16
    int device;     // data is a device pointer
    void* data;
} h_blob;

// type: "AdaptiveWindowAttention" or "SharedLinear"; params: the id=value
// fields of a .param line; model: raw weight bytes (nullptr/0: skip
// load_model).  Returns load_param's or load_model's code.
int h_layer_create(const char* type, const char* params, const void* model, long model_bytes,
                   void** out) {
    *out = 0;
    Handle* h = new Handle();
    if (strcmp(type, "AdaptiveWindowAttention") == 0) {
        h->layer = seedvr2::adaptive_window_attention_layer_creator(&h->state);
        h->destroyer = seedvr2::adaptive_window_attention_layer_destroyer;
    } else if (strcmp(type, "SharedLinear") == 0) {
        h->layer = seedvr2::shared_linear_layer_creator(0);
        h->destroyer = seedvr2::shared_linear_layer_destroyer;
    } else if (strcmp(type, "SeedVR2ChunkedMHA") == 0) {
        h->layer = seedvr2::vae_chunked_mha_layer_creator(0);
        h->destroyer = seedvr2::vae_chunked_mha_layer_destroyer;
    } else if (strcmp(type, "ExportDownsample3D") == 0) {
        h->layer = seedvr2::vae_downsample3d_layer_creator(0);
        h->destroyer = seedvr2::vae_downsample3d_layer_destroyer;
    } else if (strcmp(type, "ExportUpsample3D") == 0) {
        h->layer = seedvr2::vae_upsample3d_layer_creator(0);
        h->destroyer = seedvr2::vae_upsample3d_layer_destroyer;
    } else if (strcmp(type, "DecomposedConv3d") == 0) {
        h->layer = seedvr2::decomposed_conv3d_layer_creator(0);
        h->destroyer = seedvr2::decomposed_conv3d_layer_destroyer;
    } else {
        delete h;
        return -1;
    }
    h->layer->type = type;
    ncnn::ParamDict pd;
    int ret = pd.load_param_text(params ? params : "");
    if (ret == 0) ret = h->layer->load_param(pd);
    if (ret == 0 && model) {
        ncnn::ModelBinFromMemory mb(static_cast<const unsigned char*>(model), (size_t)model_bytes);
        ret = h->layer->load_model(mb);
    }
    *out = h;
    return ret;
}

int h_layer_create_pipeline(void* handle) {
    Handle* h = static_cast<Handle*>(handle);
    return h->layer->create_pipeline(h->opt);
}

void h_layer_destroy(void* handle) {
    Handle* h = static_cast<Handle*>(handle);
    if (!h) return;
    h->layer->destroy_pipeline(h->opt);
    h->destroyer(h->layer, 0);
    delete h;
}

// AdaptiveWindowAttention::set_runtime_shapes through the creator's
// userdata (the reference's runtime_state, seedvr2_dit.cpp:724-725).
void h_awa_set_state(void* handle, const int* shapes, const int* text_lengths, int batch) {
    Handle* h = static_cast<Handle*>(handle);
    h->state.video_shapes.resize(batch);
    h->state.text_lengths.assign(text_lengths, text_lengths + batch);
    for (int b = 0; b < batch; b++)
        for (int a = 0; a < 3; a++) h->state.video_shapes[b][a] = shapes[3 * b + a];
}

int h_awa_configure_and_set_weights(void* handle, int heads, int head_dim, const int* target,
                                    int shifted, float eps, int pairs, int int32_shapes,
                                    int official_bf16, const float* vq, const float* vk,
                                    const float* tq, const float* tk, const float* freqs) {
    Handle* h = static_cast<Handle*>(handle);
    seedvr2::AdaptiveWindowAttention* l = dynamic_cast<seedvr2::AdaptiveWindowAttention*>(h->layer);
    if (!l) return -1;
    std::array<int, 3> t = {{target[0], target[1], target[2]}};
    l->configure(heads, head_dim, t, shifted != 0, eps, pairs, int32_shapes != 0, official_bf16 != 0);
    return l->set_weights(std::vector<float>(vq, vq + head_dim), std::vector<float>(vk, vk + head_dim),
                          std::vector<float>(tq, tq + head_dim), std::vector<float>(tk, tk + head_dim),
                          std::vector<float>(freqs, freqs + pairs));
}

// ncnn's 16-bit storage options of the Option passed to forward: they pick
// fp16 or bf16 for device blobs of elemsize 2.
void h_layer_set_storage(void* handle, int use_fp16_storage, int use_bf16_storage) {
    Handle* h = static_cast<Handle*>(handle);
    h->opt.use_fp16_storage = use_fp16_storage != 0;
    h->opt.use_bf16_storage = use_bf16_storage != 0;
}

// forward(vector<Mat>) with host or device input blobs.  Outputs are copied
// into the caller's buffers (host, or device when outs[i].device); their
// shapes are reported back in outs[i].
int h_layer_forward(void* handle, int n_in, const h_blob* ins, int n_out, h_blob* outs) {
    Handle* h = static_cast<Handle*>(handle);
    std::vector<ncnn::Mat> bottoms(n_in);
    for (int i = 0; i < n_in; i++) {
        const h_blob& b = ins[i];
        if (b.dims == 0) continue;
        ncnn::Allocator* alloc = b.device ? &device_allocator() : 0;
        if (b.dims == 1)
            bottoms[i] = ncnn::Mat(b.w, b.data, (size_t)b.elemsize, alloc);
        else
            bottoms[i] = ncnn::Mat(b.w, b.h, b.data, (size_t)b.elemsize, alloc);
    }
    std::vector<ncnn::Mat> tops(n_out);
    int ret = h->layer->forward(bottoms, tops, h->opt);
    if (ret != 0) return ret;
    for (int i = 0; i < n_out; i++) {
        h_blob& o = outs[i];
        const ncnn::Mat& m = tops[i];
        const size_t bytes = m.total() * m.elemsize;
        const size_t cap = (size_t)o.w * o.h * o.elemsize;
        o.dims = m.dims;
        const bool src_dev = seedvr2::device_allocator_of(m) != 0;
        if (bytes > cap) return -3;
        o.w = m.w;
        o.h = m.h;
        o.elemsize = (int)m.elemsize;
        if (bytes == 0) continue;
        if (src_dev && o.device) ret = s2_memcpy_d2d(o.data, m.data, bytes, 0);
        else if (src_dev) ret = s2_memcpy_d2h(o.data, m.data, bytes, 0);
        else if (o.device) ret = s2_memcpy_h2d(o.data, m.data, bytes, 0);
        else memcpy(o.data, m.data, bytes);
        if (ret != 0) return ret;
    }
    ret = s2_stream_synchronize(0);
    device_allocator().clear();
    return ret;
}

// A 4-D blob (w, h, d, c) with ncnn's channel stride cstep.
typedef struct h_blob4 {
    int w, h, d, c;
    long cstep;
    int elemsize;
    int device;
    void* data;
} h_blob4;

// seedvr2::set_vae_memory_state on the calling thread: 0 DISABLED,
// 1 INITIALIZING, 2 ACTIVE.
void h_set_vae_memory_state(int state) {
    seedvr2::set_vae_memory_state(static_cast<seedvr2::MemoryState>(state));
}

// DecomposedConv3D::reset_temporal_memory / release_completed_temporal_memory
int h_conv_memory(void* handle, int reset) {
    Handle* h = static_cast<Handle*>(handle);
    seedvr2::DecomposedConv3D* l = dynamic_cast<seedvr2::DecomposedConv3D*>(h->layer);
    if (!l) return -1;
    if (reset) l->reset_temporal_memory();
    else l->release_completed_temporal_memory();
    return 0;
}

// forward(Mat, Mat) of a one-blob layer over 4-D blobs.  The output is
// copied into out->data (host, or device when out->device), whose capacity
// is out->cstep * out->c elements; its shape is reported back in *out.
int h_layer_forward4(void* handle, const h_blob4* in, h_blob4* out) {
    Handle* h = static_cast<Handle*>(handle);
    ncnn::Allocator* alloc = in->device ? &device_allocator() : 0;
    ncnn::Mat bottom(in->w, in->h, in->d, in->c, in->data, (size_t)in->elemsize, alloc);
    if ((long)bottom.cstep != in->cstep) return -4;
    ncnn::Mat top;
    int ret = h->layer->forward(bottom, top, h->opt);
    if (ret != 0) return ret;
    const size_t bytes = top.total() * top.elemsize;
    if (bytes > (size_t)out->cstep * out->c * out->elemsize) return -3;
    const bool src_dev = seedvr2::device_allocator_of(top) != 0;
    if (src_dev && out->device) ret = s2_memcpy_d2d(out->data, top.data, bytes, 0);
    else if (src_dev) ret = s2_memcpy_d2h(out->data, top.data, bytes, 0);
    else if (out->device) ret = s2_memcpy_h2d(out->data, top.data, bytes, 0);
    else memcpy(out->data, top.data, bytes);
    out->w = top.w;
    out->h = top.h;
    out->d = top.d;
    out->c = top.c;
    out->cstep = (long)top.cstep;
    out->elemsize = (int)top.elemsize;
    if (ret == 0) ret = s2_stream_synchronize(0);
    device_allocator().clear();
    return ret;
}

// forward(Mat, Mat) of a one-blob layer over 2-D blobs; the output is copied
// into out->data (capacity out->w * out->h elements) and its shape reported.
int h_layer_forward1(void* handle, const h_blob* in, h_blob* out) {
    Handle* h = static_cast<Handle*>(handle);
    ncnn::Allocator* alloc = in->device ? &device_allocator() : 0;
    ncnn::Mat bottom(in->w, in->h, in->data, (size_t)in->elemsize, alloc);
    ncnn::Mat top;
    int ret = h->layer->forward(bottom, top, h->opt);
    if (ret != 0) return ret;
    const size_t bytes = top.total() * top.elemsize;
    if (bytes > (size_t)out->w * out->h * out->elemsize) return -3;
    const bool src_dev = seedvr2::device_allocator_of(top) != 0;
    if (src_dev && out->device) ret = s2_memcpy_d2d(out->data, top.data, bytes, 0);
    else if (src_dev) ret = s2_memcpy_d2h(out->data, top.data, bytes, 0);
    else if (out->device) ret = s2_memcpy_h2d(out->data, top.data, bytes, 0);
    else memcpy(out->data, top.data, bytes);
    out->dims = top.dims;
    out->w = top.w;
    out->h = top.h;
    out->elemsize = (int)top.elemsize;
    if (ret == 0) ret = s2_stream_synchronize(0);
    device_allocator().clear();
    return ret;
}

// seedvr2::build_adaptive_window_plan (layer-level API) into flat arrays.
int h_build_plan(const int* shapes, int batch, const int* target, int shifted, int max_windows,
                 int* num_windows, int* windows, int* counts, int* indices, int* inverse,
                 int* positions) {
    std::vector<std::array<int, 3> > vs(batch);
    for (int b = 0; b < batch; b++)
        for (int a = 0; a < 3; a++) vs[b][a] = shapes[3 * b + a];
    std::array<int, 3> t = {{target[0], target[1], target[2]}};
    seedvr2::AdaptiveWindowPlan plan;
    const int ret = seedvr2::build_adaptive_window_plan(vs, t, shifted != 0, plan);
    if (ret != 0) return ret;
    *num_windows = (int)plan.windows.size();
    if ((int)plan.windows.size() > max_windows) return -3;
    for (size_t i = 0; i < plan.windows.size(); i++) {
        const seedvr2::WindowSlice& s = plan.windows[i];
        const int f[9] = {s.sample_index, s.t0, s.t1, s.h0, s.h1, s.w0, s.w1,
                          s.partition_offset, s.token_count};
        memcpy(windows + 9 * i, f, sizeof(f));
    }
    for (int b = 0; b < batch; b++) counts[b] = plan.sample_window_count[b];
    for (size_t p = 0; p < plan.video_indices.size(); p++) {
        indices[p] = plan.video_indices[p];
        inverse[p] = plan.inverse_video_indices[p];
        for (int a = 0; a < 3; a++) positions[3 * p + a] = plan.local_positions[p][a];
    }
    return 0;
}

// ---- DiT block graph (seedvr2::DiTBlockGraph over ncnn::Net) -------------------

// Loads a block graph from .param text and .bin bytes; fuse: bit 0 folds
// SharedLinear -> GELU, bit 1 folds the QKV SharedLinear into the attention,
// bit 2 folds built-in norm / modulation / residual chains.  Returns load's
// code; *out is the graph (destroy with h_graph_destroy) or null.
int h_graph_create(const char* param_text, const void* model, long model_bytes, int fp32_blobs,
                   int fuse, void** out) {
    *out = 0;
    seedvr2::DiTBlockGraph* g = new seedvr2::DiTBlockGraph(0);
    const int ret = g->load_mem(param_text, static_cast<const unsigned char*>(model),
                                (size_t)model_bytes, fp32_blobs != 0, (fuse & 1) != 0,
                                (fuse & 2) != 0, (fuse & 4) != 0);
    if (ret != 0) {
        delete g;
        return ret;
    }
    *out = g;
    return 0;
}

int h_graph_fused_gelu(void* graph) {
    return static_cast<seedvr2::DiTBlockGraph*>(graph)->fused_gelu_count();
}

int h_graph_folded_modulation(void* graph) {
    return static_cast<seedvr2::DiTBlockGraph*>(graph)->folded_modulation_count();
}

int h_graph_fused_swiglu(void* graph) {
    return static_cast<seedvr2::DiTBlockGraph*>(graph)->fused_swiglu_count();
}

int h_graph_fused_qkv(void* graph) {
    return static_cast<seedvr2::DiTBlockGraph*>(graph)->fused_qkv_count();
}

// Layer count and device bytes the graph's allocator holds (blocks in use
// plus pooled ones).
int h_graph_layer_count(void* graph) {
    return (int)static_cast<seedvr2::DiTBlockGraph*>(graph)->net.layers().size();
}

// One run: inputs[0..9] = in0..in9 (host or device blobs, dims 1 or 2);
// out0/out1 and the named checkpoint blobs are copied into the caller's
// buffers (device when .device), their shapes reported back.
static int graph_run(void* graph, const int* shapes, const int* text_lengths, int batch,
                     const h_blob* inputs, h_blob* outs, int n_checkpoints,
                     const char* const* checkpoint_names, seedvr2::HipDeviceAllocator* wrap);

int h_graph_run(void* graph, const int* shapes, const int* text_lengths, int batch,
                const h_blob* inputs, h_blob* outs, int n_checkpoints,
                const char* const* checkpoint_names) {
    return graph_run(graph, shapes, text_lengths, batch, inputs, outs, n_checkpoints,
                     checkpoint_names, 0);
}

// h_graph_run with the device inputs tagged as blobs of an allocator on
// `input_stream` (a hipStream_t), as a caller whose producer kernels ran
// there hands them over: the graph must order its stream behind that one.
int h_graph_run_from_stream(void* graph, const int* shapes, const int* text_lengths, int batch,
                            const h_blob* inputs, h_blob* outs, void* input_stream) {
    seedvr2::HipDeviceAllocator producer(input_stream);
    return graph_run(graph, shapes, text_lengths, batch, inputs, outs, 0, 0, &producer);
}

static int graph_run(void* graph, const int* shapes, const int* text_lengths, int batch,
                     const h_blob* inputs, h_blob* outs, int n_checkpoints,
                     const char* const* checkpoint_names, seedvr2::HipDeviceAllocator* wrap) {
    seedvr2::DiTBlockGraph* g = static_cast<seedvr2::DiTBlockGraph*>(graph);
    seedvr2::HipDeviceAllocator& tag = wrap ? *wrap : g->allocator();
    std::vector<std::array<int, 3> > vs(batch);
    for (int b = 0; b < batch; b++)
        for (int a = 0; a < 3; a++) vs[b][a] = shapes[3 * b + a];
    std::vector<int> tl(text_lengths, text_lengths + batch);
    ncnn::Mat ins[10];
    for (int i = 0; i < 10; i++) {
        const h_blob& b = inputs[i];
        if (b.dims == 0) continue;
        if (b.device) {
            ins[i] = b.dims == 1 ? tag.wrap_blob(b.w, 1, b.data, (size_t)b.elemsize)
                                 : tag.wrap_blob(b.w, b.h, b.data, (size_t)b.elemsize);
            if (b.dims == 1) {
                ins[i].dims = 1;
                ins[i].h = 1;
            }
        } else {
            ins[i] = b.dims == 1 ? ncnn::Mat(b.w, b.data, (size_t)b.elemsize)
                                 : ncnn::Mat(b.w, b.h, b.data, (size_t)b.elemsize);
        }
    }
    std::vector<std::string> names;
    for (int i = 0; i < n_checkpoints; i++) names.push_back(checkpoint_names[i]);
    std::vector<ncnn::Mat> cps;
    std::vector<ncnn::Mat> tops(2);
    int ret = g->run(vs, tl, ins, tops[0], tops[1], n_checkpoints ? &names : 0, &cps);
    if (ret != 0) return ret;
    for (size_t i = 0; i < cps.size(); i++) tops.push_back(cps[i]);
    for (size_t i = 0; i < tops.size(); i++) {
        h_blob& o = outs[i];
        const ncnn::Mat& m = tops[i];
        const size_t bytes = (size_t)m.w * m.h * m.elemsize;
        if (bytes > (size_t)o.w * o.h * o.elemsize) return -3;
        o.dims = m.dims;
        o.w = m.w;
        o.h = m.h;
        o.elemsize = (int)m.elemsize;
        ret = o.device ? s2_memcpy_d2d(o.data, m.data, bytes, 0) : s2_memcpy_d2h(o.data, m.data, bytes, 0);
        if (ret != 0) return ret;
    }
    return s2_stream_synchronize(0);
}

void h_graph_destroy(void* graph) { delete static_cast<seedvr2::DiTBlockGraph*>(graph); }

// Blocks the graph's device allocator holds, in use or pooled.
long h_graph_owned_blocks(void* graph) {
    return (long)static_cast<seedvr2::DiTBlockGraph*>(graph)->allocator().owned_count();
}

// Runs a graph of built-in layers through ncnn::Net: load_param_mem /
// load_model, then one extractor fed n_in named blobs and asked for n_out
// named blobs.  device != 0: the extractor's blob allocator is a device
// allocator (host inputs are uploaded, device inputs used in place) and
// outputs are copied back into the caller's buffers (host or device per
// h_blob.device); otherwise everything runs on the host.  Returns the first
// failing code.
int h_net_run(const char* param_text, const void* model, long model_bytes, int device, int n_in,
              const char* const* in_names, const h_blob* ins, int n_out,
              const char* const* out_names, h_blob* outs) {
    ncnn::Net net;
    net.opt.use_bf16_storage = false;
    net.opt.use_fp16_storage = false;
    int ret = net.load_param_mem(param_text);
    if (ret == 0) ret = net.load_model(static_cast<const unsigned char*>(model), (size_t)model_bytes);
    if (ret != 0) return ret;
    seedvr2::HipDeviceAllocator alloc(0);
    ncnn::Extractor ex = net.create_extractor();
    if (device) ex.set_blob_allocator(&alloc);
    for (int i = 0; ret == 0 && i < n_in; i++) {
        const h_blob& b = ins[i];
        ncnn::Mat m;
        if (b.device)
            m = b.dims == 1 ? alloc.wrap_blob(b.w, 1, b.data, (size_t)b.elemsize)
                            : alloc.wrap_blob(b.w, b.h, b.data, (size_t)b.elemsize);
        else
            m = b.dims == 1 ? ncnn::Mat(b.w, b.data, (size_t)b.elemsize)
                            : ncnn::Mat(b.w, b.h, b.data, (size_t)b.elemsize);
        if (b.dims == 1) {
            m.dims = 1;
            m.h = 1;
        }
        ret = ex.input(in_names[i], m);
    }
    for (int i = 0; ret == 0 && i < n_out; i++) {
        ncnn::Mat m;
        ret = ex.extract(out_names[i], m);
        if (ret != 0) break;
        h_blob& o = outs[i];
        const size_t bytes = (size_t)m.w * (m.dims == 2 ? m.h : 1) * m.elemsize;
        if (bytes > (size_t)o.w * o.h * o.elemsize) return -3;
        const bool on_device = seedvr2::device_allocator_of(m) != 0;
        if (on_device)
            ret = o.device ? s2_memcpy_d2d(o.data, m.data, bytes, 0) : s2_memcpy_d2h(o.data, m.data, bytes, 0);
        else if (o.device)
            ret = s2_memcpy_h2d(o.data, m.data, bytes, 0);
        else
            memcpy(o.data, m.data, bytes);
        o.dims = m.dims;
        o.w = m.w;
        o.h = m.dims == 2 ? m.h : 1;
        o.elemsize = (int)m.elemsize;
    }
    if (ret == 0 && device) ret = s2_stream_synchronize(0);
    return ret;
}

// An ncnn::Net with SharedLinear registered: load_param_mem, then load_model
// on the same net whatever load_param returned.  Returns the layer count
// left in the net; *param_ret / *model_ret receive the two codes.
int h_net_load(const char* param_text, const void* model, long model_bytes, int* param_ret,
               int* model_ret) {
    ncnn::Net net;
    net.register_custom_layer("SharedLinear", seedvr2::shared_linear_layer_creator,
                              seedvr2::shared_linear_layer_destroyer);
    *param_ret = net.load_param_mem(param_text);
    *model_ret = net.load_model(static_cast<const unsigned char*>(model), (size_t)model_bytes);
    return (int)net.layers().size();
}

}  // extern "C"
