// VAEChunkedMHA on MI355X: the ncnn layer surface of the reference
// (src/seedvr2/vae_chunked_mha.cpp:93-289) over the HIP C-ABI.
#include "vae_chunked_mha.h"

#include <math.h>
#include <string.h>

#include <modelbin.h>

#include "seedvr2_hip.h"

namespace seedvr2 {

VAEChunkedMHA::VAEChunkedMHA()
    : embed_dim(0), num_heads(0), weight_data_size(0), kdim(0), vdim(0), scale(0.f),
      chunk_size(128), weights_dirty(true)
{
    one_blob_only = true;
    support_inplace = false;
}

VAEChunkedMHA::~VAEChunkedMHA()
{
}

// ParamDict ids, defaults and checks of the reference load_param (:116-129).
int VAEChunkedMHA::load_param(const ncnn::ParamDict& pd)
{
    std::lock_guard<std::mutex> lock(mutex);
    embed_dim = pd.get(0, 0);
    num_heads = pd.get(1, 1);
    weight_data_size = pd.get(2, 0);
    kdim = pd.get(3, embed_dim);
    vdim = pd.get(4, embed_dim);
    scale = num_heads > 0 ? pd.get(6, 1.f / sqrtf(static_cast<float>(embed_dim / num_heads))) : 0.f;
    chunk_size = pd.get(20, 128);
    weights_dirty = true;
    if (embed_dim <= 0 || num_heads <= 0 || embed_dim % num_heads != 0 || weight_data_size <= 0 ||
        weight_data_size % embed_dim != 0 || kdim <= 0 || vdim <= 0 || chunk_size <= 0)
        return -1;
    return 0;
}

// The eight MultiHeadAttention blobs in the reference order (:131-152): q
// weight [embed][qdim] and bias, k weight [embed][kdim] and bias, v weight
// [embed][vdim] and bias, out weight [qdim][embed] and bias [qdim].
int VAEChunkedMHA::load_model(const ncnn::ModelBin& mb)
{
    std::lock_guard<std::mutex> lock(mutex);
    weights_dirty = true;
    if (embed_dim <= 0)
        return -1;
    const int qdim = weight_data_size / embed_dim;
    weights[0] = mb.load(embed_dim * qdim, 0);
    weights[1] = mb.load(embed_dim, 1);
    weights[2] = mb.load(embed_dim * kdim, 0);
    weights[3] = mb.load(embed_dim, 1);
    weights[4] = mb.load(embed_dim * vdim, 0);
    weights[5] = mb.load(embed_dim, 1);
    weights[6] = mb.load(qdim * embed_dim, 0);
    weights[7] = mb.load(qdim, 1);
    for (int i = 0; i < 8; i++)
        if (weights[i].empty())
            return -100;
    return 0;
}

int VAEChunkedMHA::create_pipeline(const ncnn::Option& /*opt*/)
{
    return layer_status(create_pipeline_impl());
}

int VAEChunkedMHA::create_pipeline_impl()
{
    std::lock_guard<std::mutex> lock(mutex);
    // the host-blob path runs on the default stream: own its scratch
    const int sret = host_scratch.take(0);
    if (sret != S2_OK)
        return sret;
    int devices = 0;
    const int qdim = embed_dim > 0 ? weight_data_size / embed_dim : 0;
    if (s2_device_count(&devices) != S2_OK || devices == 0 || weights[0].empty() ||
        kdim != qdim || vdim != qdim)
        return 0;
    return upload_weights_locked();
}

int VAEChunkedMHA::destroy_pipeline(const ncnn::Option& /*opt*/)
{
    std::lock_guard<std::mutex> lock(mutex);
    host_scratch.drop();
    prepared.release();
    workspace.release();
    staging.release();
    weights_dirty = true;
    return 0;
}

int VAEChunkedMHA::upload_weights_locked() const
{
    if (!weights_dirty && prepared.get())
        return 0;
    const int qdim = weight_data_size / embed_dim;
    const s2_mha_config cfg = {embed_dim, num_heads, qdim, scale};
    size_t bytes = 0;
    int ret = s2_mha_weight_bytes(&cfg, &bytes);
    if (ret != 0)
        return ret;
    size_t offs[9];
    offs[0] = 0;
    for (int i = 0; i < 8; i++)
        offs[i + 1] = offs[i] + ((weights[i].total() * sizeof(float) + 255) & ~size_t(255));
    DeviceBuffer tmp;
    ret = tmp.reserve(offs[8]);
    if (ret == 0)
        ret = prepared.reserve(bytes);
    unsigned char* base = static_cast<unsigned char*>(tmp.get());
    for (int i = 0; ret == 0 && i < 8; i++)
        ret = s2_memcpy_h2d(base + offs[i], weights[i].data, weights[i].total() * sizeof(float), 0);
    if (ret == 0)
    {
        const float* w[8];
        for (int i = 0; i < 8; i++)
            w[i] = reinterpret_cast<const float*>(base + offs[i]);
        ret = s2_mha_prepare_weights(&cfg, w[0], w[1], w[2], w[3], w[4], w[5], w[6], w[7],
                                     prepared.get(), 0);
    }
    if (ret == 0)
        ret = s2_stream_synchronize(0);
    if (ret == 0)
        weights_dirty = false;
    return ret;
}

// vae_chunked_mha.cpp:223-235
int VAEChunkedMHA::forward(const ncnn::Mat& bottom_blob, ncnn::Mat& top_blob,
                           const ncnn::Option& opt) const
{
    return layer_status(forward_impl(bottom_blob, top_blob, opt));
}

int VAEChunkedMHA::forward_impl(const ncnn::Mat& bottom_blob, ncnn::Mat& top_blob,
                           const ncnn::Option& opt) const
{
    std::lock_guard<std::mutex> lock(mutex);
    if (embed_dim <= 0 || weights[0].empty())
        return -1;
    const int qdim = weight_data_size / embed_dim;
    // the input is query, key and value at once: kdim and vdim must match it
    if (bottom_blob.dims != 2 || bottom_blob.w != qdim || bottom_blob.elempack != 1 ||
        kdim != qdim || vdim != qdim)
        return -1;
    HipDeviceAllocator* device = device_allocator_of(bottom_blob);
    const size_t elemsize = bottom_blob.elemsize;
    if (!device && elemsize != sizeof(float))
        return -1;
    if (device && elemsize != 4 && elemsize != 2)
        return -1;
    const int seq = bottom_blob.h;
    const s2_mha_config cfg = {embed_dim, num_heads, qdim, scale};
    size_t ws_bytes = 0;
    if (s2_mha_workspace_bytes(&cfg, seq, &ws_bytes) != S2_OK)
        return -1;
    int devices = 0;
    if (s2_device_count(&devices) != S2_OK || devices == 0)
        return S2_ERR_DEVICE;
    int ret = upload_weights_locked();
    if (ret == 0)
        ret = workspace.reserve(ws_bytes);
    if (ret != 0)
        return ret;

    if (device)
    {
        HipDeviceAllocator* out_alloc = dynamic_cast<HipDeviceAllocator*>(opt.blob_allocator);
        if (!out_alloc)
            out_alloc = device;
        top_blob = out_alloc->create_blob(qdim, seq, elemsize);
        if (top_blob.empty())
            return -100;
        const s2_dtype dtype = device_blob_dtype(elemsize, opt);
        return s2_mha_forward(&cfg, prepared.get(), bottom_blob.data, dtype, seq, top_blob.data,
                              dtype, workspace.get(), ws_bytes, device->stream());
    }

    // Host fp32 blobs: stage, compute, download, synchronise.
    const size_t bytes = (size_t)seq * qdim * sizeof(float);
    ret = staging.reserve(2 * bytes);
    if (ret != 0)
        return ret;
    unsigned char* x = static_cast<unsigned char*>(staging.get());
    unsigned char* y = x + bytes;
    ret = s2_memcpy_h2d(x, bottom_blob.data, bytes, 0);
    if (ret == 0)
        ret = s2_mha_forward(&cfg, prepared.get(), x, S2_DTYPE_F32, seq, y, S2_DTYPE_F32,
                             workspace.get(), ws_bytes, 0);
    if (ret != 0)
        return ret;
    top_blob.create(qdim, seq, 4u, opt.blob_allocator);
    if (top_blob.empty())
        return -100;
    ret = s2_memcpy_d2h(top_blob.data, y, bytes, 0);
    if (ret == 0)
        ret = s2_stream_synchronize(0);
    return ret;
}

ncnn::Layer* vae_chunked_mha_layer_creator(void* /*userdata*/)
{
    return new VAEChunkedMHA;
}

void vae_chunked_mha_layer_destroyer(ncnn::Layer* layer, void* /*userdata*/)
{
    delete layer;
}

} // namespace seedvr2
