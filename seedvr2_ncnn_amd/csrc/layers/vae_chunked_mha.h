// VAEChunkedMHA: the VAE's self attention as an ncnn custom layer whose
// forward runs on an MI355X through the HIP C-ABI (include/seedvr2_hip.h).
//
// Drop-in surface of the reference layer (src/seedvr2/vae_chunked_mha.h:12-50):
// ParamDict ids 0 embed_dim, 1 num_heads (1), 2 weight_data_size, 3 kdim, 4
// vdim, 6 scale (1/sqrt(embed_dim / num_heads)), 20 chunk_size (128);
// load_model reads the eight ncnn MultiHeadAttention blobs (q, k, v weights
// and biases, out weight and bias); forward takes one blob [seq][qdim] and
// gives [seq][qdim].  The whole sequence is one forward on the device; the
// chunk size, which bounds the reference's Vulkan memory, is kept as a
// parameter and does not change the result.
#ifndef SEEDVR2_VAE_CHUNKED_MHA_H
#define SEEDVR2_VAE_CHUNKED_MHA_H

#include <mutex>

#include <layer.h>

#include "hip_allocator.h"

namespace seedvr2 {

class VAEChunkedMHA : public ncnn::Layer
{
public:
    VAEChunkedMHA();
    virtual ~VAEChunkedMHA();

    virtual int load_param(const ncnn::ParamDict& pd);
    virtual int load_model(const ncnn::ModelBin& mb);
    virtual int create_pipeline(const ncnn::Option& opt);
    virtual int destroy_pipeline(const ncnn::Option& opt);
    // Host fp32 blobs give host fp32 outputs; device blobs (HipDeviceAllocator,
    // fp32 or 16-bit) give device outputs of the same element size.
    virtual int forward(const ncnn::Mat& bottom_blob, ncnn::Mat& top_blob,
                        const ncnn::Option& opt) const;

private:
    // forward and create_pipeline without the mapping of C-ABI codes to the
    // reference's (layer_status)
    int forward_impl(const ncnn::Mat& bottom_blob, ncnn::Mat& top_blob,
                     const ncnn::Option& opt) const;
    int create_pipeline_impl();
    int upload_weights_locked() const;

    int embed_dim;
    int num_heads;
    int weight_data_size;
    int kdim;
    int vdim;
    float scale;
    int chunk_size;
    ncnn::Mat weights[8];

    mutable std::mutex mutex;
    StreamScratchRef host_scratch;   // the default stream's kernel scratch
    mutable bool weights_dirty;
    mutable DeviceBuffer prepared;
    mutable DeviceBuffer workspace;
    mutable DeviceBuffer staging;
};

ncnn::Layer* vae_chunked_mha_layer_creator(void* userdata);
void vae_chunked_mha_layer_destroyer(ncnn::Layer* layer, void* userdata);

} // namespace seedvr2

#endif // SEEDVR2_VAE_CHUNKED_MHA_H
