// DecomposedConv3D: the causal 3-D convolution of the SeedVR2 VAE as an ncnn
// custom layer whose forward runs on an MI355X through the HIP C-ABI
// (include/seedvr2_hip.h).
//
// Drop-in surface of the reference layer (src/seedvr2/decomposed_conv3d.h:29-88):
// ParamDict ids 0-15; load_model reads the 16-value config blob (which
// overrides the ParamDict values, as in the reference), the bias when
// bias_term and one ncnn Convolution weight per temporal tap; forward takes a
// 4-D blob [num_input][frames][h][w] and gives [num_output][out frames][out h]
// [out w].  The temporal memory follows the thread's VAE memory state
// (get/set_vae_memory_state): DISABLED keeps none, INITIALIZING starts one,
// ACTIVE continues the previous slice.  The kernel runs the whole
// kt x kh x kw window as one implicit GEMM in bf16 with fp32 accumulation
// instead of one ncnn Convolution per tap; groups must be 1 and the spatial
// window at most 32 positions.
#ifndef SEEDVR2_DECOMPOSED_CONV3D_H
#define SEEDVR2_DECOMPOSED_CONV3D_H

#include <mutex>

#include <layer.h>

#include "hip_allocator.h"

namespace seedvr2 {

// decomposed_conv3d.h:15-23
enum class MemoryState
{
    DISABLED,
    INITIALIZING,
    ACTIVE
};

MemoryState get_vae_memory_state();
void set_vae_memory_state(MemoryState state);

class DecomposedConv3D : public ncnn::Layer
{
public:
    DecomposedConv3D();
    virtual ~DecomposedConv3D();

    virtual int load_param(const ncnn::ParamDict& pd);
    virtual int load_model(const ncnn::ModelBin& mb);
    virtual int create_pipeline(const ncnn::Option& opt);
    virtual int destroy_pipeline(const ncnn::Option& opt);
    // Host fp32 blobs give host fp32 outputs; device blobs (HipDeviceAllocator,
    // fp32 or 16-bit) give device outputs of the same element size.
    virtual int forward(const ncnn::Mat& bottom_blob, ncnn::Mat& top_blob,
                        const ncnn::Option& opt) const;

    void release_completed_temporal_memory() const;
    void reset_temporal_memory() const;

    // For layers built on this one (VAEDownsample3D, VAEUpsample3D): the
    // output extent {frames, h, w} of a forward under the current memory
    // state, over input frames padded with pad_right zero columns and
    // pad_bottom zero rows (-1 where forward would refuse the input) ...
    int output_shape(int frames, int h, int w, size_t elemsize, int pad_right, int pad_bottom,
                     int out[3]) const;
    // ... and forward on device memory: planar input [num_input][in_cstep] and
    // output [num_output][out_cstep] of element type dtype, on `stream`.
    int forward_device(const void* input, s2_dtype dtype, size_t elemsize, int frames, int h,
                       int w, long in_cstep, int pad_right, int pad_bottom, void* output,
                       long out_cstep, void* stream) const;

    int num_input() const { return config.num_input; }
    int num_output() const { return config.num_output; }

private:
    // forward and create_pipeline without the mapping of C-ABI codes to the
    // reference's (layer_status)
    int forward_impl(const ncnn::Mat& bottom_blob, ncnn::Mat& top_blob,
                     const ncnn::Option& opt) const;
    int create_pipeline_impl();
    int upload_weights_locked() const;
    bool config_ok() const;
    int output_shape_locked(int frames, int h, int w, size_t elemsize, int pad_right,
                            int pad_bottom, int out[3]) const;

    s2_conv3d_config config;
    ncnn::Mat bias_data;
    ncnn::Mat weight_data;   // [kernel_t][num_output][num_input][kernel_h][kernel_w]

    mutable std::mutex mutex;
    mutable bool weights_dirty;
    mutable DeviceBuffer packed_gpu;
    mutable DeviceBuffer bias_gpu;
    mutable DeviceBuffer workspace;
    mutable DeviceBuffer staging;
    // temporal memory: two buffers, the one the next forward reads and the
    // one it writes
    mutable DeviceBuffer memory[2];
    mutable int memory_current;   // index of the memory to read, -1: none
    mutable int memory_frames;
    mutable int memory_w, memory_h;
    mutable size_t memory_elemsize;
    StreamScratchRef host_scratch;   // the default stream's kernel scratch (split k ranges)
};

ncnn::Layer* decomposed_conv3d_layer_creator(void* userdata);
void decomposed_conv3d_layer_destroyer(ncnn::Layer* layer, void* userdata);

} // namespace seedvr2

#endif // SEEDVR2_DECOMPOSED_CONV3D_H
