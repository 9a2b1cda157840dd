// VAEDownsample3D and VAEUpsample3D: the VAE's resampling layers as ncnn
// custom layers on an MI355X, built on DecomposedConv3D.
//
// Drop-in surfaces of the reference layers (src/seedvr2/vae_downsample3d.h:13-44,
// vae_upsample3d.h:13-45), registered as ExportDownsample3D and
// ExportUpsample3D (seedvr2_vae.cpp:182-185).  Both take one 4-D blob
// [channels][frames][h][w] and follow the VAE memory state through their
// convolutions.
//
//   VAEDownsample3D: load_model reads a 3-value config blob (channels,
//   pad_right, pad_bottom) and a DecomposedConv3D; forward pads the frames
//   with zero columns on the right and zero rows at the bottom and runs the
//   convolution.  The padding is not materialised: the convolution kernel
//   already reads every pixel outside the frame as zero.
//
//   VAEUpsample3D: load_model reads a 4-value config blob (channels,
//   temporal_ratio, spatial_ratio, remove_temporal_head), then the post and
//   the upscale DecomposedConv3D in that order; forward runs the upscale
//   convolution to channels * ratio channels, a depth-to-space shuffle over
//   time and space (dropping shuffled time 1 outside the ACTIVE memory state
//   when remove_temporal_head), and the post convolution, all on the device.
#ifndef SEEDVR2_VAE_RESAMPLE3D_H
#define SEEDVR2_VAE_RESAMPLE3D_H

#include <mutex>

#include <layer.h>

#include "decomposed_conv3d.h"
#include "hip_allocator.h"

namespace seedvr2 {

class VAEDownsample3D : public ncnn::Layer
{
public:
    VAEDownsample3D();
    virtual ~VAEDownsample3D();

    virtual int load_model(const ncnn::ModelBin& mb);
    virtual int create_pipeline(const ncnn::Option& opt);
    virtual int destroy_pipeline(const ncnn::Option& opt);
    virtual int forward(const ncnn::Mat& bottom_blob, ncnn::Mat& top_blob,
                        const ncnn::Option& opt) const;

    void release_completed_temporal_memory() const;
    void reset_temporal_memory() const;

private:
    // forward without the mapping of C-ABI codes to the reference's
    int forward_impl(const ncnn::Mat& bottom_blob, ncnn::Mat& top_blob,
                     const ncnn::Option& opt) const;

    int channels;
    int pad_right;
    int pad_bottom;
    bool loaded;
    DecomposedConv3D convolution;
    mutable std::mutex mutex;
    mutable DeviceBuffer staging;
};

class VAEUpsample3D : public ncnn::Layer
{
public:
    VAEUpsample3D();
    virtual ~VAEUpsample3D();

    virtual int load_model(const ncnn::ModelBin& mb);
    virtual int create_pipeline(const ncnn::Option& opt);
    virtual int destroy_pipeline(const ncnn::Option& opt);
    virtual int forward(const ncnn::Mat& bottom_blob, ncnn::Mat& top_blob,
                        const ncnn::Option& opt) const;

    void release_completed_temporal_memory() const;
    void reset_temporal_memory() const;

private:
    // forward without the mapping of C-ABI codes to the reference's
    int forward_impl(const ncnn::Mat& bottom_blob, ncnn::Mat& top_blob,
                     const ncnn::Option& opt) const;
    int run(const void* input, s2_dtype dtype, size_t elemsize, int frames, int h, int w,
            long in_cstep, void* output, long out_cstep, void* stream) const;
    int output_shape(int frames, int h, int w, size_t elemsize, int out[3], int packed[3],
                     int shuffled[3], bool* remove_head) const;

    int channels;
    int temporal_ratio;
    int spatial_ratio;
    bool remove_temporal_head;
    bool loaded;
    DecomposedConv3D post_conv;
    DecomposedConv3D upscale_conv;
    mutable std::mutex mutex;
    mutable DeviceBuffer packed;
    mutable DeviceBuffer shuffled;
    mutable DeviceBuffer staging;
};

ncnn::Layer* vae_downsample3d_layer_creator(void* userdata);
void vae_downsample3d_layer_destroyer(ncnn::Layer* layer, void* userdata);
ncnn::Layer* vae_upsample3d_layer_creator(void* userdata);
void vae_upsample3d_layer_destroyer(ncnn::Layer* layer, void* userdata);

} // namespace seedvr2

#endif // SEEDVR2_VAE_RESAMPLE3D_H
