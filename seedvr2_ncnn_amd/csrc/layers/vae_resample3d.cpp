// VAEDownsample3D and VAEUpsample3D on MI355X (src/seedvr2/vae_downsample3d.cpp:77-173,
// vae_upsample3d.cpp:166-321) over DecomposedConv3D and the HIP C-ABI.
#include "vae_resample3d.h"

#include <modelbin.h>

#include "seedvr2_hip.h"

namespace seedvr2 {

namespace {

size_t align16(size_t bytes) { return (bytes + 15) & ~size_t(15); }

// ncnn's channel stride of a [c][d][h][w] Mat of elemsize bytes
long ncnn_cstep(int d, int h, int w, size_t elemsize)
{
    return (long)(align16((size_t)d * h * w * elemsize) / elemsize);
}

bool blob_ok(const ncnn::Mat& m, int channels, size_t* elemsize, HipDeviceAllocator** device)
{
    if (m.dims != 4 || m.c != channels || m.elempack != 1)
        return false;
    *device = device_allocator_of(m);
    *elemsize = m.elemsize;
    return *device ? (m.elemsize == 4 || m.elemsize == 2) : m.elemsize == sizeof(float);
}

} // namespace

// ---- VAEDownsample3D -----------------------------------------------------------

VAEDownsample3D::VAEDownsample3D() : channels(0), pad_right(0), pad_bottom(0), loaded(false)
{
    one_blob_only = true;
    support_inplace = false;
}

VAEDownsample3D::~VAEDownsample3D()
{
}

// vae_downsample3d.cpp:98-112: a raw fp32 config blob {channels, pad_right,
// pad_bottom}, then the DecomposedConv3D's blobs.
int VAEDownsample3D::load_model(const ncnn::ModelBin& mb)
{
    std::lock_guard<std::mutex> lock(mutex);
    loaded = false;
    const ncnn::Mat config = mb.load(3, 1);
    if (config.empty())
        return -100;
    const float* v = config;
    channels = static_cast<int>(v[0]);
    pad_right = static_cast<int>(v[1]);
    pad_bottom = static_cast<int>(v[2]);
    if (channels <= 0 || pad_right < 0 || pad_bottom < 0 || (pad_right == 0 && pad_bottom == 0))
        return -1;
    const int ret = convolution.load_model(mb);
    loaded = ret == 0;
    return ret;
}

int VAEDownsample3D::create_pipeline(const ncnn::Option& opt)
{
    return loaded ? convolution.create_pipeline(opt) : -1;
}

int VAEDownsample3D::destroy_pipeline(const ncnn::Option& opt)
{
    std::lock_guard<std::mutex> lock(mutex);
    staging.release();
    return convolution.destroy_pipeline(opt);
}

void VAEDownsample3D::release_completed_temporal_memory() const
{
    convolution.release_completed_temporal_memory();
}

void VAEDownsample3D::reset_temporal_memory() const
{
    convolution.reset_temporal_memory();
}

// vae_downsample3d.cpp:145-172
int VAEDownsample3D::forward(const ncnn::Mat& bottom_blob, ncnn::Mat& top_blob,
                             const ncnn::Option& opt) const
{
    return layer_status(forward_impl(bottom_blob, top_blob, opt));
}

int VAEDownsample3D::forward_impl(const ncnn::Mat& bottom_blob, ncnn::Mat& top_blob,
                             const ncnn::Option& opt) const
{
    std::lock_guard<std::mutex> lock(mutex);
    size_t elemsize = 0;
    HipDeviceAllocator* device = 0;
    if (!loaded || !blob_ok(bottom_blob, channels, &elemsize, &device) ||
        convolution.num_input() != channels)
        return -1;
    int out[3];
    if (convolution.output_shape(bottom_blob.d, bottom_blob.h, bottom_blob.w, elemsize, pad_right,
                                 pad_bottom, out) != 0)
        return -1;
    const int cout = convolution.num_output();
    if (device)
    {
        HipDeviceAllocator* out_alloc = dynamic_cast<HipDeviceAllocator*>(opt.blob_allocator);
        if (!out_alloc)
            out_alloc = device;
        top_blob = out_alloc->create_blob(out[2], out[1], out[0], cout, elemsize);
        if (top_blob.empty())
            return -100;
        return convolution.forward_device(bottom_blob.data, device_blob_dtype(elemsize, opt),
                                          elemsize, bottom_blob.d, bottom_blob.h, bottom_blob.w,
                                          (long)bottom_blob.cstep, pad_right, pad_bottom,
                                          top_blob.data, (long)top_blob.cstep, device->stream());
    }
    const size_t in_bytes = bottom_blob.cstep * bottom_blob.c * sizeof(float);
    const long out_cstep = ncnn_cstep(out[0], out[1], out[2], 4);
    const size_t out_bytes = (size_t)out_cstep * cout * sizeof(float);
    int ret = staging.reserve(align16(in_bytes) + out_bytes);
    if (ret != 0)
        return ret;
    unsigned char* x = static_cast<unsigned char*>(staging.get());
    unsigned char* y = x + align16(in_bytes);
    ret = s2_memcpy_h2d(x, bottom_blob.data, in_bytes, 0);
    if (ret == 0)
        ret = convolution.forward_device(x, S2_DTYPE_F32, 4, bottom_blob.d, bottom_blob.h,
                                         bottom_blob.w, (long)bottom_blob.cstep, pad_right,
                                         pad_bottom, y, out_cstep, 0);
    if (ret != 0)
        return ret;
    top_blob.create(out[2], out[1], out[0], cout, 4u, opt.blob_allocator);
    if (top_blob.empty())
        return -100;
    ret = s2_memcpy_d2h(top_blob.data, y, out_bytes, 0);
    if (ret == 0)
        ret = s2_stream_synchronize(0);
    return ret;
}

// ---- VAEUpsample3D -------------------------------------------------------------

VAEUpsample3D::VAEUpsample3D()
    : channels(0), temporal_ratio(0), spatial_ratio(0), remove_temporal_head(false), loaded(false)
{
    one_blob_only = true;
    support_inplace = false;
}

VAEUpsample3D::~VAEUpsample3D()
{
}

// vae_upsample3d.cpp:191-213: a raw fp32 config blob {channels,
// temporal_ratio, spatial_ratio, remove_temporal_head}, then the post and
// the upscale DecomposedConv3D (the exporter writes attributes in lexical
// order).
int VAEUpsample3D::load_model(const ncnn::ModelBin& mb)
{
    std::lock_guard<std::mutex> lock(mutex);
    loaded = false;
    const ncnn::Mat config = mb.load(4, 1);
    if (config.empty())
        return -100;
    const float* v = config;
    channels = static_cast<int>(v[0]);
    temporal_ratio = static_cast<int>(v[1]);
    spatial_ratio = static_cast<int>(v[2]);
    remove_temporal_head = static_cast<int>(v[3]) != 0;
    if (channels <= 0 || (temporal_ratio != 1 && temporal_ratio != 2) ||
        (spatial_ratio != 1 && spatial_ratio != 2) ||
        remove_temporal_head != (temporal_ratio == 2))
        return -1;
    int ret = post_conv.load_model(mb);
    if (ret == 0)
        ret = upscale_conv.load_model(mb);
    loaded = ret == 0;
    return ret;
}

int VAEUpsample3D::create_pipeline(const ncnn::Option& opt)
{
    if (!loaded)
        return -1;
    int ret = post_conv.create_pipeline(opt);
    if (ret == 0)
        ret = upscale_conv.create_pipeline(opt);
    return ret;
}

int VAEUpsample3D::destroy_pipeline(const ncnn::Option& opt)
{
    std::lock_guard<std::mutex> lock(mutex);
    packed.release();
    shuffled.release();
    staging.release();
    post_conv.destroy_pipeline(opt);
    upscale_conv.destroy_pipeline(opt);
    return 0;
}

void VAEUpsample3D::release_completed_temporal_memory() const
{
    post_conv.release_completed_temporal_memory();
    upscale_conv.release_completed_temporal_memory();
}

void VAEUpsample3D::reset_temporal_memory() const
{
    post_conv.reset_temporal_memory();
    upscale_conv.reset_temporal_memory();
}

// The extents of the three stages under the current memory state
// (vae_upsample3d.cpp:258-285).
int VAEUpsample3D::output_shape(int frames, int h, int w, size_t elemsize, int out[3],
                                int packed_shape[3], int shuffled_shape[3],
                                bool* remove_head) const
{
    const int ratio = temporal_ratio * spatial_ratio * spatial_ratio;
    if (upscale_conv.num_input() != channels || upscale_conv.num_output() != channels * ratio ||
        post_conv.num_input() != channels)
        return -1;
    if (upscale_conv.output_shape(frames, h, w, elemsize, 0, 0, packed_shape) != 0)
        return -1;
    *remove_head = remove_temporal_head && get_vae_memory_state() != MemoryState::ACTIVE;
    shuffled_shape[0] = packed_shape[0] * temporal_ratio - (*remove_head ? 1 : 0);
    shuffled_shape[1] = packed_shape[1] * spatial_ratio;
    shuffled_shape[2] = packed_shape[2] * spatial_ratio;
    if (shuffled_shape[0] <= 0)
        return -1;
    return post_conv.output_shape(shuffled_shape[0], shuffled_shape[1], shuffled_shape[2],
                                  elemsize, 0, 0, out);
}

// upscale convolution -> shuffle -> post convolution on device memory
int VAEUpsample3D::run(const void* input, s2_dtype dtype, size_t elemsize, int frames, int h,
                       int w, long in_cstep, void* output, long out_cstep, void* stream) const
{
    int out[3], ps[3], ss[3];
    bool remove_head = false;
    if (output_shape(frames, h, w, elemsize, out, ps, ss, &remove_head) != 0)
        return -1;
    const int ratio = temporal_ratio * spatial_ratio * spatial_ratio;
    const long packed_cstep = ncnn_cstep(ps[0], ps[1], ps[2], elemsize);
    const long shuffled_cstep = ncnn_cstep(ss[0], ss[1], ss[2], elemsize);
    int ret = packed.reserve((size_t)packed_cstep * channels * ratio * elemsize);
    if (ret == 0)
        ret = shuffled.reserve((size_t)shuffled_cstep * channels * elemsize);
    if (ret != 0)
        return ret;
    ret = upscale_conv.forward_device(input, dtype, elemsize, frames, h, w, in_cstep, 0, 0,
                                      packed.get(), packed_cstep, stream);
    if (ret == 0)
        ret = s2_vae_pixel_shuffle(packed.get(), dtype, channels, ps[0], ps[1], ps[2],
                                   packed_cstep, temporal_ratio, spatial_ratio,
                                   remove_head ? 1 : 0, shuffled.get(), shuffled_cstep, stream);
    if (ret == 0)
        ret = post_conv.forward_device(shuffled.get(), dtype, elemsize, ss[0], ss[1], ss[2],
                                       shuffled_cstep, 0, 0, output, out_cstep, stream);
    return ret;
}

// vae_upsample3d.cpp:258-321
int VAEUpsample3D::forward(const ncnn::Mat& bottom_blob, ncnn::Mat& top_blob,
                           const ncnn::Option& opt) const
{
    return layer_status(forward_impl(bottom_blob, top_blob, opt));
}

int VAEUpsample3D::forward_impl(const ncnn::Mat& bottom_blob, ncnn::Mat& top_blob,
                           const ncnn::Option& opt) const
{
    std::lock_guard<std::mutex> lock(mutex);
    size_t elemsize = 0;
    HipDeviceAllocator* device = 0;
    if (!loaded || !blob_ok(bottom_blob, channels, &elemsize, &device))
        return -1;
    int out[3], ps[3], ss[3];
    bool remove_head = false;
    if (output_shape(bottom_blob.d, bottom_blob.h, bottom_blob.w, elemsize, out, ps, ss,
                     &remove_head) != 0)
        return -1;
    const int cout = post_conv.num_output();
    if (device)
    {
        HipDeviceAllocator* out_alloc = dynamic_cast<HipDeviceAllocator*>(opt.blob_allocator);
        if (!out_alloc)
            out_alloc = device;
        top_blob = out_alloc->create_blob(out[2], out[1], out[0], cout, elemsize);
        if (top_blob.empty())
            return -100;
        return run(bottom_blob.data, device_blob_dtype(elemsize, opt), elemsize, bottom_blob.d,
                   bottom_blob.h, bottom_blob.w, (long)bottom_blob.cstep, top_blob.data,
                   (long)top_blob.cstep, device->stream());
    }
    const size_t in_bytes = bottom_blob.cstep * bottom_blob.c * sizeof(float);
    const long out_cstep = ncnn_cstep(out[0], out[1], out[2], 4);
    const size_t out_bytes = (size_t)out_cstep * cout * sizeof(float);
    int ret = staging.reserve(align16(in_bytes) + out_bytes);
    if (ret != 0)
        return ret;
    unsigned char* x = static_cast<unsigned char*>(staging.get());
    unsigned char* y = x + align16(in_bytes);
    ret = s2_memcpy_h2d(x, bottom_blob.data, in_bytes, 0);
    if (ret == 0)
        ret = run(x, S2_DTYPE_F32, 4, bottom_blob.d, bottom_blob.h, bottom_blob.w,
                  (long)bottom_blob.cstep, y, out_cstep, 0);
    if (ret != 0)
        return ret;
    top_blob.create(out[2], out[1], out[0], cout, 4u, opt.blob_allocator);
    if (top_blob.empty())
        return -100;
    ret = s2_memcpy_d2h(top_blob.data, y, out_bytes, 0);
    if (ret == 0)
        ret = s2_stream_synchronize(0);
    return ret;
}

ncnn::Layer* vae_downsample3d_layer_creator(void* /*userdata*/)
{
    return new VAEDownsample3D;
}

void vae_downsample3d_layer_destroyer(ncnn::Layer* layer, void* /*userdata*/)
{
    delete layer;
}

ncnn::Layer* vae_upsample3d_layer_creator(void* /*userdata*/)
{
    return new VAEUpsample3D;
}

void vae_upsample3d_layer_destroyer(ncnn::Layer* layer, void* /*userdata*/)
{
    delete layer;
}

} // namespace seedvr2
