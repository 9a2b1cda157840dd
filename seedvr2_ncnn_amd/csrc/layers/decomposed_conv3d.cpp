// DecomposedConv3D on MI355X: the ncnn layer surface of the reference
// (src/seedvr2/decomposed_conv3d.cpp:374-755) over the HIP C-ABI.
#include "decomposed_conv3d.h"

#include <string.h>

#include <modelbin.h>

#include "seedvr2_hip.h"

namespace seedvr2 {

namespace {

// decomposed_conv3d.cpp:19 (the state is per thread, as the VAE driver sets
// it around each temporal slice)
thread_local MemoryState current_memory_state = MemoryState::DISABLED;

size_t align16(size_t bytes) { return (bytes + 15) & ~size_t(15); }

} // namespace

MemoryState get_vae_memory_state()
{
    return current_memory_state;
}

void set_vae_memory_state(MemoryState state)
{
    current_memory_state = state;
}

DecomposedConv3D::DecomposedConv3D()
    : weights_dirty(true), memory_current(-1), memory_frames(0), memory_w(0), memory_h(0),
      memory_elemsize(0)
{
    one_blob_only = true;
    support_inplace = false;
    memset(&config, 0, sizeof(config));
}

DecomposedConv3D::~DecomposedConv3D()
{
}

// ParamDict ids and defaults of the reference load_param (:399-418).
int DecomposedConv3D::load_param(const ncnn::ParamDict& pd)
{
    std::lock_guard<std::mutex> lock(mutex);
    config.num_output = pd.get(0, 0);
    config.num_input = pd.get(1, 0);
    config.kernel_w = pd.get(2, 0);
    config.kernel_h = pd.get(3, 0);
    config.kernel_t = pd.get(4, 0);
    config.stride_t = pd.get(5, 1);
    config.dilation_t = pd.get(6, 1);
    config.head_frames = pd.get(7, 0);
    config.stride_w = pd.get(8, 1);
    config.stride_h = pd.get(9, 1);
    config.dilation_w = pd.get(10, 1);
    config.dilation_h = pd.get(11, 1);
    config.pad_w = pd.get(12, 0);
    config.pad_h = pd.get(13, 0);
    config.groups = pd.get(14, 1);
    config.bias_term = pd.get(15, 0) != 0;
    return 0;
}

bool DecomposedConv3D::config_ok() const
{
    const s2_conv3d_config& c = config;
    return c.num_output > 0 && c.num_input > 0 && c.kernel_w > 0 && c.kernel_h > 0 &&
           c.kernel_t > 0 && c.stride_t > 0 && c.dilation_t > 0 && c.stride_w > 0 &&
           c.stride_h > 0 && c.dilation_w > 0 && c.dilation_h > 0 && c.groups > 0 &&
           c.num_input % c.groups == 0 && c.num_output % c.groups == 0 && c.head_frames >= 0;
}

// Weight layout of the reference load_model (:420-472): a raw fp32 config
// blob of 16 values (it overrides the ParamDict), the bias [num_output] when
// bias_term, then kernel_t raw fp32 ncnn Convolution weights
// [num_output][num_input / groups][kernel_h][kernel_w].
int DecomposedConv3D::load_model(const ncnn::ModelBin& mb)
{
    std::lock_guard<std::mutex> lock(mutex);
    weights_dirty = true;
    const ncnn::Mat blob = mb.load(16, 1);
    if (blob.empty())
        return -100;
    const float* v = blob;
    int* fields = &config.num_output;
    for (int i = 0; i < 16; i++)
        fields[i] = static_cast<int>(v[i]);
    config.bias_term = config.bias_term != 0;
    if (!config_ok())
        return -1;
    if (config.bias_term)
    {
        bias_data = mb.load(config.num_output, 1);
        if (bias_data.empty())
            return -100;
    }
    const int per_tap = config.num_output * (config.num_input / config.groups) * config.kernel_w *
                        config.kernel_h;
    weight_data.create(per_tap * config.kernel_t, (size_t)4u);
    if (weight_data.empty())
        return -100;
    for (int t = 0; t < config.kernel_t; t++)
    {
        const ncnn::Mat tap = mb.load(per_tap, 1);
        if (tap.empty())
            return -100;
        memcpy(static_cast<float*>(weight_data) + (size_t)t * per_tap, tap.data,
               sizeof(float) * per_tap);
    }
    return 0;
}

int DecomposedConv3D::create_pipeline(const ncnn::Option& /*opt*/)
{
    return layer_status(create_pipeline_impl());
}

int DecomposedConv3D::create_pipeline_impl()
{
    std::lock_guard<std::mutex> lock(mutex);
    // the host-blob path runs on the default stream: own its scratch
    const int sret = host_scratch.take(0);
    if (sret != S2_OK)
        return sret;
    int devices = 0;
    if (s2_device_count(&devices) != S2_OK || devices == 0 || weight_data.empty() ||
        config.groups != 1)
        return 0;
    return upload_weights_locked();
}

int DecomposedConv3D::destroy_pipeline(const ncnn::Option& /*opt*/)
{
    std::lock_guard<std::mutex> lock(mutex);
    host_scratch.drop();
    packed_gpu.release();
    bias_gpu.release();
    workspace.release();
    staging.release();
    memory[0].release();
    memory[1].release();
    memory_current = -1;
    weights_dirty = true;
    return 0;
}

void DecomposedConv3D::release_completed_temporal_memory() const
{
    // the buffer the last forward read (the reference's previous memory)
    std::lock_guard<std::mutex> lock(mutex);
    if (memory_current >= 0)
        memory[1 - memory_current].release();
}

void DecomposedConv3D::reset_temporal_memory() const
{
    std::lock_guard<std::mutex> lock(mutex);
    memory[0].release();
    memory[1].release();
    memory_current = -1;
}

// The weights stay resident in the kernel's packed bf16 layout.
int DecomposedConv3D::upload_weights_locked() const
{
    if (!weights_dirty && packed_gpu.get())
        return 0;
    size_t packed_bytes = 0;
    int ret = s2_conv3d_packed_weight_bytes(&config, &packed_bytes);
    if (ret != 0)
        return ret;
    const size_t count = weight_data.total();
    DeviceBuffer tmp;
    ret = tmp.reserve(count * sizeof(float));
    if (ret == 0)
        ret = packed_gpu.reserve(packed_bytes);
    if (ret == 0)
        ret = s2_memcpy_h2d(tmp.get(), weight_data.data, count * sizeof(float), 0);
    if (ret == 0)
        ret = s2_conv3d_pack_weights(&config, static_cast<const float*>(tmp.get()),
                                     packed_gpu.get(), 0);
    if (ret == 0 && config.bias_term)
    {
        ret = bias_gpu.reserve(config.num_output * sizeof(float));
        if (ret == 0)
            ret = s2_memcpy_h2d(bias_gpu.get(), bias_data.data,
                                config.num_output * sizeof(float), 0);
    }
    if (ret == 0)
        ret = s2_stream_synchronize(0);
    if (ret == 0)
        weights_dirty = false;
    return ret;
}

int DecomposedConv3D::output_shape_locked(int frames, int h, int w, size_t elemsize,
                                          int pad_right, int pad_bottom, int out[3]) const
{
    if (weight_data.empty() || pad_right < 0 || pad_bottom < 0)
        return -1;
    const bool use_memory = get_vae_memory_state() == MemoryState::ACTIVE && memory_current >= 0;
    // the memory must hold frames of this input (:617-624)
    if (use_memory && (memory_w != w || memory_h != h || memory_elemsize != elemsize))
        return -1;
    return s2_conv3d_output_shape(&config, frames, h + pad_bottom, w + pad_right,
                                  use_memory ? memory_frames : 0, out) == S2_OK ? 0 : -1;
}

int DecomposedConv3D::output_shape(int frames, int h, int w, size_t elemsize, int pad_right,
                                   int pad_bottom, int out[3]) const
{
    std::lock_guard<std::mutex> lock(mutex);
    return output_shape_locked(frames, h, w, elemsize, pad_right, pad_bottom, out);
}

// decomposed_conv3d.cpp:605-755 on device memory
int DecomposedConv3D::forward_device(const void* input, s2_dtype dtype, size_t elemsize,
                                     int frames, int h, int w, long in_cstep, int pad_right,
                                     int pad_bottom, void* output, long out_cstep,
                                     void* stream) const
{
    std::lock_guard<std::mutex> lock(mutex);
    const MemoryState state = get_vae_memory_state();
    if (state != MemoryState::ACTIVE)
        memory_current = -1;
    int out[3];
    if (output_shape_locked(frames, h, w, elemsize, pad_right, pad_bottom, out) != 0)
        return -1;
    const bool use_memory = state == MemoryState::ACTIVE && memory_current >= 0;
    const int mframes = use_memory ? memory_frames : 0;
    int devices = 0;
    if (s2_device_count(&devices) != S2_OK || devices == 0)
        return S2_ERR_DEVICE;
    int ret = upload_weights_locked();
    if (ret != 0)
        return ret;
    size_t ws_bytes = 0;
    ret = s2_conv3d_workspace_bytes_padded(&config, frames, h, w, pad_right, pad_bottom, mframes,
                                           &ws_bytes);
    if (ret == 0)
        ret = workspace.reserve(ws_bytes);
    if (ret != 0)
        return ret;
    // the next memory (:727-755): kept unless the memory is disabled
    size_t mem_bytes = 0;
    int cache = 0;
    ret = s2_conv3d_memory_bytes(&config, h, w, &mem_bytes, &cache);
    if (ret != 0)
        return ret;
    const bool keep = state != MemoryState::DISABLED && cache > 0;
    const int next = memory_current == 0 ? 1 : 0;
    if (keep)
    {
        ret = memory[next].reserve(mem_bytes);
        if (ret != 0)
            return ret;
    }
    const float* bias = config.bias_term ? static_cast<const float*>(bias_gpu.get()) : 0;
    ret = s2_conv3d_forward_padded(&config, packed_gpu.get(), bias, input, dtype, frames, h, w,
                                   in_cstep, pad_right, pad_bottom,
                                   use_memory ? memory[memory_current].get() : 0, mframes, output,
                                   dtype, out_cstep, keep ? memory[next].get() : 0,
                                   workspace.get(), ws_bytes, stream);
    if (ret != 0)
        return ret;
    if (keep)
    {
        memory_current = next;
        memory_frames = cache;
        memory_w = w;
        memory_h = h;
        memory_elemsize = elemsize;
    }
    return 0;
}

// decomposed_conv3d.cpp:605-755
int DecomposedConv3D::forward(const ncnn::Mat& bottom_blob, ncnn::Mat& top_blob,
                              const ncnn::Option& opt) const
{
    return layer_status(forward_impl(bottom_blob, top_blob, opt));
}

int DecomposedConv3D::forward_impl(const ncnn::Mat& bottom_blob, ncnn::Mat& top_blob,
                              const ncnn::Option& opt) const
{
    if (bottom_blob.dims != 4 || bottom_blob.c != config.num_input || bottom_blob.elempack != 1)
        return -1;
    HipDeviceAllocator* device = device_allocator_of(bottom_blob);
    const size_t elemsize = bottom_blob.elemsize;
    if (!device && elemsize != sizeof(float))
        return -1;
    if (device && elemsize != 4 && elemsize != 2)
        return -1;
    {
        // a forward outside ACTIVE drops the memory even when it fails
        std::lock_guard<std::mutex> lock(mutex);
        if (get_vae_memory_state() != MemoryState::ACTIVE)
            memory_current = -1;
    }
    int out[3];
    if (output_shape(bottom_blob.d, bottom_blob.h, bottom_blob.w, elemsize, 0, 0, out) != 0)
        return -1;
    if (device)
    {
        HipDeviceAllocator* out_alloc = dynamic_cast<HipDeviceAllocator*>(opt.blob_allocator);
        if (!out_alloc)
            out_alloc = device;
        top_blob = out_alloc->create_blob(out[2], out[1], out[0], config.num_output, elemsize);
        if (top_blob.empty())
            return -100;
        return forward_device(bottom_blob.data, device_blob_dtype(elemsize, opt), elemsize,
                              bottom_blob.d, bottom_blob.h, bottom_blob.w, (long)bottom_blob.cstep,
                              0, 0, top_blob.data, (long)top_blob.cstep, device->stream());
    }

    // Host fp32 blobs: stage, compute, download, synchronise.
    const size_t in_bytes = bottom_blob.cstep * bottom_blob.c * sizeof(float);
    const size_t out_cstep = align16((size_t)out[0] * out[1] * out[2] * sizeof(float)) /
                             sizeof(float);
    const size_t out_bytes = out_cstep * config.num_output * sizeof(float);
    int ret;
    unsigned char* x;
    unsigned char* y;
    {
        std::lock_guard<std::mutex> lock(mutex);
        ret = staging.reserve(align16(in_bytes) + out_bytes);
        x = static_cast<unsigned char*>(staging.get());
        y = x + align16(in_bytes);
    }
    if (ret != 0)
        return ret;
    ret = s2_memcpy_h2d(x, bottom_blob.data, in_bytes, 0);
    if (ret == 0)
        ret = forward_device(x, S2_DTYPE_F32, 4, bottom_blob.d, bottom_blob.h, bottom_blob.w,
                             (long)bottom_blob.cstep, 0, 0, y, (long)out_cstep, 0);
    if (ret != 0)
        return ret;
    top_blob.create(out[2], out[1], out[0], config.num_output, 4u, opt.blob_allocator);
    if (top_blob.empty() || top_blob.cstep != out_cstep)
        return -100;
    ret = s2_memcpy_d2h(top_blob.data, y, out_bytes, 0);
    if (ret == 0)
        ret = s2_stream_synchronize(0);
    return ret;
}

ncnn::Layer* decomposed_conv3d_layer_creator(void* /*userdata*/)
{
    return new DecomposedConv3D;
}

void decomposed_conv3d_layer_destroyer(ncnn::Layer* layer, void* /*userdata*/)
{
    delete layer;
}

} // namespace seedvr2
