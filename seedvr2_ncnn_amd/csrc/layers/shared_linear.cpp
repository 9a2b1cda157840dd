// SharedLinear on MI355X: the ncnn layer surface of the reference
// (src/seedvr2/shared_linear.cpp:10-149) over the HIP C-ABI.
#include "shared_linear.h"

#include <string.h>

#include <modelbin.h>

#include "seedvr2_hip.h"

namespace seedvr2 {

SharedLinear::SharedLinear()
    : num_output(0), num_input(0), bias_term(false), activation(0), params_loaded(false),
      weights_dirty(true)
{
    one_blob_only = false;
    support_inplace = false;
}

SharedLinear::~SharedLinear()
{
}

// ParamDict ids of the reference load_param (:27-59).
int SharedLinear::load_param(const ncnn::ParamDict& pd)
{
    std::lock_guard<std::mutex> lock(mutex);
    num_output = pd.get(0, 0);
    num_input = pd.get(1, 0);
    bias_term = pd.get(2, 0) != 0;
    activation = pd.get(3, 0);
    params_loaded = false;
    if (num_output <= 0 || num_input <= 0)
        return -1;
    if (activation != S2_ACT_NONE && activation != S2_ACT_GELU && activation != S2_ACT_SWIGLU)
        return -1;
    // SwiGLU (this build's id 3 = 2): num_output gate and num_output up
    // rows; the fused epilogue needs whole 128-column blocks and 64-wide k steps
    if (activation == S2_ACT_SWIGLU && (num_output % 128 != 0 || num_input % 64 != 0))
        return -1;
    params_loaded = true;
    weights_dirty = true;
    return 0;
}

// Weight layout of the reference load_model (:61-81): raw fp32 [N][K]
// weight, then raw fp32 [N] bias when bias_term.
int SharedLinear::load_model(const ncnn::ModelBin& mb)
{
    std::lock_guard<std::mutex> lock(mutex);
    if (!params_loaded)
        return -1;
    weights_dirty = true;
    // SwiGLU: the gate projection's [N][K] weight, then the up projection's
    // (and the two biases in the same order)
    const int rows = activation == S2_ACT_SWIGLU ? 2 * num_output : num_output;
    weight_data = mb.load(num_input * rows, 1);
    if (weight_data.empty())
        return -100;
    weight_data = weight_data.reshape(num_input, rows);
    if (weight_data.empty())
        return -100;
    if (bias_term)
    {
        bias_data = mb.load(rows, 1);
        if (bias_data.empty())
            return -100;
    }
    if (activation == S2_ACT_SWIGLU)
    {
        // interleave 128-row blocks: gate rows 128j.., then up rows 128j..
        // (the weight layout of s2_shared_linear_forward's SwiGLU)
        ncnn::Mat w(num_input, rows);
        ncnn::Mat b;
        if (bias_term)
            b.create(rows);
        if (w.empty() || (bias_term && b.empty()))
            return -100;
        const size_t blk = (size_t)128 * num_input;
        for (int j = 0; j < num_output / 128; j++)
        {
            memcpy((float*)w.data + (2 * j) * blk, (const float*)weight_data.data + j * blk,
                   blk * sizeof(float));
            memcpy((float*)w.data + (2 * j + 1) * blk,
                   (const float*)weight_data.data + (num_output / 128 + j) * blk, blk * sizeof(float));
            if (bias_term)
            {
                memcpy((float*)b.data + 2 * j * 128, (const float*)bias_data.data + j * 128, 512);
                memcpy((float*)b.data + (2 * j + 1) * 128,
                       (const float*)bias_data.data + num_output + j * 128, 512);
            }
        }
        weight_data = w;
        if (bias_term)
            bias_data = b;
    }
    return 0;
}

SharedLinear* SharedLinear::stack(const std::vector<const SharedLinear*>& parts, int act)
{
    if (parts.empty() || (act != S2_ACT_NONE && act != S2_ACT_SWIGLU) ||
        (act == S2_ACT_SWIGLU && parts.size() != 2))
        return 0;
    const int k = parts[0]->num_input;
    int n = 0;
    bool any_bias = false;
    for (size_t i = 0; i < parts.size(); i++)
    {
        const SharedLinear* p = parts[i];
        std::lock_guard<std::mutex> lock(p->mutex);
        if (p->num_input != k || p->activation != S2_ACT_NONE || p->weight_data.empty())
            return 0;
        n += p->num_output;
        any_bias = any_bias || p->bias_term;
    }
    if (act == S2_ACT_SWIGLU && parts[0]->num_output != parts[1]->num_output)
        return 0;
    ncnn::Mat w((int)((size_t)k * n));
    ncnn::Mat b;
    if (any_bias)
        b.create(n);
    if (w.empty() || (any_bias && b.empty()))
        return 0;
    size_t row = 0;
    for (size_t i = 0; i < parts.size(); i++)
    {
        const SharedLinear* p = parts[i];
        std::lock_guard<std::mutex> lock(p->mutex);
        memcpy((float*)w.data + row * k, p->weight_data.data, (size_t)p->num_output * k * sizeof(float));
        if (any_bias)
        {
            float* bd = (float*)b.data + row;
            if (p->bias_term)
                memcpy(bd, p->bias_data.data, (size_t)p->num_output * sizeof(float));
            else
                memset(bd, 0, (size_t)p->num_output * sizeof(float));
        }
        row += p->num_output;
    }
    ncnn::ParamDict pd;
    pd.set(0, act == S2_ACT_SWIGLU ? n / 2 : n);
    pd.set(1, k);
    pd.set(2, any_bias ? 1 : 0);
    pd.set(3, act);
    SharedLinear* s = new SharedLinear();
    s->type = "SharedLinear";
    const ncnn::Mat mats[2] = {w, b};
    ncnn::ModelBinFromMatArray mb(mats);
    if (s->load_param(pd) != 0 || s->load_model(mb) != 0)
    {
        delete s;
        return 0;
    }
    return s;
}

int SharedLinear::set_activation(int act)
{
    if (act != S2_ACT_NONE && act != S2_ACT_GELU)
        return -1;
    std::lock_guard<std::mutex> lock(mutex);
    if (act != activation && activation != S2_ACT_NONE)
        return -1;
    activation = act;
    return 0;
}

int SharedLinear::create_pipeline(const ncnn::Option& /*opt*/)
{
    return layer_status(create_pipeline_impl());
}

int SharedLinear::create_pipeline_impl()
{
    std::lock_guard<std::mutex> lock(mutex);
    // the host-blob path runs on the default stream: own its scratch
    const int sret = host_scratch.take(0);
    if (sret != S2_OK)
        return sret;
    int devices = 0;
    if (s2_device_count(&devices) != S2_OK || devices == 0 || weight_data.empty())
        return 0;
    return upload_weights_locked();
}

int SharedLinear::destroy_pipeline(const ncnn::Option& /*opt*/)
{
    std::lock_guard<std::mutex> lock(mutex);
    host_scratch.drop();
    weight_gpu.release();
    bias_gpu.release();
    staging.release();
    weights_dirty = true;
    return 0;
}

// The weight stays resident in bf16 (rounded to nearest even once, here).
int SharedLinear::upload_weights_locked() const
{
    if (!weights_dirty && weight_gpu.get())
        return 0;
    const int rows = activation == S2_ACT_SWIGLU ? 2 * num_output : num_output;
    const size_t count = static_cast<size_t>(num_input) * rows;
    DeviceBuffer tmp;
    int ret = tmp.reserve(count * sizeof(float));
    if (ret == 0)
        ret = weight_gpu.reserve(count * sizeof(uint16_t));
    if (ret == 0)
        ret = s2_memcpy_h2d(tmp.get(), weight_data.data, count * sizeof(float), 0);
    if (ret == 0)
        ret = s2_cast_f32_to_bf16(static_cast<const float*>(tmp.get()),
                                  static_cast<uint16_t*>(weight_gpu.get()), count, 0);
    if (ret == 0 && bias_term)
    {
        ret = bias_gpu.reserve(rows * sizeof(float));
        if (ret == 0)
            ret = s2_memcpy_h2d(bias_gpu.get(), bias_data.data, rows * sizeof(float), 0);
    }
    if (ret == 0)
        ret = s2_stream_synchronize(0);
    if (ret == 0)
        weights_dirty = false;
    return ret;
}

int SharedLinear::device_weights(const uint16_t** weight, const float** bias) const
{
    std::lock_guard<std::mutex> lock(mutex);
    if (!params_loaded || weight_data.empty())
        return -1;
    const int ret = upload_weights_locked();
    if (ret != 0)
        return ret;
    *weight = static_cast<const uint16_t*>(weight_gpu.get());
    *bias = bias_term ? static_cast<const float*>(bias_gpu.get()) : 0;
    return 0;
}

int SharedLinear::forward(const std::vector<ncnn::Mat>& bottom_blobs,
                          std::vector<ncnn::Mat>& top_blobs,
                          const ncnn::Option& opt) const
{
    return layer_status(forward_impl(bottom_blobs, top_blobs, opt));
}

int SharedLinear::forward_impl(const std::vector<ncnn::Mat>& bottom_blobs,
                          std::vector<ncnn::Mat>& top_blobs,
                          const ncnn::Option& opt) const
{
    std::lock_guard<std::mutex> lock(mutex);
    // Arity and widths (reference :87-90).
    if (!params_loaded || weight_data.empty() || bottom_blobs.size() != 2 || top_blobs.size() != 2 ||
        bottom_blobs[0].dims != 2 || bottom_blobs[1].dims != 2 ||
        bottom_blobs[0].w != num_input || bottom_blobs[1].w != num_input)
        return -1;
    HipDeviceAllocator* device = device_allocator_of(bottom_blobs[0]);
    const size_t elemsize = bottom_blobs[0].elemsize;
    if ((device_allocator_of(bottom_blobs[1]) != 0) != (device != 0) ||
        bottom_blobs[1].elemsize != elemsize || bottom_blobs[0].elempack != 1 ||
        bottom_blobs[1].elempack != 1)
        return -1;
    if (!device && elemsize != sizeof(float))
        return -1;
    if (device && elemsize != 4 && elemsize != 2)
        return -1;
    if (num_input % 8 != 0)
        return -1;   // 16-byte operand rows

    int devices = 0;
    if (s2_device_count(&devices) != S2_OK || devices == 0)
        return S2_ERR_DEVICE;
    int ret = upload_weights_locked();
    if (ret != 0)
        return ret;
    const float* bias = bias_term ? static_cast<const float*>(bias_gpu.get()) : 0;
    const int m0 = bottom_blobs[0].h;
    const int m1 = bottom_blobs[1].h;

    if (device)
    {
        HipDeviceAllocator* out_alloc = dynamic_cast<HipDeviceAllocator*>(opt.blob_allocator);
        if (!out_alloc)
            out_alloc = device;
        top_blobs[0] = out_alloc->create_blob(num_output, m0, elemsize);
        top_blobs[1] = out_alloc->create_blob(num_output, m1, elemsize);
        if ((m0 > 0 && top_blobs[0].empty()) || (m1 > 0 && top_blobs[1].empty()))
            return -100;
        const s2_dtype dtype = device_blob_dtype(elemsize, opt);
        return s2_shared_linear_forward(bottom_blobs[0].data, m0, bottom_blobs[1].data, m1, dtype,
                                        static_cast<const uint16_t*>(weight_gpu.get()), bias,
                                        num_output, num_input, activation, top_blobs[0].data,
                                        top_blobs[1].data, dtype, device->stream());
    }

    // Host fp32 blobs: stage, compute, download, synchronise.
    const size_t in0 = static_cast<size_t>(m0) * num_input;
    const size_t in1 = static_cast<size_t>(m1) * num_input;
    const size_t out0 = static_cast<size_t>(m0) * num_output;
    const size_t out1 = static_cast<size_t>(m1) * num_output;
    // (SwiGLU: room for bf16 copies of the inputs after the fp32 buffers)
    const size_t swiglu_extra = activation == S2_ACT_SWIGLU ? (in0 + in1 + 8) / 2 : 0;
    ret = staging.reserve((in0 + in1 + out0 + out1 + swiglu_extra + 4) * sizeof(float));
    if (ret != 0)
        return ret;
    float* x0 = static_cast<float*>(staging.get());
    float* x1 = x0 + in0;
    float* y0 = x1 + in1;
    float* y1 = y0 + out0;
    ret = s2_memcpy_h2d(x0, bottom_blobs[0].data, in0 * sizeof(float), 0);
    if (ret == 0)
        ret = s2_memcpy_h2d(x1, bottom_blobs[1].data, in1 * sizeof(float), 0);
    if (ret == 0 && activation == S2_ACT_SWIGLU)
    {
        // the SwiGLU epilogue runs on bf16 operands: round the staged fp32
        // rows into their own buffer (16-byte aligned), as the MFMA staging
        // of the other activations rounds them
        uintptr_t hb = reinterpret_cast<uintptr_t>(y1 + out1);
        hb = (hb + 15) & ~static_cast<uintptr_t>(15);
        uint16_t* h0 = reinterpret_cast<uint16_t*>(hb);
        uint16_t* h1 = h0 + (in0 + 7) / 8 * 8;
        ret = s2_cast_f32_to_bf16(x0, h0, in0, 0);
        if (ret == 0)
            ret = s2_cast_f32_to_bf16(x1, h1, in1, 0);
        if (ret == 0)
            ret = s2_shared_linear_forward(h0, m0, h1, m1, S2_DTYPE_BF16,
                                           static_cast<const uint16_t*>(weight_gpu.get()), bias,
                                           num_output, num_input, activation, y0, y1,
                                           S2_DTYPE_F32, 0);
    }
    else if (ret == 0)
        ret = s2_shared_linear_forward(x0, m0, x1, m1, S2_DTYPE_F32,
                                       static_cast<const uint16_t*>(weight_gpu.get()), bias,
                                       num_output, num_input, activation, y0, y1, S2_DTYPE_F32, 0);
    if (ret != 0)
        return ret;
    top_blobs[0].create(num_output, m0, 4u, opt.blob_allocator);
    top_blobs[1].create(num_output, m1, 4u, opt.blob_allocator);
    if ((m0 > 0 && top_blobs[0].empty()) || (m1 > 0 && top_blobs[1].empty()))
        return -100;
    ret = s2_memcpy_d2h(top_blobs[0].data, y0, out0 * sizeof(float), 0);
    if (ret == 0)
        ret = s2_memcpy_d2h(top_blobs[1].data, y1, out1 * sizeof(float), 0);
    if (ret == 0)
        ret = s2_stream_synchronize(0);
    return ret;
}

ncnn::Layer* shared_linear_layer_creator(void* /*userdata*/)
{
    return new SharedLinear;
}

void shared_linear_layer_destroyer(ncnn::Layer* layer, void* /*userdata*/)
{
    delete layer;
}

} // namespace seedvr2
