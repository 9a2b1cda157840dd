// DiT block norm / AdaSingle modulation layers (dit_block_ops.h) over the
// s2_dit_ada_* C-ABI.
#include "dit_block_ops.h"

#include <modelbin.h>
#include <paramdict.h>

#include "seedvr2_hip.h"

namespace seedvr2 {

namespace {

const int kVectorCount[3] = {4, 2, 6};
const int kBottoms[3] = {4, 5, 7};
const int kTops[3] = {2, 2, 4};

// A [batch][hidden] fp32 modulation blob on the device.
bool modulation_ok(const ncnn::Mat& m, int hidden, int batch)
{
    if (!device_allocator_of(m) || m.elemsize != 4 || m.elempack != 1)
        return false;
    if (m.dims == 2)
        return m.w == hidden && m.h == batch;
    return m.dims == 1 && m.w == hidden * batch;
}

bool rows_ok(const ncnn::Mat& m, int hidden, int rows)
{
    return device_allocator_of(m) && m.dims == 2 && m.elempack == 1 && m.w == hidden &&
           m.h == rows && (m.elemsize == 4 || m.elemsize == 2);
}

}  // namespace

DiTBlockOp::DiTBlockOp(int _kind, const AdaptiveWindowRuntimeState* _state)
    : kind(_kind), state(_state), hidden(0), epsilon(1e-5f), stream_vectors(0), dirty(true)
{
    one_blob_only = false;
    support_inplace = false;
}

DiTBlockOp::~DiTBlockOp()
{
}

int DiTBlockOp::load_param(const ncnn::ParamDict& pd)
{
    std::lock_guard<std::mutex> lock(mutex);
    hidden = pd.get(0, 0);
    epsilon = pd.get(1, 1e-5f);
    stream_vectors = pd.get(2, 0);
    if (hidden <= 0 || hidden % 4 != 0 || hidden > 4096 || epsilon < 0.f ||
        (stream_vectors != 0 && stream_vectors != 1))
        return -1;
    vectors.clear();
    dirty = true;
    return 0;
}

int DiTBlockOp::load_model(const ncnn::ModelBin& mb)
{
    std::lock_guard<std::mutex> lock(mutex);
    vectors.clear();
    dirty = true;
    if (!stream_vectors)
        return 0;
    for (int i = 0; i < kVectorCount[kind]; i++)
    {
        ncnn::Mat v = mb.load(hidden, 1);
        if (v.empty())
            return -100;
        vectors.push_back(v);
    }
    return 0;
}

int DiTBlockOp::create_pipeline(const ncnn::Option& /*opt*/)
{
    std::lock_guard<std::mutex> lock(mutex);
    int devices = 0;
    if (s2_device_count(&devices) != S2_OK || devices == 0)
        return 0;
    return layer_status(upload_locked());
}

int DiTBlockOp::destroy_pipeline(const ncnn::Option& /*opt*/)
{
    std::lock_guard<std::mutex> lock(mutex);
    vectors_gpu.release();
    dirty = true;
    return 0;
}

int DiTBlockOp::upload_locked() const
{
    if (!dirty || vectors.empty())
        return S2_OK;
    const size_t bytes = (size_t)hidden * sizeof(float);
    int ret = vectors_gpu.reserve(bytes * vectors.size());
    for (size_t i = 0; ret == S2_OK && i < vectors.size(); i++)
        ret = s2_memcpy_h2d((char*)vectors_gpu.get() + i * bytes, vectors[i].data, bytes, 0);
    if (ret == S2_OK)
        ret = s2_stream_synchronize(0);
    if (ret == S2_OK)
        dirty = false;
    return ret;
}

int DiTBlockOp::forward(const std::vector<ncnn::Mat>& bottom_blobs,
                        std::vector<ncnn::Mat>& top_blobs, const ncnn::Option& opt) const
{
    std::lock_guard<std::mutex> lock(mutex);
    if (!state || hidden <= 0 || (int)bottom_blobs.size() != kBottoms[kind] ||
        (int)top_blobs.size() != kTops[kind])
        return -1;
    const int batch = (int)state->video_shapes.size();
    if (batch <= 0 || batch > 64 || (int)state->text_lengths.size() != batch)
        return -1;
    std::vector<int> vrows(batch), trows(batch);
    int lv = 0, lt = 0;
    for (int b = 0; b < batch; b++)
    {
        const std::array<int, 3>& s = state->video_shapes[b];
        if (s[0] <= 0 || s[1] <= 0 || s[2] <= 0 || state->text_lengths[b] < 0)
            return -1;
        vrows[b] = s[0] * s[1] * s[2];
        trows[b] = state->text_lengths[b];
        lv += vrows[b];
        lt += trows[b];
    }
    const ncnn::Mat& xv = bottom_blobs[0];
    const ncnn::Mat& xt = bottom_blobs[1];
    if (!rows_ok(xv, hidden, lv) || (lt > 0 && !rows_ok(xt, hidden, lt)) ||
        (lt > 0 && xt.elemsize != xv.elemsize))
        return -1;
    HipDeviceAllocator* dev = device_allocator_of(xv);
    HipDeviceAllocator* out = dynamic_cast<HipDeviceAllocator*>(opt.blob_allocator);
    if (!out)
        out = dev;
    int ret = upload_locked();
    if (ret != S2_OK)
        return layer_status(ret);
    const float* sv = vectors.empty() ? 0 : static_cast<const float*>(vectors_gpu.get());
    const s2_dtype x_dtype = device_blob_dtype(xv.elemsize, opt);
    const size_t h_elem = (opt.use_bf16_storage || opt.use_fp16_storage) ? 2 : 4;
    const s2_dtype h_dtype = device_blob_dtype(h_elem, opt);
    const int* tr = lt > 0 ? &trows[0] : 0;
    void* stream = dev->stream();

    if (kind == 0)
    {
        const ncnn::Mat& shift = bottom_blobs[2];
        const ncnn::Mat& scale = bottom_blobs[3];
        if (!modulation_ok(shift, hidden, batch) || !modulation_ok(scale, hidden, batch))
            return -1;
        top_blobs[0] = out->create_blob(hidden, lv, h_elem);
        top_blobs[1] = lt > 0 ? out->create_blob(hidden, lt, h_elem) : ncnn::Mat();
        if (top_blobs[0].empty() || (lt > 0 && top_blobs[1].empty()))
            return -100;
        ret = s2_dit_ada_in(hidden, epsilon, batch, &vrows[0], tr, xv.data, lt ? xt.data : 0,
                            x_dtype, hidden, (const float*)shift.data, (const float*)scale.data,
                            sv ? sv : 0, sv ? sv + hidden : 0, sv ? sv + 2 * hidden : 0,
                            sv ? sv + 3 * hidden : 0, top_blobs[0].data,
                            lt ? top_blobs[1].data : 0, h_dtype, hidden, stream);
        return layer_status(ret);
    }

    const ncnn::Mat& yv = bottom_blobs[2];
    const ncnn::Mat& yt = bottom_blobs[3];
    const ncnn::Mat& gate = bottom_blobs[4];
    if (!rows_ok(yv, hidden, lv) || (lt > 0 && !rows_ok(yt, hidden, lt)) ||
        (lt > 0 && yt.elemsize != yv.elemsize) || !modulation_ok(gate, hidden, batch))
        return -1;
    const s2_dtype y_dtype = device_blob_dtype(yv.elemsize, opt);
    top_blobs[0] = out->create_blob(hidden, lv, xv.elemsize);
    top_blobs[1] = lt > 0 ? out->create_blob(hidden, lt, xv.elemsize) : ncnn::Mat();
    if (top_blobs[0].empty() || (lt > 0 && top_blobs[1].empty()))
        return -100;
    if (kind == 1)
    {
        ret = s2_dit_ada_out(hidden, batch, &vrows[0], tr, xv.data, lt ? xt.data : 0, x_dtype,
                             hidden, yv.data, lt ? yt.data : 0, y_dtype, hidden,
                             (const float*)gate.data, sv ? sv : 0, sv ? sv + hidden : 0,
                             top_blobs[0].data, lt ? top_blobs[1].data : 0, hidden, stream);
        return layer_status(ret);
    }
    const ncnn::Mat& shift = bottom_blobs[5];
    const ncnn::Mat& scale = bottom_blobs[6];
    if (!modulation_ok(shift, hidden, batch) || !modulation_ok(scale, hidden, batch))
        return -1;
    top_blobs[2] = out->create_blob(hidden, lv, h_elem);
    top_blobs[3] = lt > 0 ? out->create_blob(hidden, lt, h_elem) : ncnn::Mat();
    if (top_blobs[2].empty() || (lt > 0 && top_blobs[3].empty()))
        return -100;
    ret = s2_dit_ada_out_in(hidden, batch, &vrows[0], tr, xv.data, lt ? xt.data : 0, x_dtype,
                            hidden, yv.data, lt ? yt.data : 0, y_dtype, hidden,
                            (const float*)gate.data, sv ? sv : 0, sv ? sv + hidden : 0,
                            top_blobs[0].data, lt ? top_blobs[1].data : 0, hidden, epsilon,
                            (const float*)shift.data, (const float*)scale.data,
                            sv ? sv + 2 * hidden : 0, sv ? sv + 3 * hidden : 0,
                            sv ? sv + 4 * hidden : 0, sv ? sv + 5 * hidden : 0, top_blobs[2].data,
                            lt ? top_blobs[3].data : 0, h_dtype, hidden, stream);
    return layer_status(ret);
}

ncnn::Layer* dit_ada_in_layer_creator(void* userdata)
{
    return new DiTBlockOp(0, static_cast<const AdaptiveWindowRuntimeState*>(userdata));
}

ncnn::Layer* dit_ada_out_layer_creator(void* userdata)
{
    return new DiTBlockOp(1, static_cast<const AdaptiveWindowRuntimeState*>(userdata));
}

ncnn::Layer* dit_ada_out_in_layer_creator(void* userdata)
{
    return new DiTBlockOp(2, static_cast<const AdaptiveWindowRuntimeState*>(userdata));
}

void dit_block_op_layer_destroyer(ncnn::Layer* layer, void* /*userdata*/)
{
    delete layer;
}

}  // namespace seedvr2
