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

DiTStreamOp::DiTStreamOp(int _kind, int _stream, const AdaptiveWindowRuntimeState* _state,
                         float _epsilon, const ncnn::Mat& gate, const ncnn::Mat& shift,
                         const ncnn::Mat& scale)
    : kind(_kind), stream(_stream), state(_state), epsilon(_epsilon), dirty(true)
{
    one_blob_only = false;
    support_inplace = false;
    vectors[0] = gate;
    vectors[1] = shift;
    vectors[2] = scale;
}

DiTStreamOp::~DiTStreamOp()
{
}

int DiTStreamOp::create_pipeline(const ncnn::Option& /*opt*/)
{
    std::lock_guard<std::mutex> lock(mutex);
    int devices = 0;
    if (s2_device_count(&devices) != S2_OK || devices == 0)
        return 0;
    return layer_status(upload_locked());
}

int DiTStreamOp::destroy_pipeline(const ncnn::Option& /*opt*/)
{
    std::lock_guard<std::mutex> lock(mutex);
    vectors_gpu.release();
    dirty = true;
    return 0;
}

int DiTStreamOp::upload_locked() const
{
    if (!dirty)
        return S2_OK;
    int hidden = 0;
    for (int i = 0; i < 3; i++)
        if (!vectors[i].empty())
            hidden = vectors[i].w;
    if (hidden == 0)
    {
        dirty = false;
        return S2_OK;
    }
    const size_t bytes = (size_t)hidden * sizeof(float);
    int ret = vectors_gpu.reserve(3 * bytes);
    for (int i = 0; ret == S2_OK && i < 3; i++)
        if (!vectors[i].empty())
            ret = s2_memcpy_h2d((char*)vectors_gpu.get() + i * bytes, vectors[i].data, bytes, 0);
    if (ret == S2_OK)
        ret = s2_stream_synchronize(0);
    if (ret == S2_OK)
        dirty = false;
    return ret;
}

int DiTStreamOp::forward(const std::vector<ncnn::Mat>& bottom_blobs,
                         std::vector<ncnn::Mat>& top_blobs, const ncnn::Option& opt) const
{
    std::lock_guard<std::mutex> lock(mutex);
    const int n_bottoms[3] = {3, 3, 5};
    const int n_tops[3] = {1, 1, 2};
    if (!state || (int)bottom_blobs.size() != n_bottoms[kind] || (int)top_blobs.size() != n_tops[kind])
        return -1;
    const int batch = (int)state->video_shapes.size();
    if (batch <= 0 || batch > 64 || (int)state->text_lengths.size() != batch)
        return -1;
    // this stream's rows per sample; the other stream has none
    std::vector<int> rows(batch), none(batch, 0);
    int total = 0;
    for (int b = 0; b < batch; b++)
    {
        const std::array<int, 3>& s = state->video_shapes[b];
        rows[b] = stream == 0 ? s[0] * s[1] * s[2] : state->text_lengths[b];
        if (rows[b] < 0)
            return -1;
        total += rows[b];
    }
    const ncnn::Mat& x = bottom_blobs[0];
    const int hidden = x.w;
    for (int i = 0; i < 3; i++)
        if (!vectors[i].empty() && vectors[i].w != hidden)
            return -1;
    if (hidden <= 0 || hidden % 4 != 0 || hidden > 4096 || !rows_ok(x, hidden, total))
        return -1;
    HipDeviceAllocator* dev = device_allocator_of(x);
    HipDeviceAllocator* out = dynamic_cast<HipDeviceAllocator*>(opt.blob_allocator);
    if (!out)
        out = dev;
    int ret = upload_locked();
    if (ret != S2_OK)
        return layer_status(ret);
    const float* sv = vectors_gpu.get() ? static_cast<const float*>(vectors_gpu.get()) : 0;
    const float* own[3];
    for (int i = 0; i < 3; i++)
        own[i] = vectors[i].empty() ? 0 : sv + (size_t)i * hidden;
    const s2_dtype x_dtype = device_blob_dtype(x.elemsize, opt);
    const size_t h_elem = (opt.use_bf16_storage || opt.use_fp16_storage) ? 2 : 4;
    const s2_dtype h_dtype = device_blob_dtype(h_elem, opt);
    const int* vr = stream == 0 ? &rows[0] : &none[0];
    const int* tr = stream == 0 ? 0 : &rows[0];
    void* s = dev->stream();
    // pointers of this stream in its slot of the two-stream entry points
    const void* xv = stream == 0 ? x.data : 0;
    const void* xt = stream == 0 ? 0 : x.data;
    auto vec = [&](int i, int want_stream) { return stream == want_stream ? own[i] : 0; };

    if (kind == 0)
    {
        const ncnn::Mat& shift = bottom_blobs[1];
        const ncnn::Mat& scale = bottom_blobs[2];
        if (!modulation_ok(shift, hidden, batch) || !modulation_ok(scale, hidden, batch))
            return -1;
        top_blobs[0] = out->create_blob(hidden, total, h_elem);
        if (top_blobs[0].empty())
            return -100;
        void* hv = stream == 0 ? top_blobs[0].data : 0;
        void* ht = stream == 0 ? 0 : top_blobs[0].data;
        ret = s2_dit_ada_in(hidden, epsilon, batch, vr, tr, xv, xt, x_dtype, hidden,
                            (const float*)shift.data, (const float*)scale.data, vec(1, 0), vec(2, 0),
                            vec(1, 1), vec(2, 1), hv, ht, h_dtype, hidden, s);
        return layer_status(ret);
    }
    const ncnn::Mat& y = bottom_blobs[1];
    const ncnn::Mat& gate = bottom_blobs[2];
    if (!rows_ok(y, hidden, total) || !modulation_ok(gate, hidden, batch))
        return -1;
    const s2_dtype y_dtype = device_blob_dtype(y.elemsize, opt);
    const void* yv = stream == 0 ? y.data : 0;
    const void* yt = stream == 0 ? 0 : y.data;
    top_blobs[0] = out->create_blob(hidden, total, x.elemsize);
    if (top_blobs[0].empty())
        return -100;
    void* ov = stream == 0 ? top_blobs[0].data : 0;
    void* ot = stream == 0 ? 0 : top_blobs[0].data;
    if (kind == 1)
    {
        ret = s2_dit_ada_out(hidden, batch, vr, tr, xv, xt, x_dtype, hidden, yv, yt, y_dtype, hidden,
                             (const float*)gate.data, vec(0, 0), vec(0, 1), ov, ot, hidden, s);
        return layer_status(ret);
    }
    const ncnn::Mat& shift = bottom_blobs[3];
    const ncnn::Mat& scale = bottom_blobs[4];
    if (!modulation_ok(shift, hidden, batch) || !modulation_ok(scale, hidden, batch))
        return -1;
    top_blobs[1] = out->create_blob(hidden, total, h_elem);
    if (top_blobs[1].empty())
        return -100;
    void* hv = stream == 0 ? top_blobs[1].data : 0;
    void* ht = stream == 0 ? 0 : top_blobs[1].data;
    ret = s2_dit_ada_out_in(hidden, batch, vr, tr, xv, xt, x_dtype, hidden, yv, yt, y_dtype, hidden,
                            (const float*)gate.data, vec(0, 0), vec(0, 1), ov, ot, hidden, epsilon,
                            (const float*)shift.data, (const float*)scale.data, vec(1, 0), vec(2, 0),
                            vec(1, 1), vec(2, 1), hv, ht, h_dtype, hidden, s);
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
