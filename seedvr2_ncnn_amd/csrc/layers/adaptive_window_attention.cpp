// AdaptiveWindowAttention on MI355X: the ncnn layer surface of the reference
// (src/seedvr2/adaptive_window_attention.cpp:657-978) over the HIP C-ABI.
// The host code validates blobs exactly as the reference does, keeps the
// device plan and weights cached, and either runs zero-copy on device blobs
// or stages host fp32 blobs through device memory.
#include "adaptive_window_attention.h"

#include <string.h>

#include <algorithm>
#include <memory>

#include <modelbin.h>

#include "seedvr2_hip.h"

namespace seedvr2 {

namespace {

// read_shape_value (reference :475-485): float-encoded unless int32 values.
int read_shape_value(const ncnn::Mat& values, int row, int column, bool int32_values)
{
    if (values.dims == 1)
        return int32_values ? static_cast<const int*>(values.data)[column]
                            : static_cast<int>(static_cast<const float*>(values.data)[column]);
    return int32_values ? values.row<const int>(row)[column]
                        : static_cast<int>(values.row(row)[column]);
}

int copy_vector(const std::vector<float>& src, int expected, ncnn::Mat& dst)
{
    if (static_cast<int>(src.size()) != expected)
        return -1;
    dst.create(expected);
    if (dst.empty())
        return -100;
    memcpy(dst.data, src.data(), src.size() * sizeof(float));
    return 0;
}

} // namespace

int build_adaptive_window_plan(const std::vector<std::array<int, 3> >& video_shapes,
                               const std::array<int, 3>& target_windows,
                               bool shifted,
                               AdaptiveWindowPlan& plan)
{
    plan = AdaptiveWindowPlan();
    const int batch = static_cast<int>(video_shapes.size());
    std::vector<int> shapes(3 * video_shapes.size());
    for (size_t i = 0; i < video_shapes.size(); i++)
        for (int a = 0; a < 3; a++)
            shapes[3 * i + a] = video_shapes[i][a];
    int num_windows = 0;
    int tokens = 0;
    plan.sample_window_count.resize(video_shapes.size());
    int ret = s2_awa_plan_windows(shapes.data(), batch, target_windows.data(), shifted ? 1 : 0,
                                  0, 0, &num_windows, plan.sample_window_count.data(), &tokens);
    if (ret != S2_OK)
        return ret;
    std::vector<s2_window_slice> slices(num_windows);
    ret = s2_awa_plan_windows(shapes.data(), batch, target_windows.data(), shifted ? 1 : 0,
                              slices.data(), num_windows, &num_windows, 0, 0);
    if (ret != S2_OK)
        return ret;

    // Per-token tables: window tokens in t,h,w row-major order.
    std::vector<int> sample_offset(batch, 0);
    for (int s = 1; s < batch; s++)
        sample_offset[s] = sample_offset[s - 1] +
                           video_shapes[s - 1][0] * video_shapes[s - 1][1] * video_shapes[s - 1][2];
    plan.windows.resize(num_windows);
    plan.video_indices.reserve(tokens);
    plan.local_positions.reserve(tokens);
    for (int i = 0; i < num_windows; i++)
    {
        const s2_window_slice& s = slices[i];
        WindowSlice& w = plan.windows[i];
        w.sample_index = s.sample_index;
        w.t0 = s.t0;
        w.t1 = s.t1;
        w.h0 = s.h0;
        w.h1 = s.h1;
        w.w0 = s.w0;
        w.w1 = s.w1;
        w.partition_offset = s.partition_offset;
        w.token_count = s.token_count;
        const int h = video_shapes[s.sample_index][1];
        const int wd = video_shapes[s.sample_index][2];
        for (int t = s.t0; t < s.t1; t++)
            for (int y = s.h0; y < s.h1; y++)
                for (int x = s.w0; x < s.w1; x++)
                {
                    plan.video_indices.push_back(sample_offset[s.sample_index] + (t * h + y) * wd + x);
                    std::array<int, 3> p = {{t - s.t0, y - s.h0, x - s.w0}};
                    plan.local_positions.push_back(p);
                }
    }
    if (static_cast<int>(plan.video_indices.size()) != tokens)
        return -2;
    plan.inverse_video_indices.assign(tokens, -1);
    for (int p = 0; p < tokens; p++)
    {
        const int src = plan.video_indices[p];
        if (src < 0 || src >= tokens || plan.inverse_video_indices[src] != -1)
            return -2;
        plan.inverse_video_indices[src] = p;
    }
    return 0;
}

AdaptiveWindowAttention::AdaptiveWindowAttention()
    : AdaptiveWindowAttention(0)
{
}

// Defaults of the reference constructor (:662-677).
AdaptiveWindowAttention::AdaptiveWindowAttention(AdaptiveWindowRuntimeState* new_runtime_state)
    : heads(20), head_dim(128), target_windows({{4, 3, 3}}), shifted(false),
      epsilon(1e-5f), rope_pairs_per_axis(21), shared_norm(false),
      shape_values_are_int32(false), official_bf16_attention(false),
      runtime_state(new_runtime_state), weights_dirty(true), plan(0), plan_rope_cached(false),
      qkv_projection(0)
{
    one_blob_only = false;
    support_inplace = false;
}

AdaptiveWindowAttention::~AdaptiveWindowAttention()
{
    std::lock_guard<std::mutex> lock(mutex);
    release_device_locked();
}

void AdaptiveWindowAttention::configure(int new_heads, int new_head_dim,
                                        const std::array<int, 3>& new_target_windows,
                                        bool new_shifted, float new_epsilon,
                                        int new_rope_pairs_per_axis,
                                        bool new_shape_values_are_int32,
                                        bool new_official_bf16_attention)
{
    std::lock_guard<std::mutex> lock(mutex);
    heads = new_heads;
    head_dim = new_head_dim;
    target_windows = new_target_windows;
    shifted = new_shifted;
    epsilon = new_epsilon;
    rope_pairs_per_axis = new_rope_pairs_per_axis;
    shape_values_are_int32 = new_shape_values_are_int32;
    official_bf16_attention = new_official_bf16_attention;
    release_device_locked();
}

// ParamDict ids and defaults of the reference load_param (:700-714).
int AdaptiveWindowAttention::load_param(const ncnn::ParamDict& pd)
{
    std::lock_guard<std::mutex> lock(mutex);
    heads = pd.get(0, 20);
    head_dim = pd.get(1, 128);
    target_windows[0] = pd.get(2, 4);
    target_windows[1] = pd.get(3, 3);
    target_windows[2] = pd.get(4, 3);
    shifted = pd.get(5, 0) != 0;
    epsilon = pd.get(6, 1e-5f);
    rope_pairs_per_axis = pd.get(7, 21);
    shared_norm = pd.get(8, 0) != 0;
    shape_values_are_int32 = pd.get(9, 0) != 0;
    official_bf16_attention = pd.get(10, 0) != 0;
    release_device_locked();
    return 0;
}

// Weight order of the reference load_model (:716-738): raw fp32 video_norm_q,
// video_norm_k, [text_norm_q, text_norm_k unless shared], rope_freqs.
int AdaptiveWindowAttention::load_model(const ncnn::ModelBin& mb)
{
    std::lock_guard<std::mutex> lock(mutex);
    weights_dirty = true;
    video_norm_q = mb.load(head_dim, 1);
    video_norm_k = mb.load(head_dim, 1);
    if (video_norm_q.empty() || video_norm_k.empty())
        return -100;

    if (shared_norm)
    {
        text_norm_q = video_norm_q;
        text_norm_k = video_norm_k;
    }
    else
    {
        text_norm_q = mb.load(head_dim, 1);
        text_norm_k = mb.load(head_dim, 1);
        if (text_norm_q.empty() || text_norm_k.empty())
            return -100;
    }

    rope_freqs = mb.load(rope_pairs_per_axis, 1);
    return rope_freqs.empty() ? -100 : 0;
}

int AdaptiveWindowAttention::set_weights(const std::vector<float>& new_video_norm_q,
                                         const std::vector<float>& new_video_norm_k,
                                         const std::vector<float>& new_text_norm_q,
                                         const std::vector<float>& new_text_norm_k,
                                         const std::vector<float>& new_rope_freqs)
{
    std::lock_guard<std::mutex> lock(mutex);
    weights_dirty = true;
    if (copy_vector(new_video_norm_q, head_dim, video_norm_q) != 0 ||
        copy_vector(new_video_norm_k, head_dim, video_norm_k) != 0 ||
        copy_vector(new_text_norm_q, head_dim, text_norm_q) != 0 ||
        copy_vector(new_text_norm_k, head_dim, text_norm_k) != 0 ||
        copy_vector(new_rope_freqs, rope_pairs_per_axis, rope_freqs) != 0)
        return -1;
    return 0;
}

void AdaptiveWindowAttention::set_runtime_shapes(
    const std::vector<std::array<int, 3> >& video_shapes,
    const std::vector<int>& text_lengths)
{
    owned_runtime_state.video_shapes = video_shapes;
    owned_runtime_state.text_lengths = text_lengths;
    runtime_state = &owned_runtime_state;
}

int AdaptiveWindowAttention::create_pipeline(const ncnn::Option& /*opt*/)
{
    return layer_status(create_pipeline_impl());
}

int AdaptiveWindowAttention::create_pipeline_impl()
{
    std::lock_guard<std::mutex> lock(mutex);
    // the host-blob path runs on the default stream: own its scratch
    const int sret = host_scratch.take(0);
    if (sret != S2_OK)
        return sret;
    int devices = 0;
    if (s2_device_count(&devices) != S2_OK || devices == 0)
        return 0;   // nothing to prepare without a device; forward reports it
    if (video_norm_q.empty() || rope_freqs.empty())
        return 0;   // configured through set_weights later
    return upload_weights_locked();
}

int AdaptiveWindowAttention::destroy_pipeline(const ncnn::Option& /*opt*/)
{
    std::lock_guard<std::mutex> lock(mutex);
    host_scratch.drop();
    release_device_locked();
    return 0;
}

void AdaptiveWindowAttention::release_device_locked() const
{
    if (plan)
        s2_awa_plan_destroy(plan);
    plan = 0;
    plan_rope_cached = false;
    plan_shapes.clear();
    plan_text_lengths.clear();
    workspace.release();
    staging.release();
    weights_gpu.release();
    weights_dirty = true;
}

// Device copy of the weights, packed as [video_q | video_k | text_q | text_k]
// (the reference upload_model packing, :1047-1053) followed by rope_freqs.
int AdaptiveWindowAttention::upload_weights_locked() const
{
    if (!weights_dirty && weights_gpu.get())
        return 0;
    const int d = head_dim;
    std::vector<float> host(4 * d + rope_pairs_per_axis);
    const ncnn::Mat* norms[4] = {&video_norm_q, &video_norm_k, &text_norm_q, &text_norm_k};
    for (int i = 0; i < 4; i++)
    {
        if (norms[i]->empty() || static_cast<int>(norms[i]->total()) < d)
            return -1;
        memcpy(&host[i * d], norms[i]->data, d * sizeof(float));
    }
    if (static_cast<int>(rope_freqs.total()) < rope_pairs_per_axis)
        return -1;
    memcpy(&host[4 * d], rope_freqs.data, rope_pairs_per_axis * sizeof(float));
    int ret = weights_gpu.reserve(host.size() * sizeof(float));
    if (ret != 0)
        return ret;
    ret = s2_memcpy_h2d(weights_gpu.get(), host.data(), host.size() * sizeof(float), 0);
    if (ret == 0)
        ret = s2_stream_synchronize(0);
    if (ret == 0)
        weights_dirty = false;
    plan_rope_cached = false;   // new frequencies (or a new buffer)
    return ret;
}

int AdaptiveWindowAttention::plan_for_locked(const std::vector<int>& shapes,
                                             const std::vector<int>& text_lengths) const
{
    if (plan && shapes == plan_shapes && text_lengths == plan_text_lengths)
        return 0;
    if (plan)
        s2_awa_plan_destroy(plan);
    plan = 0;
    plan_rope_cached = false;
    s2_awa_config config;
    config.heads = heads;
    config.head_dim = head_dim;
    config.target_windows[0] = target_windows[0];
    config.target_windows[1] = target_windows[1];
    config.target_windows[2] = target_windows[2];
    config.shifted = shifted ? 1 : 0;
    config.epsilon = epsilon;
    config.rope_pairs_per_axis = rope_pairs_per_axis;
    config.shared_norm = shared_norm ? 1 : 0;
    config.official_bf16_attention = official_bf16_attention ? 1 : 0;
    const int ret = s2_awa_plan_create(&config, shapes.data(), text_lengths.data(),
                                       static_cast<int>(text_lengths.size()), &plan);
    if (ret != 0)
        return ret;
    plan_shapes = shapes;
    plan_text_lengths = text_lengths;
    return 0;
}

int AdaptiveWindowAttention::set_qkv_projection(const SharedLinear* qkv)
{
    std::lock_guard<std::mutex> lock(mutex);
    if (qkv)
    {
        const int inner = heads * head_dim;
        if ((head_dim != 64 && head_dim != 128) || inner % 256 != 0 ||
            qkv->output_width() != 3 * inner || qkv->activation_kind() != S2_ACT_NONE ||
            qkv->input_width() <= 0 || qkv->input_width() % 64 != 0)
            return -1;
    }
    qkv_projection = qkv;
    return 0;
}

int AdaptiveWindowAttention::forward(const std::vector<ncnn::Mat>& bottom_blobs,
                                     std::vector<ncnn::Mat>& top_blobs,
                                     const ncnn::Option& opt) const
{
    return layer_status(forward_impl(bottom_blobs, top_blobs, opt));
}

int AdaptiveWindowAttention::forward_impl(const std::vector<ncnn::Mat>& bottom_blobs,
                                     std::vector<ncnn::Mat>& top_blobs,
                                     const ncnn::Option& opt) const
{
    std::lock_guard<std::mutex> lock(mutex);
    // Arity, configuration and weights (reference :768-772).
    const bool split_qkv = bottom_blobs.size() == 8;
    if ((!split_qkv && bottom_blobs.size() != 4) || top_blobs.size() != 2 || heads <= 0 || head_dim <= 0 ||
        rope_pairs_per_axis * 6 > head_dim || video_norm_q.empty() || video_norm_k.empty() ||
        text_norm_q.empty() || text_norm_k.empty() || rope_freqs.empty())
        return -1;

    const ncnn::Mat& video_qkv = bottom_blobs[0];
    const ncnn::Mat& text_qkv = bottom_blobs[split_qkv ? 3 : 1];
    const ncnn::Mat& video_shape_blob = bottom_blobs[split_qkv ? 6 : 2];
    const ncnn::Mat& text_length_blob = bottom_blobs[split_qkv ? 7 : 3];
    const int inner_dim = heads * head_dim;

    // Host blobs must be fp32 (as the reference CPU path); device blobs may
    // be fp32, bf16 or fp16 (device_blob_dtype) but must agree.
    HipDeviceAllocator* device = device_allocator_of(video_qkv);
    const size_t elemsize = video_qkv.elemsize;
    const int n_data = split_qkv ? 6 : 2;
    for (int part = 0; part < n_data; part++)
    {
        const ncnn::Mat& m = bottom_blobs[part];
        if ((device_allocator_of(m) != 0) != (device != 0) || m.elemsize != elemsize ||
            m.elempack != 1)
            return -1;
    }
    if (!device && elemsize != sizeof(float))
        return -1;
    if (device && elemsize != 4 && elemsize != 2)
        return -1;
    // fused QKV projection: the first two blobs are its device bf16 inputs
    const SharedLinear* qkv = split_qkv ? 0 : qkv_projection;
    if (qkv && (!device || elemsize != 2 || device_blob_dtype(elemsize, opt) != S2_DTYPE_BF16))
        return -1;
    const int in_width = qkv ? qkv->input_width() : inner_dim * 3;

    // Blob shapes (reference :783-797).
    if (split_qkv)
    {
        for (int part = 0; part < 6; part++)
        {
            if (bottom_blobs[part].dims != 2 || bottom_blobs[part].w != inner_dim)
                return -1;
        }
    }
    else if (video_qkv.dims != 2 || text_qkv.dims != 2 || video_qkv.w != in_width ||
             text_qkv.w != in_width)
        return -1;

    // Runtime shapes: from host shape blobs (reference :799-817), or from
    // the runtime state when no shape blob is given or they are device
    // blobs, which the host cannot read (the reference device path,
    // :1065-1067, 1090-1100).
    std::vector<int> shapes;
    std::vector<int> text_lengths;
    int expected_video_tokens = 0;
    int expected_text_tokens = 0;
    const bool host_shape_blobs = !device_allocator_of(video_shape_blob) &&
                                  !device_allocator_of(text_length_blob);
    if ((!video_shape_blob.empty() || !text_length_blob.empty()) && host_shape_blobs)
    {
        if (video_shape_blob.w != 3)
            return -1;
        const int batch = video_shape_blob.dims == 1 ? 1 : video_shape_blob.h;
        const int text_batch = text_length_blob.dims == 1 ? text_length_blob.w : text_length_blob.h;
        if (batch <= 0 || text_batch != batch)
            return -1;
        shapes.resize(3 * batch);
        text_lengths.resize(batch);
        for (int sample = 0; sample < batch; sample++)
        {
            for (int axis = 0; axis < 3; axis++)
                shapes[3 * sample + axis] =
                    read_shape_value(video_shape_blob, sample, axis, shape_values_are_int32);
            text_lengths[sample] = read_shape_value(text_length_blob, sample, 0, shape_values_are_int32);
        }
    }
    else
    {
        if (!runtime_state || runtime_state->video_shapes.empty() ||
            runtime_state->video_shapes.size() != runtime_state->text_lengths.size())
            return -1;
        for (size_t sample = 0; sample < runtime_state->video_shapes.size(); sample++)
        {
            for (int axis = 0; axis < 3; axis++)
                shapes.push_back(runtime_state->video_shapes[sample][axis]);
            text_lengths.push_back(runtime_state->text_lengths[sample]);
        }
    }
    for (size_t sample = 0; sample < text_lengths.size(); sample++)
    {
        if (text_lengths[sample] <= 0)
            return -1;
        expected_video_tokens += shapes[3 * sample] * shapes[3 * sample + 1] * shapes[3 * sample + 2];
        expected_text_tokens += text_lengths[sample];
    }
    // Token counts against the blobs (reference :818-831).
    if (split_qkv)
    {
        for (int part = 0; part < 3; part++)
        {
            if (bottom_blobs[part].h != expected_video_tokens ||
                bottom_blobs[part + 3].h != expected_text_tokens)
                return -1;
        }
    }
    else if (expected_video_tokens != video_qkv.h || expected_text_tokens != text_qkv.h)
        return -1;

    // The gfx950 kernels are specialised for these head sizes.
    if (head_dim != 64 && head_dim != 128)
        return -1;

    int devices = 0;
    if (s2_device_count(&devices) != S2_OK || devices == 0)
        return S2_ERR_DEVICE;

    int ret = plan_for_locked(shapes, text_lengths);
    if (ret != 0)
        return ret;
    ret = upload_weights_locked();
    if (ret != 0)
        return ret;
    if (!plan_rope_cached)
    {
        // the frequencies are weights: the plan keeps their cos/sin table
        // until the plan or the weights change
        ret = s2_awa_plan_cache_rope(plan, static_cast<const float*>(weights_gpu.get()) + 4 * head_dim, 0);
        if (ret == 0)
            ret = s2_stream_synchronize(0);
        if (ret != 0)
            return ret;
        plan_rope_cached = true;
    }
    s2_awa_plan_info info;
    s2_awa_plan_get_info(plan, &info);
    ret = workspace.reserve(info.workspace_bytes);
    if (ret != 0)
        return ret;

    const float* norms = static_cast<const float*>(weights_gpu.get());
    const float* freqs = norms + 4 * head_dim;
    const size_t lv = static_cast<size_t>(expected_video_tokens);
    const size_t lt = static_cast<size_t>(expected_text_tokens);

    if (device)
    {
        // Zero-copy: inputs and outputs stay in device memory.
        HipDeviceAllocator* out_alloc = dynamic_cast<HipDeviceAllocator*>(opt.blob_allocator);
        if (!out_alloc)
            out_alloc = device;
        top_blobs[0] = out_alloc->create_blob(inner_dim, expected_video_tokens, elemsize);
        top_blobs[1] = out_alloc->create_blob(inner_dim, expected_text_tokens, elemsize);
        if (top_blobs[0].empty() || top_blobs[1].empty())
            return -100;
        const unsigned char* v = static_cast<const unsigned char*>(video_qkv.data);
        const unsigned char* t = static_cast<const unsigned char*>(text_qkv.data);
        const void* vq = v;
        const void* vk = split_qkv ? bottom_blobs[1].data : v + inner_dim * elemsize;
        const void* vv = split_qkv ? bottom_blobs[2].data : v + 2 * inner_dim * elemsize;
        const void* tq = t;
        const void* tk = split_qkv ? bottom_blobs[4].data : t + inner_dim * elemsize;
        const void* tv = split_qkv ? bottom_blobs[5].data : t + 2 * inner_dim * elemsize;
        const long vstride = split_qkv ? inner_dim : 3 * inner_dim;
        const s2_dtype dtype = device_blob_dtype(elemsize, opt);
        if (qkv)
        {
            const uint16_t* w = 0;
            const float* b = 0;
            ret = qkv->device_weights(&w, &b);
            if (ret != 0)
                return ret;
            return s2_awa_qkv_forward(plan, video_qkv.data, text_qkv.data, in_width, w, b, norms, freqs,
                                      top_blobs[0].data, top_blobs[1].data, dtype, workspace.get(),
                                      workspace.size(), device->stream());
        }
        return s2_awa_forward(plan, norms, freqs, vq, vk, vv, vstride, tq, tk, tv, vstride, dtype,
                              top_blobs[0].data, top_blobs[1].data, dtype, workspace.get(),
                              workspace.size(), device->stream());
    }

    // Host fp32 blobs: stage inputs, compute, download, synchronise.
    const size_t vin = lv * (split_qkv ? inner_dim : 3 * inner_dim);
    const size_t tin = lt * (split_qkv ? inner_dim : 3 * inner_dim);
    const int parts = split_qkv ? 3 : 1;
    const size_t in_floats = parts * (vin + tin);
    const size_t out_floats = (lv + lt) * inner_dim;
    ret = staging.reserve((in_floats + out_floats) * sizeof(float));
    if (ret != 0)
        return ret;
    float* dev = static_cast<float*>(staging.get());
    float* dev_v[3];
    float* dev_t[3];
    for (int p = 0; p < parts; p++)
    {
        dev_v[p] = dev + p * vin;
        dev_t[p] = dev + parts * vin + p * tin;
        ret = s2_memcpy_h2d(dev_v[p], bottom_blobs[p].data, vin * sizeof(float), 0);
        if (ret == 0)
            ret = s2_memcpy_h2d(dev_t[p], bottom_blobs[split_qkv ? 3 + p : 1].data, tin * sizeof(float), 0);
        if (ret != 0)
            return ret;
    }
    float* dev_out_v = dev + in_floats;
    float* dev_out_t = dev_out_v + lv * inner_dim;
    const long stride = split_qkv ? inner_dim : 3 * inner_dim;
    const float* vq = dev_v[0];
    const float* vk = split_qkv ? dev_v[1] : dev_v[0] + inner_dim;
    const float* vv = split_qkv ? dev_v[2] : dev_v[0] + 2 * inner_dim;
    const float* tq = dev_t[0];
    const float* tk = split_qkv ? dev_t[1] : dev_t[0] + inner_dim;
    const float* tv = split_qkv ? dev_t[2] : dev_t[0] + 2 * inner_dim;
    ret = s2_awa_forward(plan, norms, freqs, vq, vk, vv, stride, tq, tk, tv, stride, S2_DTYPE_F32,
                         dev_out_v, dev_out_t, S2_DTYPE_F32, workspace.get(), workspace.size(), 0);
    if (ret != 0)
        return ret;

    ncnn::Mat& video_output = top_blobs[0];
    ncnn::Mat& text_output = top_blobs[1];
    video_output.create(inner_dim, expected_video_tokens, 4u, opt.blob_allocator);
    text_output.create(inner_dim, expected_text_tokens, 4u, opt.blob_allocator);
    if (video_output.empty() || text_output.empty())
        return -100;
    ret = s2_memcpy_d2h(video_output.data, dev_out_v, lv * inner_dim * sizeof(float), 0);
    if (ret == 0)
        ret = s2_memcpy_d2h(text_output.data, dev_out_t, lt * inner_dim * sizeof(float), 0);
    if (ret == 0)
        ret = s2_stream_synchronize(0);
    return ret;
}

ncnn::Layer* adaptive_window_attention_layer_creator(void* userdata)
{
    return new AdaptiveWindowAttention(static_cast<AdaptiveWindowRuntimeState*>(userdata));
}

void adaptive_window_attention_layer_destroyer(ncnn::Layer* layer, void* /*userdata*/)
{
    delete layer;
}

} // namespace seedvr2
