// AdaptiveWindowAttention: SeedVR2's DiT window attention as an ncnn custom
// layer whose forward runs on an MI355X through the HIP C-ABI
// (include/seedvr2_hip.h).
//
// Drop-in surface of the reference layer (src/seedvr2/adaptive_window_attention.h:14-120):
// same types (WindowSlice, AdaptiveWindowPlan, AdaptiveWindowRuntimeState),
// the same build_adaptive_window_plan, the same ParamDict ids and load_model
// weight order, the same forward(std::vector<Mat>...) blob contract and
// return codes, the same creator taking an AdaptiveWindowRuntimeState*, and
// the same test helpers (configure, set_weights, set_runtime_shapes).  The
// Vulkan virtuals are replaced by create_pipeline/destroy_pipeline owning
// the HIP resources.
#ifndef SEEDVR2_ADAPTIVE_WINDOW_ATTENTION_H
#define SEEDVR2_ADAPTIVE_WINDOW_ATTENTION_H

#include <array>
#include <mutex>
#include <vector>

#include <layer.h>

#include "hip_allocator.h"
#include "shared_linear.h"

struct s2_awa_plan;

namespace seedvr2 {

struct WindowSlice
{
    int sample_index;
    int t0;
    int t1;
    int h0;
    int h1;
    int w0;
    int w1;
    int partition_offset;
    int token_count;
};

struct AdaptiveWindowPlan
{
    std::vector<WindowSlice> windows;
    std::vector<int> sample_window_count;
    std::vector<int> video_indices;
    std::vector<int> inverse_video_indices;
    std::vector<std::array<int, 3> > local_positions;
};

struct AdaptiveWindowRuntimeState
{
    std::vector<std::array<int, 3> > video_shapes;
    std::vector<int> text_lengths;
};

// SeedVR2's 720p adaptive window construction; the window tuple is a target
// number of windows, not a fixed token extent.  Returns 0, -1 or -2.
int build_adaptive_window_plan(const std::vector<std::array<int, 3> >& video_shapes,
                               const std::array<int, 3>& target_windows,
                               bool shifted,
                               AdaptiveWindowPlan& plan);

class AdaptiveWindowAttention : public ncnn::Layer
{
public:
    AdaptiveWindowAttention();
    explicit AdaptiveWindowAttention(AdaptiveWindowRuntimeState* runtime_state);
    virtual ~AdaptiveWindowAttention();

    virtual int load_param(const ncnn::ParamDict& pd);
    virtual int load_model(const ncnn::ModelBin& mb);
    virtual int create_pipeline(const ncnn::Option& opt);
    virtual int destroy_pipeline(const ncnn::Option& opt);

    // Blobs as the reference: 4 inputs (video_qkv, text_qkv, video_shape,
    // text_length) or 8 (video q,k,v, text q,k,v, shapes); 2 outputs.  Host
    // fp32 blobs give host fp32 outputs.  Device blobs (HipDeviceAllocator,
    // fp32 or bf16) give device outputs of the same element size, allocated
    // from opt.blob_allocator when it is a HipDeviceAllocator, else from the
    // inputs' allocator.  Shapes come from the shape blobs (host Mats); when
    // those are empty the runtime state's shapes are used, as on the
    // reference's device path.
    virtual int forward(const std::vector<ncnn::Mat>& bottom_blobs,
                        std::vector<ncnn::Mat>& top_blobs,
                        const ncnn::Option& opt) const;

    // Test/runtime setup helper. Exported NCNN models use load_param/load_model.
    void configure(int heads, int head_dim, const std::array<int, 3>& target_windows,
                   bool shifted, float epsilon, int rope_pairs_per_axis,
                   bool shape_values_are_int32 = false,
                   bool official_bf16_attention = false);
    int set_weights(const std::vector<float>& video_norm_q,
                    const std::vector<float>& video_norm_k,
                    const std::vector<float>& text_norm_q,
                    const std::vector<float>& text_norm_k,
                    const std::vector<float>& rope_freqs);
    void set_runtime_shapes(const std::vector<std::array<int, 3> >& video_shapes,
                            const std::vector<int>& text_lengths);

    // Fused QKV projection (s2_awa_qkv_forward), set by a graph optimiser:
    // the 4-input form's first two blobs are then the projection's inputs
    // (width qkv->input_width(), device bf16), and `qkv` supplies the
    // weights.  Requires a bias-free or biased SharedLinear of width
    // 3 * heads * head_dim without activation, head_dim 64 or 128,
    // heads * head_dim a multiple of 256 and an input width that is a
    // multiple of 64; returns -1 otherwise.  nullptr undoes it.
    int set_qkv_projection(const SharedLinear* qkv);

private:
    // forward and create_pipeline without the mapping of C-ABI codes to the
    // reference's (layer_status)
    int forward_impl(const std::vector<ncnn::Mat>& bottom_blobs, std::vector<ncnn::Mat>& top_blobs,
                     const ncnn::Option& opt) const;
    int create_pipeline_impl();
    int upload_weights_locked() const;
    int plan_for_locked(const std::vector<int>& shapes, const std::vector<int>& text_lengths) const;
    void release_device_locked() const;

    int heads;
    int head_dim;
    std::array<int, 3> target_windows;
    bool shifted;
    float epsilon;
    int rope_pairs_per_axis;
    bool shared_norm;
    bool shape_values_are_int32;
    bool official_bf16_attention;

    ncnn::Mat video_norm_q;
    ncnn::Mat video_norm_k;
    ncnn::Mat text_norm_q;
    ncnn::Mat text_norm_k;
    ncnn::Mat rope_freqs;

    AdaptiveWindowRuntimeState owned_runtime_state;
    AdaptiveWindowRuntimeState* runtime_state;

    // Device state (guarded by mutex; forward is const and may be called
    // from several threads).
    mutable std::mutex mutex;
    StreamScratchRef host_scratch;   // the default stream's kernel scratch
    mutable bool weights_dirty;
    mutable DeviceBuffer weights_gpu;      // [4][d] norms then [P] freqs, fp32
    mutable s2_awa_plan* plan;
    mutable bool plan_rope_cached;         // the plan holds the table of weights_gpu's freqs
    const SharedLinear* qkv_projection;    // fused QKV projection, or null
    mutable std::vector<int> plan_shapes;
    mutable std::vector<int> plan_text_lengths;
    mutable DeviceBuffer workspace;
    mutable DeviceBuffer staging;
};

ncnn::Layer* adaptive_window_attention_layer_creator(void* userdata);
void adaptive_window_attention_layer_destroyer(ncnn::Layer* layer, void* userdata);

} // namespace seedvr2

#endif // SEEDVR2_ADAPTIVE_WINDOW_ATTENTION_H
