// SharedLinear: one linear projection applied to the video and the text token
// streams, as an ncnn custom layer whose forward runs on an MI355X through the
// HIP C-ABI (include/seedvr2_hip.h).
//
// Drop-in surface of the reference layer (src/seedvr2/shared_linear.h:12-48):
// ParamDict ids 0 num_output, 1 num_input, 2 bias_term; raw fp32 weight
// [num_output][num_input] then bias [num_output]; forward takes 2 blobs and
// gives 2.  Both streams run in one grouped MFMA launch that shares the
// resident bf16 weight.  ParamDict id 3 (activation: 0 none, 1 erf-GELU,
// applied after the bias) is an extension of this build: the reference
// leaves activations to separate graph layers.
#ifndef SEEDVR2_SHARED_LINEAR_H
#define SEEDVR2_SHARED_LINEAR_H

#include <mutex>
#include <vector>

#include <layer.h>

#include "hip_allocator.h"

namespace seedvr2 {

class SharedLinear : public ncnn::Layer
{
public:
    SharedLinear();
    virtual ~SharedLinear();

    virtual int load_param(const ncnn::ParamDict& pd);
    virtual int load_model(const ncnn::ModelBin& mb);
    virtual int create_pipeline(const ncnn::Option& opt);
    virtual int destroy_pipeline(const ncnn::Option& opt);
    // Host fp32 blobs give host fp32 outputs; device blobs (HipDeviceAllocator,
    // fp32 or bf16) give device outputs of the same element size.
    virtual int forward(const std::vector<ncnn::Mat>& bottom_blobs,
                        std::vector<ncnn::Mat>& top_blobs,
                        const ncnn::Option& opt) const;

    // Epilogue activation, switched by a graph optimiser that folds a
    // following GELU layer: S2_ACT_GELU on a layer without one (param 3 = 0),
    // or the activation the layer already has.  Returns 0, or -1 for any
    // other change (a GELU or SwiGLU epilogue loaded from param 3 is kept).
    int set_activation(int act);

    // For a graph optimiser that fuses this projection into the attention
    // layer consuming it: the widths, the activation, and the device copy of
    // the weights (bf16 [N][K], uploaded first if needed) and bias (fp32 [N],
    // or null without a bias term).  device_weights returns 0 or an error code.
    int input_width() const { return num_input; }
    int output_width() const { return num_output; }
    int activation_kind() const { return activation; }
    int device_weights(const uint16_t** weight, const float** bias) const;

    // A new projection whose outputs are these projections' outputs side by
    // side (their [N][K] weight rows stacked in order; zero bias rows for a
    // part without a bias term), for graph folds: the q, k and v projections
    // of split graphs (activation S2_ACT_NONE), or a gate and an up
    // projection (S2_ACT_SWIGLU, exactly two parts of one width).  The parts
    // must share num_input, carry no activation and hold their weights.
    // Null when they do not, or when the result breaks load_param's rules.
    static SharedLinear* stack(const std::vector<const SharedLinear*>& parts, int activation);

private:
    // forward and create_pipeline without the mapping of C-ABI codes to the
    // reference's (layer_status)
    int forward_impl(const std::vector<ncnn::Mat>& bottom_blobs, std::vector<ncnn::Mat>& top_blobs,
                     const ncnn::Option& opt) const;
    int create_pipeline_impl();
    int upload_weights_locked() const;

    int num_output;
    int num_input;
    bool bias_term;
    int activation;
    bool params_loaded;
    ncnn::Mat weight_data;
    ncnn::Mat bias_data;

    mutable std::mutex mutex;
    StreamScratchRef host_scratch;   // the default stream's kernel scratch
    mutable bool weights_dirty;
    mutable DeviceBuffer weight_gpu;   // bf16 [N][K]
    mutable DeviceBuffer bias_gpu;     // fp32 [N]
    mutable DeviceBuffer staging;
};

ncnn::Layer* shared_linear_layer_creator(void* userdata);
void shared_linear_layer_destroyer(ncnn::Layer* layer, void* userdata);

} // namespace seedvr2

#endif // SEEDVR2_SHARED_LINEAR_H
