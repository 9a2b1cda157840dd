// ncnn-compatible subset: Layer defaults (see allocator.h for the scope of this directory).
#include "layer.h"

namespace ncnn {

Layer::Layer()
    : one_blob_only(false), support_inplace(false), support_vulkan(false), support_packing(false),
      support_bf16_storage(false), support_fp16_storage(false), support_int8_storage(false),
      support_vulkan_packing(false), support_vulkan_any_packing(false), userdata(0),
      typeindex(-1) {}

Layer::~Layer() {}

int Layer::load_param(const ParamDict&) { return 0; }
int Layer::load_model(const ModelBin&) { return 0; }
int Layer::create_pipeline(const Option&) { return 0; }
int Layer::destroy_pipeline(const Option&) { return 0; }

// Default forwards follow ncnn: the multi-blob form falls back to the
// in-place form on a copy of the inputs when the layer supports it.
int Layer::forward(const std::vector<Mat>& bottom_blobs, std::vector<Mat>& top_blobs,
                   const Option& opt) const {
    if (!support_inplace) return -1;
    top_blobs = bottom_blobs;
    for (size_t i = 0; i < top_blobs.size(); i++) {
        top_blobs[i] = bottom_blobs[i].clone(opt.blob_allocator);
        if (top_blobs[i].empty()) return -100;
    }
    return forward_inplace(top_blobs, opt);
}

int Layer::forward(const Mat& bottom_blob, Mat& top_blob, const Option& opt) const {
    if (!support_inplace) return -1;
    top_blob = bottom_blob.clone(opt.blob_allocator);
    if (top_blob.empty()) return -100;
    return forward_inplace(top_blob, opt);
}

int Layer::forward_inplace(std::vector<Mat>&, const Option&) const { return -1; }
int Layer::forward_inplace(Mat&, const Option&) const { return -1; }

}  // namespace ncnn
