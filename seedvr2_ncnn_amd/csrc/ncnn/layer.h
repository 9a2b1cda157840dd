// ncnn-compatible subset: Layer (see allocator.h for the scope of this directory).
//
// The CPU-surface virtuals of ncnn::Layer.  The Vulkan virtuals
// (upload_model, forward(VkMat...)) are absent: the MI355X layers run their
// device work from forward(Mat...) through the HIP C-ABI.
#ifndef NCNN_LAYER_H
#define NCNN_LAYER_H

#include <string>
#include <vector>

#include "mat.h"
#include "modelbin.h"
#include "option.h"
#include "paramdict.h"

#ifndef NCNN_VULKAN
#define NCNN_VULKAN 0
#endif

namespace ncnn {

class Layer {
public:
    Layer();
    virtual ~Layer();

    virtual int load_param(const ParamDict& pd);
    virtual int load_model(const ModelBin& mb);
    virtual int create_pipeline(const Option& opt);
    virtual int destroy_pipeline(const Option& opt);

    virtual int forward(const std::vector<Mat>& bottom_blobs, std::vector<Mat>& top_blobs,
                        const Option& opt) const;
    virtual int forward(const Mat& bottom_blob, Mat& top_blob, const Option& opt) const;
    virtual int forward_inplace(std::vector<Mat>& bottom_top_blobs, const Option& opt) const;
    virtual int forward_inplace(Mat& bottom_top_blob, const Option& opt) const;

    bool one_blob_only;
    bool support_inplace;
    bool support_vulkan;
    bool support_packing;
    bool support_bf16_storage;
    bool support_fp16_storage;
    bool support_int8_storage;
    bool support_vulkan_packing;
    bool support_vulkan_any_packing;

    void* userdata;
    int typeindex;
    std::string type;
    std::string name;
    std::vector<int> bottoms;
    std::vector<int> tops;
    std::vector<Mat> bottom_shapes;
    std::vector<Mat> top_shapes;
};

typedef Layer* (*layer_creator_func)(void*);
typedef void (*layer_destroyer_func)(Layer*, void*);

}  // namespace ncnn

#endif  // NCNN_LAYER_H
