// ncnn-compatible subset: Option (see allocator.h for the scope of this directory).
#ifndef NCNN_OPTION_H
#define NCNN_OPTION_H

#include "allocator.h"

namespace ncnn {

class Option {
public:
    Option();

    bool lightmode;
    int num_threads;
    Allocator* blob_allocator;
    Allocator* workspace_allocator;
    bool use_vulkan_compute;
    bool use_fp16_packed;
    bool use_fp16_storage;
    bool use_fp16_arithmetic;
    bool use_bf16_packed;
    bool use_bf16_storage;
    bool use_packing_layout;
    bool use_cooperative_matrix;
    bool use_shader_local_memory;
    bool use_subgroup_ops;
};

}  // namespace ncnn

#endif  // NCNN_OPTION_H
