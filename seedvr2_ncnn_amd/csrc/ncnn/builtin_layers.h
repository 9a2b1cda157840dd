// ncnn-compatible subset: the built-in layers that exported SeedVR2 graphs
// use around the custom layers, beyond Input / Split / GELU (net.cpp).
//
//   MemoryData  Gemm  BinaryOp  UnaryOp  Sigmoid  Swish  Reduction  RMSNorm
//   Reshape  Slice  Concat  Crop
//
// Each keeps ncnn's ParamDict ids, defaults and .bin weight layout, and works
// on blobs of dims 1 and 2 (a 2-D blob is h rows of w elements; a 1-D blob of
// w elements broadcasts as one row, numpy-style).  Host blobs are fp32 and
// computed on the CPU; device blobs (HipDeviceAllocator) of fp32, bf16 or
// fp16 run the gfx950 kernels of the C-ABI on the blob's allocator's stream,
// outputs in the element type of the operand that has the output's shape.
// Return codes are ncnn's: 0, -1 (bad parameter, shape or a form this build
// does not run), -100 (allocation).
//
// Not run here (load_param returns -1): Reduction without reduce_all and
// with the legacy axis numbering (param 5 fixbug0 = 0); Gemm with a constant
// A, transposed A or output, two input blobs, or (on the device) alpha != 1;
// Crop with a reference blob; blobs of more than two dimensions.
#ifndef NCNN_BUILTIN_LAYERS_H
#define NCNN_BUILTIN_LAYERS_H

#include <string>

#include "layer.h"

namespace ncnn {

// A new built-in layer of the given type, or null when there is none.
Layer* create_builtin_layer(const std::string& type);

// For graph rewrites: the data of a MemoryData layer (host fp32), or null
// when the layer is not one.
const Mat* memory_data_of(const Layer* layer);

// For graph rewrites: BinaryOp's op type, with_scalar and scalar b, or -1
// when the layer is not a BinaryOp.
int binary_op_of(const Layer* layer, int* with_scalar, float* b);

// UnaryOp's op type, or -1 when the layer is not a UnaryOp.
int unary_op_of(const Layer* layer);

// Reduction: operation, reduce_all, coeff, keepdims and whether the axes
// select the last axis only (of any blob of dims 1 or 2); -1 otherwise.
int reduction_of(const Layer* layer, int* reduce_all, float* coeff, int* keepdims,
                 bool* last_axis_only);

// RMSNorm: eps and affine; -1 when the layer is not an RMSNorm.
int rms_norm_of(const Layer* layer, float* eps, int* affine);

}  // namespace ncnn

#endif  // NCNN_BUILTIN_LAYERS_H
