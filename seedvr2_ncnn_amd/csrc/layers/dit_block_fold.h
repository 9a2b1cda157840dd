// Graph fold: the DiT block's norm, AdaSingle modulation and gated residual
// written with ncnn built-ins become fused passes (DiTStreamOp over the
// s2_dit_ada_* kernels), one per token stream.
//
// The exported block graph (src/seedvr2/seedvr2_dit.cpp:603-633) holds these
// operations as built-in layers between the six per-sample modulation inputs
// in4..in9 and the custom layers.  The chains folded, per stream:
//
//   ada_in      h = add(mul(norm(x), S), T)
//   ada_out     out = add(x, mul(y, G))
//   ada_out_in  an ada_out whose output (through Splits) is an ada_in's x
//
// norm(x) is an RMSNorm layer without affine, or x * rsqrt(mean(square(x),
// last axis, keepdims) + eps) as UnaryOp / Reduction / BinaryOp layers;
// S, T and G are graph inputs without a token stream (in4..in9, through
// Splits), or such an input plus a MemoryData [hidden] vector of the block.
// Operands may come in either order.  The token stream of a blob is traced
// from in0 (video) and in1 (text) through the layers.  Unlike the built-in
// chain, whose BinaryOp broadcast can only spread one [1][hidden] row over
// all rows (one sample), the fused passes take each row's sample from the
// runtime state, so a folded graph runs any batch.  Folded layers stop
// running; their intermediate blobs can no longer be extracted.
#ifndef SEEDVR2_DIT_BLOCK_FOLD_H
#define SEEDVR2_DIT_BLOCK_FOLD_H

#include <net.h>

#include "adaptive_window_attention.h"

namespace seedvr2 {

// Call after load_model.  Returns the number of fused passes made.
int fold_dit_modulation(ncnn::Net& net, const AdaptiveWindowRuntimeState* state);

}  // namespace seedvr2

#endif  // SEEDVR2_DIT_BLOCK_FOLD_H
