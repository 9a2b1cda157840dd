// Host launchers of the gfx950 kernels (awa_kernels.hip, linear_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "awa_plan.h"
#include "block_kernels.h"

// Activation element types (in_kind, out_kind, x_kind, y_kind) are the
// s2_dtype values: 0 fp32, 1 bf16, 2 fp16.
namespace s2 {

hipError_t launch_rope_table(const float* freqs, int pairs, int positions, float2* table,
                             hipStream_t stream);
hipError_t launch_awa_prologue(const s2_awa_plan& plan, const void* vq, const void* vk,
                               const void* vv, long vstride, const void* tq, const void* tk,
                               const void* tv, long tstride, int in_kind, const float* norm,
                               const float2* rope, uint16_t* q_out, uint16_t* k_out,
                               uint16_t* vt_out, hipStream_t stream);
hipError_t launch_awa_attention(const s2_awa_plan& plan, const uint16_t* q, const uint16_t* k,
                                const uint16_t* vt, void* out_video, int out_kind,
                                float* text_partial, const float* norm, hipStream_t stream);
hipError_t launch_awa_text_pool(const s2_awa_plan& plan, const float* partial, void* out_text,
                                int out_kind, hipStream_t stream);
hipError_t launch_awa_plan_tables(const s2_awa_plan& plan, int* indices, int* inverse,
                                  int* positions, hipStream_t stream);

// The fused QKV projection + attention prologue (x [L][k] bf16, W [3 inner][k]):
// writes the plan's Q, K and V^T workspace, text tokens to their staging rows.
hipError_t launch_awa_qkv(const s2_awa_plan& plan, const uint16_t* x_video, const uint16_t* x_text,
                          int k, const uint16_t* w, const float* bias, const float* norm,
                          const float2* rope, uint16_t* q, uint16_t* kk, uint16_t* vt,
                          hipStream_t stream);

hipError_t launch_cast_f32_bf16(const float* src, uint16_t* dst, size_t n, hipStream_t stream);
hipError_t launch_gelu(const void* x, void* y, size_t n, int kind, hipStream_t stream);
hipError_t launch_cast_bf16_f32(const uint16_t* src, float* dst, size_t n, hipStream_t stream);
// Grouped y_s = act(x_s W^T + b) over the video and text streams.
hipError_t launch_shared_linear(const void* x0, int m0, const void* x1, int m1, int x_kind,
                                const uint16_t* w, const float* bias, int n, int k, int act,
                                void* y0, void* y1, int y_kind, hipStream_t stream);
// The same with the split-k scratch in a static device array: no allocation.
hipError_t launch_shared_linear_noalloc(const void* x0, int m0, const void* x1, int m1,
                                        int x_kind, const uint16_t* w, const float* bias, int n,
                                        int k, int act, void* y0, void* y1, int y_kind,
                                        hipStream_t stream);

// The DiT block's gated residual sum in the epilogue of the projection that
// feeds it (the attention's out projection, the MLP's down projection):
// out = x + y * (gate[sample] + gate_s), y the projection rounded to bf16 (the
// value a bf16 output blob holds), out in the element type of x, as
// launch_ada_out computes it from that blob.  Rows have pitch n; a row's
// sample comes from the cumulative row ends of its stream.
struct LinearResidual {
    const void* x[2];          // residual rows of the video / text stream
    void* out[2];              // output rows (may be x)
    int x_kind;                // residual and out element type
    const float* gate;         // [batch][n]
    const float* gate_s[2];    // the stream's own [n] vector, or null
    AdaRows rows;
};
// y = x W^T + b over the two streams (bf16 activations, k % 64 == 0,
// n % 8 == 0) with the residual epilogue in place of the y stores.
hipError_t launch_shared_linear_residual(const uint16_t* x0, int m0, const uint16_t* x1, int m1,
                                         const uint16_t* w, const float* bias, int n, int k,
                                         const LinearResidual& res, hipStream_t stream);

}  // namespace s2
