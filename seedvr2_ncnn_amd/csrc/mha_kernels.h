// Host launchers of the VAEChunkedMHA kernels (mha_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace s2 {

// rows of x (element type kind: 0 fp32, 1 bf16, 2 fp16; row width qdim) ->
// bf16 xp [rows_padded][qdim], zero rows from `rows` on
hipError_t launch_mha_stage(const void* x, int kind, int rows, int rows_padded, int qdim,
                            uint16_t* xp, hipStream_t stream);
// out[i] = bf16(w[i] * scale), i < n
hipError_t launch_mha_weight(const float* w, long n, float scale, uint16_t* out,
                             hipStream_t stream);
// out[i] = b[i] * scale, i < n
hipError_t launch_mha_bias(const float* b, int n, float scale, float* out, hipStream_t stream);
// P[r][c] = softmax over c < cols of S[r] (row stride ld_s), bf16, row
// stride ld_p, zero for cols <= c < ld_p
hipError_t launch_mha_softmax(const float* s, long ld_s, int rows, int cols, int ld_p,
                              uint16_t* p, hipStream_t stream);
// oh [rows][d] -> columns [h*d, (h+1)*d) of o [rows][embed]
hipError_t launch_mha_interleave(const uint16_t* oh, int rows, int d, int embed, int h,
                                 uint16_t* o, hipStream_t stream);

}  // namespace s2
