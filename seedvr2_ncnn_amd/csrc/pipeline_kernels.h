// Host launchers of the DiT frontend/tail and sampler-step kernels
// (pipeline_kernels.hip).  All tensors are fp32 device memory; a video
// sample is a frames x height x width token grid with even height and width.
// Every launcher checks only what its kernels need to stay in bounds (sizes
// that fit the 32-bit in-row indexing); shape validation is the caller's.
#pragma once

#include <hip/hip_runtime.h>

namespace s2 {

// [frames*height*width][33] tokens -> [frames*(height/2)*(width/2)][132]
// patches (tokens and patches 8-byte aligned)
hipError_t launch_patchify(const float* tokens, int frames, int height, int width, float* patches,
                           hipStream_t stream);
// channel-planar latent and condition (16 planes each, plane stride
// `channel_stride` floats) -> the patches of the tokens [latent | condition | 1]
hipError_t launch_latent_patches(const float* latent, const float* condition, long channel_stride,
                                 int frames, int height, int width, float* patches,
                                 hipStream_t stream);
// [patches][64] -> [frames*height*width][16] (both 16-byte aligned)
hipError_t launch_unpatchify(const float* patches, int frames, int height, int width,
                             float* tokens, hipStream_t stream);
// `count` host timesteps -> [count][256] sinusoidal embedding
hipError_t launch_timestep_embedding(const float* timesteps, int count, float* embedding,
                                     hipStream_t stream);
// out = neg + scale (pos - neg) over `count` floats; when rescale != 0 and
// count >= 2, out is then multiplied by the std-ratio factor (16-byte aligned
// operands)
hipError_t launch_cfg(const float* pos, const float* neg, long count, float scale, float rescale,
                      float* out, hipStream_t stream);
// latent[c][t] += delta * prediction[t][c] for c < 16, t < tokens
// (prediction 16-byte aligned)
hipError_t launch_euler(float* latent, long channel_stride, const float* prediction, long tokens,
                        float delta, hipStream_t stream);
// One sampler update of one sample straight from its patchified predictions
// ([patches][64], 16-byte aligned): g = pos when neg is null, else
// neg + scale (pos - neg) with the std-ratio rescale of launch_cfg; then
// latent[c][token] += delta * g at the unpatchified token position.
hipError_t launch_denoise_update(const float* pos_patches, const float* neg_patches, int frames,
                                 int height, int width, float scale, float rescale, float delta,
                                 float* latent, long channel_stride, hipStream_t stream);

}  // namespace s2
