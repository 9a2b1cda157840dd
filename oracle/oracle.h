/*
 * CPU oracle for the SeedVR2 window-attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * layers' CPU forward (Chisato623/seedvr2_ncnn), the reference result of the
 * test suite and of __graft_entry__.smoke(), and bench.py's cpu_baseline leg.
 * Nothing in the product path (seedvr2_ncnn_amd/) may link, load or call it.
 *
 * Every function names the reference file:line it restates.  Floating-point
 * work is fp32 with the reference's operation order where the reference
 * states one; SDPA and Gemm live in the (absent) ncnn library and are
 * restated as textbook fp32 kernels.
 *
 * Pinning (how each function is checked independently of this file):
 *   orc_plan_*        closed-form window counts/extents at the benchmark shapes,
 *                     permutation invariants, brute force against an exact
 *                     rational-arithmetic plan written in the tests.
 *   orc_round_bf16    torch bfloat16 RNE conversion; tie, Inf and NaN cases.
 *   orc_rms_norm      unit-RMS rows at weight 1; float64 numpy closed form.
 *   orc_apply_mm_rope identity at freq 0 / position 0; complex rotation.
 *   orc_sdpa          torch scaled_dot_product_attention in float64;
 *                     constant-K -> mean(V); one-hot logits.
 *   orc_linear        torch matmul in float64; GELU vs torch erf-GELU.
 *   orc_awa_forward   an independent torch float64 implementation of the
 *                     layer semantics; single-window pooling identity.
 *   orc_patchify_video, orc_unpatchify_prediction
 *                     numpy reshape/transpose of the (t, h, w) grids;
 *                     unpatchify of a patchified grid returns its tokens.
 *   orc_timestep_embedding  float64 closed form; t = 0 gives sin 0, cos 1.
 *   orc_apply_cfg     without rescale bit-exact against numpy fp32 (each
 *                     operation rounded); with it, the float64 numpy closed
 *                     form; scale 0 gives neg; zero spread keeps the
 *                     unrescaled result.
 *   orc_euler_step    numpy closed form with a strided channel layout.
 *   orc_video_tokens  numpy transpose of the channel planes.
 *   orc_mha           torch float64 multi_head_attention_forward (self
 *                     attention, default and explicit scale); a subset of
 *                     query rows equals the same rows of the full run.
 *   orc_vae_pixel_shuffle  torch reshape/permute (depth-to-space over time
 *                     and space) with the head-frame removal.
 *   orc_ada_in        torch float64 rms_norm; unit-RMS rows at scale 1 and
 *                     shift 0; invariance under scaling of a row (eps 0);
 *                     per-sample constants identify each row's sample.
 *   orc_ada_out       gate 0 leaves the stream bit-exact; gate 1 adds y
 *                     bit-exact; per-sample constants identify each row's
 *                     sample.
 *   orc_decomposed_conv3d  torch float64 conv3d over the temporally padded
 *                     input (frame 0 replicated head_frames times); a run
 *                     split into slices chained through the memory equals
 *                     the unsplit run; a 1x1x1 kernel is a per-pixel matmul.
 */
#ifndef SEEDVR2_ORACLE_H
#define SEEDVR2_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same fields as the reference WindowSlice (adaptive_window_attention.h:16-27). */
typedef struct orc_slice {
    int sample_index;
    int t0, t1, h0, h1, w0, w1;
    int partition_offset;
    int token_count;
} orc_slice;

/* Layer configuration: the reference ParamDict ids 0..10
 * (adaptive_window_attention.cpp:700-714). */
typedef struct orc_awa_params {
    int heads;                    /* id 0 */
    int head_dim;                 /* id 1 */
    int target_windows[3];        /* ids 2,3,4 */
    int shifted;                  /* id 5 */
    float epsilon;                /* id 6 */
    int rope_pairs_per_axis;      /* id 7 */
    int official_bf16_attention;  /* id 10 */
} orc_awa_params;

/* Number of windows and video tokens a plan will hold (walks the same loops
 * as orc_plan_build without storing anything).  Returns 0 or -1. */
int orc_plan_count(const int* video_shapes, int batch, const int target_windows[3],
                   int shifted, int* num_windows, int* total_tokens);

/* build_adaptive_window_plan (adaptive_window_attention.cpp:565-655).
 * video_shapes: [batch][3] (t,h,w).  Output arrays are sized by orc_plan_count:
 * windows[num_windows], sample_window_count[batch], video_indices[L],
 * inverse_video_indices[L], local_positions[L][3].  Any output may be NULL.
 * Returns 0, -1 (bad shape) or -2 (not a permutation). */
int orc_plan_build(const int* video_shapes, int batch, const int target_windows[3],
                   int shifted, orc_slice* windows, int max_windows,
                   int* sample_window_count, int* video_indices,
                   int* inverse_video_indices, int* local_positions);

/* round_bf16 (adaptive_window_attention.cpp:499-508). */
float orc_round_bf16(float value);
/* Elementwise round_bf16 over an array (bit patterns pass through untouched). */
void orc_round_bf16_array(const float* in, float* out, long count);

/* rms_norm (adaptive_window_attention.cpp:510-519). */
void orc_rms_norm(const float* input, const float* weight, int size, float epsilon,
                  float* output);

/* apply_mm_rope (adaptive_window_attention.cpp:521-543). */
void orc_apply_mm_rope(float* values, int head_dim, const float* freqs,
                       int pairs_per_axis, const int position[3]);

/* Textbook SDPA standing in for ncnn SDPA with params {5:0, 6:0.f, 7:0}
 * (adaptive_window_attention.cpp:847-861, 943): per head,
 * softmax(Q K^T / sqrt(d)) V, unmasked.  q,k,v,out: [heads][seq][d] fp32. */
void orc_sdpa(const float* q, const float* k, const float* v, int heads, int seq,
              int head_dim, float* out, int num_threads);

/* AdaptiveWindowAttention::forward (adaptive_window_attention.cpp:764-978).
 * Video rows have stride video_stride floats and hold q at +0, k at +inner
 * (fused form) or come from separate pointers (split form): the caller passes
 * the three base pointers either way.  Outputs are fp32 [Lv][inner] and
 * [Lt][inner], zero-filled here.  window_subset (optional) restricts the
 * computation to those plan windows; text output is then partial.
 * Returns the reference's codes (0, -1, -2, -100). */
int orc_awa_forward(const orc_awa_params* params,
                    const float* video_norm_q, const float* video_norm_k,
                    const float* text_norm_q, const float* text_norm_k,
                    const float* rope_freqs,
                    const int* video_shapes, const int* text_lengths, int batch,
                    const float* video_q, const float* video_k, const float* video_v,
                    long video_stride,
                    const float* text_q, const float* text_k, const float* text_v,
                    long text_stride,
                    float* out_video, float* out_text,
                    const int* window_subset, int num_subset, int num_threads);

/* SharedLinear / ncnn Gemm restated (shared_linear.cpp:27-96):
 * Y[m][n] = sum_k X[m][k] * W[n][k] + b[n], fp32; activation 1 applies
 * erf-GELU after the bias.  rows: optional list of rows of X to compute
 * (num_rows of them, Y then holds num_rows rows in that order). */
void orc_linear(const float* x, int m, int k, const float* w, const float* bias, int n,
                int activation, float* y, const int* rows, int num_rows, int num_threads);

/* ---- DiT frontend and tail (the steps either side of the block stack) ---- */

/* patchify_video (seedvr2_dit.cpp:167-230): source [tokens][33] of samples
 * with video shapes (t, h, w), h and w even, -> destination
 * [sum t*(h/2)*(w/2)][132]; patch (f, py, px) holds the 2x2 tokens
 * (f, 2py+y, 2px+x) at feature offset (2y+x)*33.  Returns 0 or -1. */
int orc_patchify_video(const float* source, long tokens, const int* shapes, int batch,
                       float* destination);

/* make_timestep_embedding (seedvr2_dit.cpp:232-253): [count][256],
 * sin(t * exp(-log(10000) * i / 128)) at i, the cos at i + 128, fp32. */
void orc_timestep_embedding(const float* timesteps, int count, float* embedding);

/* unpatchify_prediction (seedvr2_dit.cpp:255-326): source [patches][64] ->
 * destination [tokens][16]; token (f, 2py+y, 2px+x) takes features
 * (2y+x)*16 .. +15 of patch (f, py, px).  shapes are the unpatchified
 * (t, h, w), h and w even.  Returns 0 or -1. */
int orc_unpatchify_prediction(const float* source, long patches, const int* shapes, int batch,
                              float* destination);

/* apply_cfg (seedvr2_pipeline.cpp:171-210): out = neg + scale*(pos - neg) in
 * fp32; with rescale != 0 and count >= 2 it is then multiplied by
 * float(rescale * std(pos) / std(out) + (1 - rescale)), the means and the
 * (count - 1)-normalised deviations in double, unless std(out) is 0. */
void orc_apply_cfg(const float* positive, const float* negative, long count, float scale,
                   float rescale, float* output);

/* Euler update of SeedVR2Pipeline::denoise (seedvr2_pipeline.cpp:575-588):
 * latent channel c (channel_stride floats apart) at token t
 * += delta * prediction[t][c], c < 16, as a product then a sum. */
void orc_euler_step(float* latent, long channel_stride, const float* prediction, long tokens,
                    float delta);

/* The norm and AdaSingle modulation around the DiT block's attention and MLP.
 * The block graph takes six modulation inputs of [batch][hidden] floats
 * (in4..in9, seedvr2_dit.cpp:441-448, 734-738); the operations between them
 * and the hot path are ncnn built-ins of the exported .param, which is not in
 * the reference.  They are restated from the published SeedVR2 NaDiT block:
 * a norm without affine (RMSNorm), the modulation "in"
 * h * (scale_a + scale_b) + (shift_a + shift_b) before the attention and the
 * MLP, the modulation "out" h * (gate_a + gate_b), and the residual sum.
 * The *_a vectors are the per-sample modulation inputs [batch][dim], the *_b
 * vectors the block's own [dim] parameters (NULL: zero).
 *
 * orc_ada_in: row r of sample b (sample_rows[b] rows per sample, in order):
 * out = (x * rs) * (scale_a[b] + scale_b) + (shift_a[b] + shift_b),
 * rs = 1 / sqrt(mean(x^2) + eps), the mean of squares summed in double and
 * rounded to float; every other operation fp32, in this order. */
void orc_ada_in(const float* x, int dim, float eps, const int* sample_rows, int batch,
                const float* shift_a, const float* scale_a, const float* shift_b,
                const float* scale_b, float* out);

/* orc_ada_out: x += y * (gate_a[b] + gate_b) per row of sample b, the
 * gate sum, the product and the residual sum each rounded to fp32. */
void orc_ada_out(float* x, const float* y, int dim, const int* sample_rows, int batch,
                 const float* gate_a, const float* gate_b);

/* The video tokens of SeedVR2Pipeline::predict (seedvr2_pipeline.cpp:296-317):
 * row t of destination [tokens][33] is latent channel 0..15 at t, condition
 * channel 0..15 at t, then 1.  Channels are channel_stride floats apart. */
void orc_video_tokens(const float* latent, const float* condition, long channel_stride,
                      long tokens, float* destination);

/* VAEChunkedMHA::forward (vae_chunked_mha.cpp:223-235): ncnn
 * MultiHeadAttention over one blob (self attention).  x [seq][qdim];
 * wq, wk, wv [embed][qdim] and bq, bk, bv [embed]; wo [qdim][embed], bo
 * [qdim] (the load_model order, :138-152).  Per head h of d = embed / heads:
 * softmax(scale q_h k_h^T) v_h, heads concatenated, then the output
 * projection.  Evaluated in fp64, rounded once to fp32.  rows (or NULL):
 * only the query rows listed (count of them) are computed; out then holds
 * those rows in that order. */
void orc_mha(const float* x, int seq, int qdim, int embed, int heads, float scale,
             const float* wq, const float* bq, const float* wk, const float* bk, const float* wv,
             const float* bv, const float* wo, const float* bo, const int* rows, int count,
             float* out, int num_threads);

/* The depth-to-space shuffle of VAEUpsample3D::forward
 * (vae_upsample3d.cpp:270-318): packed [channels * tr * sr * sr][frames][h][w]
 * (channel stride packed_cstep) -> out [channels][out_t][h * sr][w * sr]
 * (channel stride out_cstep), out_t = frames * tr - remove_head.  Packed
 * channel ((yo * sr + xo) * tr + z) * channels + c, frame f, pixel (y, x)
 * lands at channel c, time f * tr + z (minus one after the removed time 1),
 * pixel (y * sr + yo, x * sr + xo). */
void orc_vae_pixel_shuffle(const float* packed, int channels, int frames, int h, int w,
                           long packed_cstep, int tr, int sr, int remove_head, float* out,
                           long out_cstep);

/* The 16 configuration values of DecomposedConv3D, in the order of its
 * config blob (decomposed_conv3d.cpp:422-441). */
typedef struct orc_conv3d {
    int num_output, num_input, kernel_w, kernel_h, kernel_t, stride_t, dilation_t, head_frames;
    int stride_w, stride_h, dilation_w, dilation_h, pad_w, pad_h, groups, bias_term;
} orc_conv3d;

/* DecomposedConv3D::forward (decomposed_conv3d.cpp:605-755).  input: planar
 * [num_input][frames][height][width], channel stride in_cstep.  memory:
 * planar [num_input][memory_frames][height][width] (channel stride
 * mem_cstep) of the previous slice, or NULL: then the temporal prefix is
 * head_frames copies of input frame 0.  weights: [kernel_t][num_output]
 * [num_input][kernel_h][kernel_w] (one ncnn Convolution weight per temporal
 * tap); bias [num_output] or NULL.  output: planar [num_output][out_t][oh]
 * [ow], channel stride out_cstep.  Each tap's 2-D convolution is evaluated
 * in fp64 and rounded to fp32, then the taps are added in tap order in fp32.
 * next_memory (or NULL): planar [num_input][kernel_t - stride_t][height]
 * [width], channel stride next_cstep: the last kernel_t - stride_t frames of
 * the padded input.  Returns out_t, or -1 (bad configuration, groups != 1,
 * too few frames). */
int orc_decomposed_conv3d(const orc_conv3d* cfg, const float* input, int frames, int height,
                          int width, long in_cstep, const float* memory, int memory_frames,
                          long mem_cstep, const float* weights, const float* bias, float* output,
                          long out_cstep, float* next_memory, long next_cstep, int num_threads);

#ifdef __cplusplus
}
#endif

#endif
