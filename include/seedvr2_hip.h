/*
 * seedvr2_hip.h -- C-ABI of the MI355X (gfx950) window-attention hot path.
 *
 * This is the boundary the C++ ncnn-surface layers (AdaptiveWindowAttention,
 * SharedLinear) call.  Plain C: plain pointers and sizes, no HIP or torch
 * types.  Device pointers are HIP device addresses; a stream is a hipStream_t
 * passed as void* (NULL = the default stream).  No function throws; every
 * function returns one of the codes below, which mirror the reference layers'
 * int returns (src/seedvr2/adaptive_window_attention.cpp:764-978,
 * src/seedvr2/shared_linear.cpp:83-96).
 */
#ifndef SEEDVR2_HIP_H
#define SEEDVR2_HIP_H

#include <stddef.h>
#include <stdint.h>

/* Only the functions below are exported; the library is built with hidden
 * default visibility. */
#if defined(__GNUC__) || defined(__clang__)
#define S2_API __attribute__((visibility("default")))
#else
#define S2_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define S2_OK 0
#define S2_ERR_INVALID (-1)    /* bad configuration, shape or arity (reference -1) */
#define S2_ERR_PLAN (-2)       /* window plan is not a permutation (reference -2) */
#define S2_ERR_ALLOC (-100)    /* allocation failure (reference -100) */
#define S2_ERR_DEVICE (-200)   /* HIP runtime error or no usable gfx950 device */

typedef void* s2_stream_t;

/* Element types of activations.  The 16-bit ones are the two storage types
 * of the reference's Vulkan path (adaptive_window_attention.cpp:1082-1087,
 * 1141: blobs of elembits 16, fp16 or bf16 by ncnn's storage options). */
typedef enum s2_dtype {
    S2_DTYPE_F32 = 0,
    S2_DTYPE_BF16 = 1,
    S2_DTYPE_F16 = 2   /* IEEE binary16 */
} s2_dtype;

typedef enum s2_activation {
    S2_ACT_NONE = 0,
    S2_ACT_GELU = 1,   /* erf-GELU, 0.5 x (1 + erf(x / sqrt 2)) */
    S2_ACT_SWIGLU = 2  /* silu(gate) * up over a gate/up weight pair, see
                          s2_shared_linear_forward */
} s2_activation;

/* One attention window.  Same fields and meaning as the reference
 * seedvr2::WindowSlice (adaptive_window_attention.h:16-27). */
typedef struct s2_window_slice {
    int sample_index;
    int t0, t1, h0, h1, w0, w1;
    int partition_offset;
    int token_count;
} s2_window_slice;

/* AdaptiveWindowAttention configuration.  Field i corresponds to ParamDict
 * id i of the reference load_param (adaptive_window_attention.cpp:700-714);
 * id 9 (shape_values_are_int32) is a blob-decoding detail of the layer and
 * does not reach this boundary. */
typedef struct s2_awa_config {
    int heads;                    /* id 0, default 20 */
    int head_dim;                 /* id 1, default 128; 64 and 128 supported */
    int target_windows[3];        /* ids 2,3,4, default 4,3,3 */
    int shifted;                  /* id 5, default 0 */
    float epsilon;                /* id 6, default 1e-5 */
    int rope_pairs_per_axis;      /* id 7, default 21; 6*pairs <= head_dim */
    int shared_norm;              /* id 8: informational, weights arrive as 4 rows */
    int official_bf16_attention;  /* id 10: round q,k,v and context to bf16 */
} s2_awa_config;

typedef struct s2_awa_plan s2_awa_plan;   /* opaque, device-resident plan */

typedef struct s2_awa_plan_info {
    int batch;
    int num_windows;
    int video_tokens;          /* sum over samples of t*h*w */
    int text_tokens;           /* sum of text lengths */
    size_t workspace_bytes;    /* device workspace s2_awa_forward needs */
} s2_awa_plan_info;

/* ---- device memory (so layer host code needs no HIP headers) ---------- */

/* Number of gfx950 devices visible; 0 with S2_OK when there are none. */
S2_API int s2_device_count(int* count);
S2_API int s2_malloc(void** ptr, size_t bytes);
S2_API int s2_free(void* ptr);
S2_API int s2_memcpy_h2d(void* dst, const void* src, size_t bytes, s2_stream_t stream);
S2_API int s2_memcpy_d2h(void* dst, const void* src, size_t bytes, s2_stream_t stream);
S2_API int s2_memcpy_d2d(void* dst, const void* src, size_t bytes, s2_stream_t stream);
S2_API int s2_stream_synchronize(s2_stream_t stream);
/* Orders `waiter` after the work enqueued on `producer` so far, without a
 * host wait (an event recorded on producer and waited for on waiter).  No
 * counterpart in the reference (one Vulkan queue there): the layers use it
 * when a blob produced on one stream is consumed on another. */
S2_API int s2_stream_wait(s2_stream_t waiter, s2_stream_t producer);
/* Scratch that the split-k GEMM tail and the guidance statistics share
 * between the workgroups of one launch, one allocation per (device, stream)
 * (about 64 MB on MI355X).  An owner of a stream -- a device allocator, a
 * layer whose host path runs on the default stream -- acquires it when it is
 * created: it is allocated then and zeroed on that stream, with no host wait.
 * Each acquire takes one reference; the last release waits for that stream
 * and frees it.  Forward calls only look it up; on a stream nobody acquired,
 * the first forward that needs it makes it the same way (zeroed on its
 * stream, no device-wide synchronisation) and it is kept until the process
 * ends.  No counterpart in the reference (ncnn's Vulkan allocators own their
 * workspaces). */
S2_API int s2_stream_scratch_acquire(s2_stream_t stream);
S2_API int s2_stream_scratch_release(s2_stream_t stream);
/* Last HIP error string recorded by this library on the calling thread. */
S2_API const char* s2_last_error(void);

/* ---- window plan -------------------------------------------------------- */

/* Host-side window list of build_adaptive_window_plan
 * (adaptive_window_attention.cpp:565-655): windows in the reference order
 * (w outer, h, t inner, per sample).  video_shapes is [batch][3] (t,h,w).
 * Pass windows == NULL to query *num_windows.  sample_window_count
 * ([batch]) and video_tokens may be NULL.  Returns S2_OK or S2_ERR_INVALID. */
S2_API int s2_awa_plan_windows(const int* video_shapes, int batch, const int target_windows[3],
                        int shifted, s2_window_slice* windows, int max_windows,
                        int* num_windows, int* sample_window_count, int* video_tokens);

/* Builds the device-resident plan for one set of runtime shapes (the
 * reference rebuilds its plan on every forward, :833-836 and :1116-1120; a
 * caller keeps this handle while the shapes stay the same).  text_lengths is
 * [batch], each > 0 (reference :813-814). */
S2_API int s2_awa_plan_create(const s2_awa_config* config, const int* video_shapes,
                       const int* text_lengths, int batch, s2_awa_plan** plan);
S2_API int s2_awa_plan_get_info(const s2_awa_plan* plan, s2_awa_plan_info* info);
/* Copies the plan's window list / per-sample window counts to host arrays. */
S2_API int s2_awa_plan_get_windows(const s2_awa_plan* plan, s2_window_slice* windows,
                            int max_windows, int* sample_window_count);
S2_API int s2_awa_plan_destroy(s2_awa_plan* plan);

/* Computes the plan's RoPE (cos, sin) table, angle pos * freq[p] for every
 * position the plan's windows and text tokens use (apply_mm_rope,
 * adaptive_window_attention.cpp:521-543, which forms the same angles per
 * token on every forward), once, into memory the plan owns.  Forwards whose
 * rope_freqs argument is this same pointer then read it instead of
 * recomputing it in their workspace; other pointers are unaffected.  After
 * rewriting the frequencies in place, call this again (rope_freqs == NULL
 * clears the cache).  The table is written on `stream`: it must be complete
 * before forwards on other streams use it, and no forward may run on the plan
 * while this call does. */
S2_API int s2_awa_plan_cache_rope(s2_awa_plan* plan, const float* rope_freqs, s2_stream_t stream);

/* Materialises the plan's per-token tables on the device with the same
 * integer index math the forward kernels use: video_indices[L] (partition ->
 * source token), inverse_video_indices[L], local_positions[L][3]
 * (AdaptiveWindowPlan, adaptive_window_attention.h:29-36).  int32 device
 * arrays; any may be NULL. */
S2_API int s2_awa_plan_tables(const s2_awa_plan* plan, int* video_indices,
                       int* inverse_video_indices, int* local_positions,
                       s2_stream_t stream);

/* ---- AdaptiveWindowAttention forward ------------------------------------ */

/* The whole layer (reference CPU forward adaptive_window_attention.cpp:764-978,
 * Vulkan forward :1059-1270): per window, gather video q/k/v by plan index,
 * append the sample's text tokens, RMSNorm q and k, 3-axis RoPE, softmax
 * (q k^T / sqrt(d)) v over window+text, scatter video rows back to source
 * order and mean-pool text rows over the sample's windows.
 *
 * norm_weights: device fp32 [4][head_dim] = video_norm_q, video_norm_k,
 *   text_norm_q, text_norm_k (the upload_model packing, :1047-1053).
 * rope_freqs: device fp32 [rope_pairs_per_axis].
 * video_q/k/v: device rows of width heads*head_dim with row stride
 *   video_row_stride elements: the fused [L][3*inner] blob gives
 *   (base, base+inner, base+2*inner, 3*inner), the split blobs give three
 *   pointers with stride inner (reference 4- and 8-input forms, :768-797).
 * in_dtype: F32, BF16 or F16 for all six inputs.
 * out_video [video_tokens][inner], out_text [text_tokens][inner] in out_dtype.
 * workspace: device memory of at least info.workspace_bytes, 256-byte aligned.
 * All work is enqueued on stream; nothing is synchronised. */
S2_API int s2_awa_forward(const s2_awa_plan* plan, const float* norm_weights,
                   const float* rope_freqs,
                   const void* video_q, const void* video_k, const void* video_v,
                   long video_row_stride,
                   const void* text_q, const void* text_k, const void* text_v,
                   long text_row_stride, s2_dtype in_dtype,
                   void* out_video, void* out_text, s2_dtype out_dtype,
                   void* workspace, size_t workspace_bytes, s2_stream_t stream);

/* The QKV projection and the attention layer in one call: SharedLinear::forward
 * with the fused QKV weight (shared_linear.cpp:83-96) feeding
 * AdaptiveWindowAttention::forward in its 4-input form
 * (adaptive_window_attention.cpp:764-978), as the fused seedvr2_blocks graph
 * chains them.  The projection's epilogue writes the attention's window-ordered
 * Q, K and V^T directly (RMSNorm and RoPE applied), so the [L][3*inner]
 * QKV blob never reaches memory and the gather pass of s2_awa_forward is not
 * needed.  Numerically the norm reads the fp32 projection (+ bias) instead of
 * a rounded QKV blob; everything else is as s2_awa_forward.
 *
 * x_video [video_tokens][hidden], x_text [text_tokens][hidden]: device bf16
 *   rows, contiguous, 16-byte aligned.
 * qkv_weight: device bf16 [3*inner][hidden] (columns [q|k|v] of the output,
 *   head h at h*head_dim, :890-892); qkv_bias: device fp32 [3*inner] or NULL.
 * norm_weights, rope_freqs, out_*, workspace, stream: as s2_awa_forward
 *   (the same workspace size, info.workspace_bytes).
 * Requires heads*head_dim a multiple of 256, head_dim 64 or 128 and hidden a
 * multiple of 64; otherwise S2_ERR_INVALID (use s2_shared_linear_forward and
 * s2_awa_forward).  The projection shares the split-k scratch of
 * s2_shared_linear_forward (per device and stream). */
S2_API int s2_awa_qkv_forward(const s2_awa_plan* plan, const void* x_video, const void* x_text,
                       int hidden, const uint16_t* qkv_weight, const float* qkv_bias,
                       const float* norm_weights, const float* rope_freqs,
                       void* out_video, void* out_text, s2_dtype out_dtype,
                       void* workspace, size_t workspace_bytes, s2_stream_t stream);

/* Stage timing of s2_awa_forward, a diagnostic with no counterpart in the
 * reference.  While enabled on the calling thread, every s2_awa_forward
 * records HIP events on its stream around its four kernels: RoPE table,
 * prologue (window gather, RMSNorm, RoPE), attention, text pool
 * (s2_awa_qkv_forward: RoPE table, QKV projection with the fused prologue,
 * attention, text pool).
 * s2_awa_stage_times waits for the last such forward and returns the four
 * durations in milliseconds. */
S2_API int s2_awa_stage_timing(int enable);
S2_API int s2_awa_stage_times(float stage_ms[4]);

/* ---- SharedLinear -------------------------------------------------------- */

/* fp32 -> bf16 (round to nearest even) on the device; used to keep weights
 * resident in bf16 (SharedLinear::load_model, shared_linear.cpp:61-81). */
S2_API int s2_cast_f32_to_bf16(const float* src, uint16_t* dst, size_t count, s2_stream_t stream);
S2_API int s2_cast_bf16_to_f32(const uint16_t* src, float* dst, size_t count, s2_stream_t stream);

/* The SwiGLU weight layout of s2_shared_linear_forward from a gate and an up
 * projection: gate, up device bf16 [n][k]; gate_bias, up_bias device fp32
 * [n] (both or neither); packed bf16 [2n][k] and packed_bias fp32 [2n] (NULL
 * when there is no bias).  n a multiple of 128.  Device copies on stream. */
S2_API int s2_swiglu_pack_weight(const uint16_t* gate, const uint16_t* up,
                                 const float* gate_bias, const float* up_bias, int n, int k,
                                 uint16_t* packed, float* packed_bias, s2_stream_t stream);

/* Elementwise erf-GELU, y = x * Phi(x), over count values of dtype (fp32
 * arithmetic; y may equal x).  The device path of the ncnn GELU layer
 * (param 0 fast_gelu = 0) when a block graph keeps its MLP activation as a
 * layer of its own instead of SharedLinear's fused epilogue (param 3). */
S2_API int s2_gelu(const void* x, void* y, size_t count, s2_dtype dtype, s2_stream_t stream);

/* ---- ncnn built-in layers of exported graphs ----------------------------- */
/* The device paths of the ncnn built-ins that exported SeedVR2 graphs place
 * around the custom layers (the graphs the reference loads at
 * src/seedvr2/seedvr2_dit.cpp:603-633, 1424-1449): BinaryOp, UnaryOp,
 * Sigmoid, Swish, Reduction (whose Vulkan path the reference patches for
 * large row counts, patches/ncnn/0002-seedvr2-large-vulkan-workloads.patch:
 * 256-284), RMSNorm, and the copies behind Slice, Concat, Crop and Reshape.
 * Operands are 2-D [rows][cols] views with a row stride in elements; element
 * types fp32 / bf16 / fp16, fp32 arithmetic; outputs must not overlap
 * inputs. */

/* ncnn BinaryOp (op: 0 add, 1 sub, 2 mul, 3 div, 4 max, 5 min, 6 pow, 7 rsub,
 * 8 rdiv, 9 rpow, 10 atan2, 11 ratan2): y[r][c] = op(a[r][c], b[r][c]) over
 * [rows][cols], each operand broadcast numpy-style: a_rows (b_rows) is rows
 * or 1, a_cols (b_cols) is cols or 1.  b == NULL: the scalar b_scalar
 * (ncnn's with_scalar). */
S2_API int s2_binary_op(int op, const void* a, s2_dtype a_dtype, int a_rows, int a_cols,
                        long a_stride, const void* b, s2_dtype b_dtype, int b_rows, int b_cols,
                        long b_stride, float b_scalar, void* y, s2_dtype y_dtype, int rows,
                        int cols, long y_stride, s2_stream_t stream);

/* ncnn UnaryOp (op 0 abs, 1 neg, 2 floor, 3 ceil, 4 square, 5 sqrt, 6 rsqrt,
 * 7 exp, 8 log, 9 sin, 10 cos, 11 tan, 12 asin, 13 acos, 14 atan,
 * 15 reciprocal, 16 tanh, 17 log10, 18 round (half to even), 19 trunc), and
 * this build's 100 Sigmoid (1 / (1 + e^-x)) and 101 Swish (x / (1 + e^-x)),
 * over count contiguous values. */
S2_API int s2_unary_op(int op, const void* x, s2_dtype x_dtype, void* y, s2_dtype y_dtype,
                       size_t count, s2_stream_t stream);

/* ncnn Reduction (op 0 sum, 1 asum, 2 sumsq, 3 mean, 4 max, 5 min, 6 prod,
 * 7 l1, 8 l2, 9 logsum, 10 logsumexp; the result times coeff) of a
 * [rows][cols] view: axis 1 reduces each row (y: rows values), axis 0 each
 * column (y: cols values).  y is contiguous. */
S2_API int s2_reduce(int op, float coeff, int axis, const void* x, s2_dtype x_dtype, int rows,
                     int cols, long x_stride, void* y, s2_dtype y_dtype, s2_stream_t stream);

/* ncnn RMSNorm over each row: y = x / sqrt(mean(x^2) + epsilon), times
 * gamma[cols] (fp32, device) when gamma is not NULL. */
S2_API int s2_rms_norm(const void* x, s2_dtype x_dtype, int rows, int cols, long x_stride,
                       const float* gamma, float epsilon, void* y, s2_dtype y_dtype,
                       long y_stride, s2_stream_t stream);

/* dst[r][c] = src[r][c] over [rows][cols], converting the element type. */
S2_API int s2_copy_2d(const void* src, s2_dtype src_dtype, long src_stride, void* dst,
                      s2_dtype dst_dtype, long dst_stride, int rows, int cols,
                      s2_stream_t stream);

/* SharedLinear::forward (shared_linear.cpp:83-96): one projection applied to
 * two token streams in ONE grouped launch sharing the weight:
 *   y_video = act(x_video W^T + b),  y_text = act(x_text W^T + b).
 * weight: device bf16 [n][k] row-major (the reference [N][K] layout,
 * :66-69); bias: device fp32 [n] or NULL (param 2).  x_*: device
 * [m_*][k] in x_dtype; y_*: device [m_*][n] in y_dtype.  The MFMAs take bf16
 * operands: fp32 and fp16 activations are rounded to bf16 (nearest even) as
 * they are staged.  Either stream may have m == 0 (its pointers are then
 * ignored).  k must be a multiple of 8; x, y and weight 16-byte aligned.
 * When the last wave of output tiles would leave the chip mostly idle, its
 * tiles are split along k over several workgroups, which meet in the
 * stream's scratch of partial tiles (one 256 KB slot per compute unit, 64 MB
 * on MI355X, plus counters; see s2_stream_scratch_acquire).  Calls on
 * different streams therefore never share scratch and may run concurrently. *
 * activation S2_ACT_SWIGLU (v3 graphs' MLP, seedvr2_pipeline.cpp:434-438):
 * y = silu(x Wg^T + bg) * (x Wu^T + bu) in one launch.  weight is [2n][k]
 * with the gate and up rows interleaved in blocks of 128 (rows 256j ..
 * 256j+127 are gate rows 128j .., rows 256j+128 .. 256j+255 up rows 128j ..;
 * s2_swiglu_pack_weight builds it), bias likewise [2n] or NULL; n (the
 * output width) a multiple of 128, bf16 activations, k a multiple of 64. */
S2_API int s2_shared_linear_forward(const void* x_video, int m_video, const void* x_text, int m_text,
                             s2_dtype x_dtype, const uint16_t* weight, const float* bias,
                             int n, int k, int activation,
                             void* y_video, void* y_text, s2_dtype y_dtype,
                             s2_stream_t stream);

/* s2_shared_linear_forward without any device allocation.  No counterpart in
 * the reference: it is for callers that cannot allocate (HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments,
 * kernels and results (bit-identical); the split-k scratch is a static
 * device array of about 64 MB (256 partial-tile slots of 256 KB and their
 * counters) that each GPU the library runs on holds until the process ends.
 * A split needing more than 256 sharing workgroups returns S2_ERR_INVALID
 * (it cannot happen on a device of at most 256 compute units).  Every call
 * on one GPU shares that array: calls whose kernels overlap in time on one
 * GPU (different streams) race and must not be made. */
S2_API int s2_shared_linear_forward_noalloc(const void* x_video, int m_video, const void* x_text,
                                            int m_text, s2_dtype x_dtype, const uint16_t* weight,
                                            const float* bias, int n, int k, int activation,
                                            void* y_video, void* y_text, s2_dtype y_dtype,
                                            s2_stream_t stream);

/* ---- DiT frontend and tail, sampler step -------------------------------- */
/* The steps either side of the block stack, on device fp32 buffers.  A video
 * sample is a (frames, height, width) token grid; shapes are int[3] per
 * sample.  Returns S2_ERR_INVALID where the reference returns -1: a
 * non-positive extent, an odd height or width, or sizes that do not match. */

/* patchify_video (src/seedvr2/seedvr2_dit.cpp:167-230): tokens [tokens][33]
 * -> patches [sum t*(h/2)*(w/2)][132]; patch (f, py, px) is the four tokens
 * (2py+y, 2px+x), y outer, each 33 wide.  video_shapes: int[batch][3] on the
 * host.  Both buffers 8-byte aligned. */
S2_API int s2_patchify_video(const float* video, long tokens, const int* video_shapes, int batch,
                             float* patches, s2_stream_t stream);

/* The video tokens SeedVR2Pipeline::predict assembles from the latent and
 * the condition (src/seedvr2/seedvr2_pipeline.cpp:296-317: token t is
 * [latent[0..15][t] | condition[0..15][t] | 1]) and patchifies in
 * SeedVR2DiT::forward (seedvr2_dit.cpp:1224), in one pass without the
 * [tokens][33] intermediate.  latent, condition: 16 channel planes of one
 * sample, plane c at c * channel_stride floats (an ncnn Mat's cstep). */
S2_API int s2_latent_patches(const float* latent, const float* condition, long channel_stride,
                             int frames, int height, int width, float* patches,
                             s2_stream_t stream);

/* make_timestep_embedding (src/seedvr2/seedvr2_dit.cpp:232-253): count
 * timesteps (HOST memory, like the reference's std::vector<float>) ->
 * device [count][256], row s = [sin(t_s f_i) | cos(t_s f_i)],
 * f_i = exp(-ln(10000) i / 128).  Values are the correctly rounded sin/cos of
 * the reference's fp32 phase (within 1 ulp of a C library's sinf/cosf). */
S2_API int s2_timestep_embedding(const float* timesteps, int count, float* embedding,
                                 s2_stream_t stream);

/* unpatchify_prediction (src/seedvr2/seedvr2_dit.cpp:255-326): patches
 * [sum t*(h/2)*(w/2)][64] -> prediction [sum t*h*w][16], the inverse token
 * order of patchify with 16 channels per token.  The patchified shapes are
 * (t, h/2, w/2) of video_shapes.  Both buffers 16-byte aligned. */
S2_API int s2_unpatchify_prediction(const float* patches, long patch_count,
                                    const int* video_shapes, int batch, float* prediction,
                                    s2_stream_t stream);

/* apply_cfg (src/seedvr2/seedvr2_pipeline.cpp:171-210): output = negative +
 * scale (positive - negative), each operation rounded to fp32; when
 * rescale != 0 and count >= 2, output *= (float)(rescale std(positive) /
 * std(output) + (1 - rescale)) (sample standard deviations, accumulated in
 * fp64), unless std(output) is 0.  16-byte aligned operands.  The rescale
 * uses the stream's statistics scratch (40 KB, s2_stream_scratch_acquire),
 * so rescaling calls on different streams never share it. */
S2_API int s2_apply_cfg(const float* positive, const float* negative, long count, float scale,
                        float rescale, float* output, s2_stream_t stream);

/* The Euler update of SeedVR2Pipeline::denoise (src/seedvr2/
 * seedvr2_pipeline.cpp:575-588): latent[c][t] += delta * prediction[t][c]
 * for c < 16, t < tokens, the product rounded before the sum.  latent: 16
 * planes at channel_stride floats; prediction [tokens][16], 16-byte
 * aligned. */
S2_API int s2_euler_step(float* latent, long channel_stride, const float* prediction, long tokens,
                         float delta, s2_stream_t stream);

/* One sampler step after the predictions (src/seedvr2/
 * seedvr2_pipeline.cpp:553-588 with the unpatchify of seedvr2_dit.cpp:1492),
 * straight from the patchified predictions [t*(h/2)*(w/2)][64] of one sample:
 * negative_patches NULL takes the positive prediction as is (the reference's
 * cfg_scale == 1 branch); otherwise apply_cfg(positive, negative, cfg_scale,
 * cfg_rescale).  Then the Euler update of the latent planes.  Equal to
 * s2_unpatchify_prediction, s2_apply_cfg and s2_euler_step in sequence;
 * shares s2_apply_cfg's statistics scratch. */
S2_API int s2_denoise_update(const float* positive_patches, const float* negative_patches,
                             int frames, int height, int width, float cfg_scale,
                             float cfg_rescale, float delta, float* latent, long channel_stride,
                             s2_stream_t stream);

/* ---- DiT block: norm and AdaSingle modulation ---------------------------- */
/* The operations of the DiT block graph between its residual stream, its six
 * per-sample modulation inputs in4..in9 ([batch][hidden] fp32 each,
 * src/seedvr2/seedvr2_dit.cpp:441-448, 734-738) and the SharedLinear /
 * AdaptiveWindowAttention layers.  The exported graph holds them as ncnn
 * built-ins (its .param is not in the reference); they follow the published
 * SeedVR2 NaDiT block: a norm without affine (RMSNorm) and h * scale + shift
 * before the attention and the MLP ("in"), the branch output times gate and
 * the residual sum after them ("out").  Each of scale, shift and gate is the
 * per-sample input plus the block's own [hidden] vector for the stream
 * (video_* / text_*, NULL for none).
 *
 * Rows: video_rows[b] / text_rows[b] (host arrays, text_rows may be NULL for
 * no text) rows of sample b, samples in order, batch 1..64.  hidden is a
 * multiple of 4, at most 4096; row strides are in elements, at least hidden
 * and a multiple of 4; fp32 rows 16-byte and 16-bit rows 8-byte aligned;
 * modulation vectors 16-byte aligned. */

/* out = rmsnorm(x) * (scale[b] + *_scale) + (shift[b] + *_shift), with
 * rmsnorm(x) = x / sqrt(mean(x^2) + epsilon); fp32 arithmetic.  out must not
 * overlap x. */
S2_API int s2_dit_ada_in(int hidden, float epsilon, int batch, const int* video_rows,
                         const int* text_rows, const void* x_video, const void* x_text,
                         s2_dtype x_dtype, long x_stride, const float* shift, const float* scale,
                         const float* video_shift, const float* video_scale,
                         const float* text_shift, const float* text_scale, void* out_video,
                         void* out_text, s2_dtype out_dtype, long out_stride,
                         s2_stream_t stream);

/* out = x + y * (gate[b] + *_gate), out of x's element type; out is either x
 * (in place, same row stride) or does not overlap x or y.  Each product and
 * sum is rounded to fp32. */
S2_API int s2_dit_ada_out(int hidden, int batch, const int* video_rows, const int* text_rows,
                          const void* x_video, const void* x_text, s2_dtype x_dtype,
                          long x_stride, const void* y_video, const void* y_text,
                          s2_dtype y_dtype, long y_stride, const float* gate,
                          const float* video_gate, const float* text_gate, void* out_video,
                          void* out_text, long out_stride, s2_stream_t stream);

/* s2_dit_ada_out and then s2_dit_ada_in on its output in one pass over the
 * residual stream: out = x + y * (gate[b] + *_gate), and h = rmsnorm(out) *
 * (scale[b] + *_scale) + (shift[b] + *_shift), the norm taken over out as
 * stored.  The attention branch's gate and residual sum with the MLP's norm
 * and modulation (or the MLP's with the next block's).  h must not overlap
 * x, y or out. */
S2_API int s2_dit_ada_out_in(int hidden, int batch, const int* video_rows, const int* text_rows,
                             const void* x_video, const void* x_text, s2_dtype x_dtype,
                             long x_stride, const void* y_video, const void* y_text,
                             s2_dtype y_dtype, long y_stride, const float* gate,
                             const float* video_gate, const float* text_gate, void* out_video,
                             void* out_text, long out_stride, float epsilon, const float* shift,
                             const float* scale, const float* video_shift,
                             const float* video_scale, const float* text_shift,
                             const float* text_scale, void* h_video, void* h_text,
                             s2_dtype h_dtype, long h_stride, s2_stream_t stream);

/* The attention's out projection or the MLP's down projection with the gated
 * residual sum in its epilogue: y = x W^T + bias over the video and text
 * streams as s2_shared_linear_forward computes it with bf16 y (no
 * activation), then out = res + y * (gate[b] + *_gate) as s2_dit_ada_out
 * computes it from that y, bit for bit, without writing y to memory.  x is
 * bf16 [m][k] per stream, k % 64 == 0; n (the hidden size) % 8 == 0, at most
 * 4096; video_rows / text_rows as above, summing to m_video / m_text.  res
 * and out rows have pitch n and res_dtype, 16-byte aligned; out is either
 * res (in place) or does not overlap it.  No counterpart in the reference
 * (there the branch output is a blob the next layers read,
 * seedvr2_dit.cpp:722-833); it is the block's two GEMM + residual pairs in
 * one pass over the residual rows. */
S2_API int s2_shared_linear_residual(const void* x_video, int m_video, const void* x_text,
                                     int m_text, const uint16_t* weight, const float* bias,
                                     int n, int k, int batch, const int* video_rows,
                                     const int* text_rows, const void* res_video,
                                     const void* res_text, s2_dtype res_dtype,
                                     const float* gate, const float* video_gate,
                                     const float* text_gate, void* out_video, void* out_text,
                                     s2_stream_t stream);

/* ---- DecomposedConv3D (VAE) ---------------------------------------------- */
/* The causal 3-D convolution of the VAE (src/seedvr2/decomposed_conv3d.h:33-88,
 * decomposed_conv3d.cpp:605-755) as one implicit GEMM on the matrix cores:
 * bf16 operands, fp32 accumulation over the whole kt x kh x kw x num_input
 * window. */

/* The 16 values of the layer's config blob, in blob order
 * (decomposed_conv3d.cpp:422-441). */
typedef struct s2_conv3d_config {
    int num_output, num_input, kernel_w, kernel_h, kernel_t, stride_t, dilation_t, head_frames;
    int stride_w, stride_h, dilation_w, dilation_h, pad_w, pad_h, groups, bias_term;
} s2_conv3d_config;

/* Output (frames, height, width) of a forward over `frames` input frames
 * with `memory_frames` cached frames (0: the prefix is head_frames copies of
 * frame 0), by the reference's arithmetic (:621-634) and ncnn Convolution's
 * output size.  S2_ERR_INVALID where the reference returns -1, including
 * groups != 1 (the reference hands the weights of a grouped configuration to
 * an ungrouped ncnn Convolution). */
S2_API int s2_conv3d_output_shape(const s2_conv3d_config* config, int frames, int height,
                                  int width, int memory_frames, int out_shape[3]);

/* Device weights in the kernel's layout: bf16 [num_output][kp], k = window
 * position ((t * kernel_h + y) * kernel_w + x) * cpad + channel, with cpad 8,
 * 16 or 32 for at most 32 input channels and num_input rounded up to 64
 * otherwise, and kp the positions times cpad rounded up to 64.  `weights`
 * is the reference's per-tap ncnn Convolution weights, device fp32
 * [kernel_t][num_output][num_input][kernel_h][kernel_w] (load_model,
 * :457-471). */
S2_API int s2_conv3d_packed_weight_bytes(const s2_conv3d_config* config, size_t* bytes);
S2_API int s2_conv3d_pack_weights(const s2_conv3d_config* config, const float* weights,
                                  void* packed, s2_stream_t stream);

/* The temporal memory (:727-755): the last kernel_t - stride_t frames of the
 * padded input, kept in this library's staged layout (bf16 channel-last);
 * only s2_conv3d_forward reads or writes it.  *frames = kernel_t - stride_t
 * (0: the layer keeps no memory).  Layers of at most 3 output channels with
 * a 3x3x3 window, unit strides and dilations, one pixel of spatial padding
 * and 16..128 input channels (a multiple of 16; the VAE's RGB output conv)
 * keep instead what those two frames contribute to the next forward's first
 * two output frames: fp32 [2][num_output][height][width]. */
S2_API int s2_conv3d_memory_bytes(const s2_conv3d_config* config, int height, int width,
                                  size_t* bytes, int* frames);
/* Workspace of a forward: the staged input frames (and copied memory
 * frames), plus, for layers whose output tiles would leave most of the chip
 * idle, fp32 partial tiles of a k loop split into ranges of k-steps.  A
 * smaller workspace that still holds the staged frames is accepted; the
 * forward then runs the k loop unsplit.  Layers of more than 128 output
 * channels whose split fits one workgroup per compute unit sum the ranges
 * in the stream's split-k scratch instead (as s2_shared_linear does) and
 * leave that part of the workspace unused.  The layers of at most 3 output
 * channels above read their input in place: their workspace is a copy of
 * the memory, used only when next_memory overlaps memory and the forward
 * has more than 4 output frames (it may be NULL otherwise), and they take no
 * pad_right / pad_bottom. */
S2_API int s2_conv3d_workspace_bytes(const s2_conv3d_config* config, int frames, int height,
                                     int width, int memory_frames, size_t* bytes);
/* The workspace of s2_conv3d_forward_padded: the staged frames are those of
 * the unpadded input, the output extent (and with it the partial tiles of a
 * split k loop) that of the frames padded with pad_right columns and
 * pad_bottom rows, as in VAEDownsample3D (vae_downsample3d.cpp:145-172).
 * Valid for inputs that only the padding makes large enough. */
S2_API int s2_conv3d_workspace_bytes_padded(const s2_conv3d_config* config, int frames,
                                            int height, int width, int pad_right, int pad_bottom,
                                            int memory_frames, size_t* bytes);

/* DecomposedConv3D::forward (decomposed_conv3d.cpp:605-755).  input: device
 * planar [num_input][frames][height][width] in in_dtype, channel stride
 * in_cstep elements (an ncnn Mat's cstep; a multiple of 4, 16-byte aligned
 * base).  memory: the memory a previous forward wrote (memory_frames
 * frames), or NULL: the prefix is then head_frames copies of frame 0.
 * output: planar [num_output][out frames][out h][out w], channel stride
 * out_cstep, out_dtype.  next_memory (or NULL): receives the new memory
 * (s2_conv3d_memory_bytes); it may be the same buffer as memory.  bias:
 * device fp32 [num_output] or NULL.  workspace: s2_conv3d_workspace_bytes,
 * 256-byte aligned. */
S2_API int s2_conv3d_forward(const s2_conv3d_config* config, const void* packed_weights,
                             const float* bias, const void* input, s2_dtype in_dtype, int frames,
                             int height, int width, long in_cstep, const void* memory,
                             int memory_frames, void* output, s2_dtype out_dtype, long out_cstep,
                             void* next_memory, void* workspace, size_t workspace_bytes,
                             s2_stream_t stream);

/* s2_conv3d_forward over the input padded with pad_right zero columns and
 * pad_bottom zero rows: VAEDownsample3D's padding (vae_downsample3d.cpp:145-172)
 * without materialising it.  The output extent is s2_conv3d_output_shape of
 * (height + pad_bottom, width + pad_right); the memory is that of the
 * unpadded frames; the workspace is s2_conv3d_workspace_bytes_padded. */
S2_API int s2_conv3d_forward_padded(const s2_conv3d_config* config, const void* packed_weights,
                                    const float* bias, const void* input, s2_dtype in_dtype,
                                    int frames, int height, int width, long in_cstep,
                                    int pad_right, int pad_bottom, const void* memory,
                                    int memory_frames, void* output, s2_dtype out_dtype,
                                    long out_cstep, void* next_memory, void* workspace,
                                    size_t workspace_bytes, s2_stream_t stream);

/* VAEUpsample3D's depth-to-space shuffle (vae_upsample3d.cpp:270-318): packed
 * [channels * tr * sr * sr][frames][height][width] (channel stride
 * packed_cstep) -> output [channels][frames * tr - remove_head][height * sr]
 * [width * sr] (channel stride out_cstep), both in dtype.  Packed channel
 * ((yo * sr + xo) * tr + z) * channels + c of frame f goes to channel c, time
 * f * tr + z (one less after the removed time 1 when remove_head), pixel
 * (y * sr + yo, x * sr + xo). */
S2_API int s2_vae_pixel_shuffle(const void* packed, s2_dtype dtype, int channels, int frames,
                                int height, int width, long packed_cstep, int temporal_ratio,
                                int spatial_ratio, int remove_head, void* output,
                                long out_cstep, s2_stream_t stream);

/* ---- VAEChunkedMHA (VAE) -------------------------------------------------- */
/* ncnn MultiHeadAttention over one blob (self attention), the CPU forward of
 * VAEChunkedMHA (src/seedvr2/vae_chunked_mha.cpp:223-235; the Vulkan forward
 * :247-281 computes the same in query chunks of param 20).  Per head h of
 * d = embed_dim / num_heads: softmax(scale q_h k_h^T) v_h with q = x Wq^T +
 * bq (likewise k, v), heads concatenated, then out = o Wo^T + bo.  The
 * projections and both attention products run on the matrix cores in bf16
 * with fp32 accumulation; the scores are kept in fp32 until the softmax. */

/* ParamDict ids 0, 1 and 6 of the reference load_param (:116-129); qdim =
 * weight_data_size / embed_dim (the input width).  kdim and vdim equal qdim
 * in the layer's self attention. */
typedef struct s2_mha_config {
    int embed_dim;
    int num_heads;
    int qdim;
    float scale;
} s2_mha_config;

/* Device weights in the kernels' form (bf16 matrices, fp32 biases, the scale
 * folded into the query projection).  The inputs are the reference's
 * load_model blobs (:131-152) as device fp32: wq, wk, wv [embed_dim][qdim],
 * bq, bk, bv [embed_dim], wo [qdim][embed_dim], bo [qdim]. */
S2_API int s2_mha_weight_bytes(const s2_mha_config* config, size_t* bytes);
S2_API int s2_mha_prepare_weights(const s2_mha_config* config, const float* wq, const float* bq,
                                  const float* wk, const float* bk, const float* wv,
                                  const float* bv, const float* wo, const float* bo,
                                  void* prepared, s2_stream_t stream);
/* Workspace of a forward over seq tokens: about seq^2 * 6 bytes (the fp32
 * scores and bf16 probabilities of one head) plus the projections. */
S2_API int s2_mha_workspace_bytes(const s2_mha_config* config, int seq, size_t* bytes);
/* x: device [seq][qdim] in in_dtype; out: device [seq][qdim] in out_dtype;
 * 16-byte aligned rows (qdim a multiple of 8); workspace 256-byte aligned. */
S2_API int s2_mha_forward(const s2_mha_config* config, const void* prepared, const void* x,
                          s2_dtype in_dtype, int seq, void* out, s2_dtype out_dtype,
                          void* workspace, size_t workspace_bytes, s2_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SEEDVR2_HIP_H */
