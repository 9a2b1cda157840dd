/*
 * CPU oracle for the SeedVR2 window-attention hot path -- TEST INFRASTRUCTURE.
 * Used only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
 * always as the reference result or the CPU baseline, never as the product.
 * See oracle.h for the pinning of each function.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ceil_div_extent (adaptive_window_attention.cpp:434-437) */
static int ceil_div_extent(int extent, int window) { return (extent + window - 1) / window; }

/* python_round_positive (adaptive_window_attention.cpp:439-444): nearbyint in
 * the default round-to-nearest-even mode. */
static int python_round_positive(double value) { return (int)nearbyint(value); }

static int imin(int a, int b) { return a < b ? a : b; }
static int imax(int a, int b) { return a > b ? a : b; }

/* Per-sample loop bounds (adaptive_window_attention.cpp:576-606). */
typedef struct {
    int t, h, w, wt, wh, ww;
    double st, sh, sw;
    int loop_nt, loop_nh, loop_nw;
} sample_geometry;

static int sample_setup(const int* shape, const int target[3], int shifted,
                        sample_geometry* g)
{
    g->t = shape[0];
    g->h = shape[1];
    g->w = shape[2];
    if (g->t <= 0 || g->h <= 0 || g->w <= 0 || target[0] <= 0 || target[1] <= 0 ||
        target[2] <= 0)
        return -1;
    const double scale = sqrt(3600.0 / (double)(g->h * g->w));     /* :583 */
    const int resized_h = python_round_positive(g->h * scale);     /* :584 */
    const int resized_w = python_round_positive(g->w * scale);     /* :585 */
    g->wt = ceil_div_extent(imin(g->t, 30), target[0]);             /* :586 */
    g->wh = ceil_div_extent(resized_h, target[1]);                  /* :587 */
    g->ww = ceil_div_extent(resized_w, target[2]);                  /* :588 */
    if (g->wt <= 0 || g->wh <= 0 || g->ww <= 0)
        return -1;
    g->st = shifted && g->wt < g->t ? 0.5 : 0.0;                    /* :592-594 */
    g->sh = shifted && g->wh < g->h ? 0.5 : 0.0;
    g->sw = shifted && g->ww < g->w ? 0.5 : 0.0;
    const int nt = g->st > 0.0 ? (int)ceil((g->t - g->st) / g->wt) + 1 : 1;   /* :596-598 */
    const int nh = g->sh > 0.0 ? (int)ceil((g->h - g->sh) / g->wh) + 1 : 1;
    const int nw = g->sw > 0.0 ? (int)ceil((g->w - g->sw) / g->ww) + 1 : 1;
    g->loop_nt = shifted ? nt : ceil_div_extent(g->t, g->wt);       /* :601-606 */
    g->loop_nh = shifted ? nh : ceil_div_extent(g->h, g->wh);
    g->loop_nw = shifted ? nw : ceil_div_extent(g->w, g->ww);
    return 0;
}

/* Window bounds along one axis (adaptive_window_attention.cpp:611-613,
 * 619-621, 627-629).  The casts truncate toward zero like static_cast<int>. */
static void axis_bounds(int shifted, int i, double s, int e, int n, int* lo, int* hi)
{
    if (shifted) {
        *lo = imax((int)((i - s) * e), 0);
        *hi = imin((int)((i - s + 1.0) * e), n);
    } else {
        *lo = i * e;
        *hi = imin((i + 1) * e, n);
    }
}

typedef struct {
    orc_slice* windows;
    int max_windows;
    int num_windows;
    int* video_indices;
    int* local_positions;
    int num_tokens;
} plan_sink;

/* append_slice (adaptive_window_attention.cpp:446-473): tokens inside a
 * window in t,h,w row-major order. */
static void append_slice(plan_sink* sink, int sample_index, int sample_offset,
                         const sample_geometry* g, int t0, int t1, int h0, int h1,
                         int w0, int w1)
{
    if (sink->windows && sink->num_windows < sink->max_windows) {
        orc_slice* s = &sink->windows[sink->num_windows];
        s->sample_index = sample_index;
        s->t0 = t0; s->t1 = t1; s->h0 = h0; s->h1 = h1; s->w0 = w0; s->w1 = w1;
        s->partition_offset = sink->num_tokens;
        s->token_count = (t1 - t0) * (h1 - h0) * (w1 - w0);
    }
    sink->num_windows++;
    for (int ti = t0; ti < t1; ti++)
        for (int hi = h0; hi < h1; hi++)
            for (int wi = w0; wi < w1; wi++) {
                const int p = sink->num_tokens++;
                if (sink->video_indices)
                    sink->video_indices[p] = sample_offset + (ti * g->h + hi) * g->w + wi;
                if (sink->local_positions) {
                    sink->local_positions[p * 3 + 0] = ti - t0;
                    sink->local_positions[p * 3 + 1] = hi - h0;
                    sink->local_positions[p * 3 + 2] = wi - w0;
                }
            }
}

/* The window loops (adaptive_window_attention.cpp:608-640): w outer, then h,
 * then t innermost; empty windows are skipped. */
static int walk_plan(const int* video_shapes, int batch, const int target[3], int shifted,
                     plan_sink* sink, int* sample_window_count, int* total_tokens)
{
    int total = 0;
    for (int sample = 0; sample < batch; sample++) {
        sample_geometry g;
        if (sample_setup(video_shapes + sample * 3, target, shifted, &g) != 0)
            return -1;
        const int first = sink->num_windows;
        for (int iw = 0; iw < g.loop_nw; iw++) {
            int w0, w1;
            axis_bounds(shifted, iw, g.sw, g.ww, g.w, &w0, &w1);
            if (w1 <= w0)
                continue;
            for (int ih = 0; ih < g.loop_nh; ih++) {
                int h0, h1;
                axis_bounds(shifted, ih, g.sh, g.wh, g.h, &h0, &h1);
                if (h1 <= h0)
                    continue;
                for (int it = 0; it < g.loop_nt; it++) {
                    int t0, t1;
                    axis_bounds(shifted, it, g.st, g.wt, g.t, &t0, &t1);
                    if (t1 <= t0)
                        continue;
                    append_slice(sink, sample, total, &g, t0, t1, h0, h1, w0, w1);
                }
            }
        }
        if (sample_window_count)
            sample_window_count[sample] = sink->num_windows - first;
        total += g.t * g.h * g.w;
    }
    *total_tokens = total;
    return 0;
}

int orc_plan_count(const int* video_shapes, int batch, const int target_windows[3],
                   int shifted, int* num_windows, int* total_tokens)
{
    plan_sink sink = {0};
    int total = 0;
    if (batch <= 0)
        return -1;
    const int ret = walk_plan(video_shapes, batch, target_windows, shifted, &sink, NULL, &total);
    if (ret != 0)
        return ret;
    *num_windows = sink.num_windows;
    *total_tokens = total;
    return 0;
}

int orc_plan_build(const int* video_shapes, int batch, const int target_windows[3],
                   int shifted, orc_slice* windows, int max_windows,
                   int* sample_window_count, int* video_indices,
                   int* inverse_video_indices, int* local_positions)
{
    plan_sink sink = {0};
    sink.windows = windows;
    sink.max_windows = max_windows;
    int total = 0;
    int own_indices = 0;
    if (batch <= 0)
        return -1;
    int nwin = 0, ntok = 0;
    if (orc_plan_count(video_shapes, batch, target_windows, shifted, &nwin, &ntok) != 0)
        return -1;
    if (windows && nwin > max_windows)
        return -1;
    if (!video_indices) {
        video_indices = (int*)malloc(sizeof(int) * (size_t)(ntok > 0 ? ntok : 1));
        if (!video_indices)
            return -100;
        own_indices = 1;
    }
    sink.video_indices = video_indices;
    sink.local_positions = local_positions;
    int ret = walk_plan(video_shapes, batch, target_windows, shifted, &sink,
                        sample_window_count, &total);
    /* Permutation check (adaptive_window_attention.cpp:642-653). */
    if (ret == 0 && sink.num_tokens != total)
        ret = -2;
    if (ret == 0) {
        int* inverse = inverse_video_indices;
        int own_inverse = 0;
        if (!inverse) {
            inverse = (int*)malloc(sizeof(int) * (size_t)(total > 0 ? total : 1));
            own_inverse = 1;
        }
        for (int i = 0; i < total; i++)
            inverse[i] = -1;
        for (int p = 0; p < sink.num_tokens && ret == 0; p++) {
            const int src = video_indices[p];
            if (src < 0 || src >= total || inverse[src] != -1)
                ret = -2;
            else
                inverse[src] = p;
        }
        if (own_inverse)
            free(inverse);
    }
    if (own_indices)
        free(video_indices);
    return ret;
}

float orc_round_bf16(float value)
{
    uint32_t bits;
    memcpy(&bits, &value, sizeof(bits));
    if ((bits & 0x7f800000u) != 0x7f800000u)
        bits += 0x00007fffu + ((bits >> 16) & 1u);
    bits &= 0xffff0000u;
    memcpy(&value, &bits, sizeof(value));
    return value;
}

void orc_round_bf16_array(const float* in, float* out, long count)
{
    for (long i = 0; i < count; i++)
        out[i] = orc_round_bf16(in[i]);
}

void orc_rms_norm(const float* input, const float* weight, int size, float epsilon,
                  float* output)
{
    float square_sum = 0.f;
    for (int i = 0; i < size; i++)
        square_sum += input[i] * input[i];
    const float inv_rms = 1.f / sqrtf(square_sum / size + epsilon);
    for (int i = 0; i < size; i++)
        output[i] = input[i] * inv_rms * weight[i];
}

void orc_apply_mm_rope(float* values, int head_dim, const float* freqs,
                       int pairs_per_axis, const int position[3])
{
    const int axis_width = pairs_per_axis * 2;
    const int rotary_width = axis_width * 3;
    if (rotary_width > head_dim)
        return;
    for (int axis = 0; axis < 3; axis++) {
        float* axis_values = values + axis * axis_width;
        for (int pair = 0; pair < pairs_per_axis; pair++) {
            const float angle = position[axis] * freqs[pair];
            const float cosine = cosf(angle);
            const float sine = sinf(angle);
            const float x0 = axis_values[pair * 2];
            const float x1 = axis_values[pair * 2 + 1];
            axis_values[pair * 2] = x0 * cosine - x1 * sine;
            axis_values[pair * 2 + 1] = x0 * sine + x1 * cosine;
        }
    }
}

/* One head of textbook SDPA: logits = q.k * scale, softmax with max
 * subtraction, then the probability-weighted sum of v. */
static void sdpa_head(const float* q, const float* k, const float* v, int seq, int d,
                      float scale, float* out, float* logits)
{
    for (int i = 0; i < seq; i++) {
        const float* qi = q + (size_t)i * d;
        float m = -INFINITY;
        for (int j = 0; j < seq; j++) {
            const float* kj = k + (size_t)j * d;
            float dot = 0.f;
            for (int c = 0; c < d; c++)
                dot += qi[c] * kj[c];
            logits[j] = dot * scale;
            if (logits[j] > m)
                m = logits[j];
        }
        float sum = 0.f;
        for (int j = 0; j < seq; j++) {
            logits[j] = expf(logits[j] - m);
            sum += logits[j];
        }
        const float inv = 1.f / sum;
        float* oi = out + (size_t)i * d;
        for (int c = 0; c < d; c++)
            oi[c] = 0.f;
        for (int j = 0; j < seq; j++) {
            const float p = logits[j] * inv;
            const float* vj = v + (size_t)j * d;
            for (int c = 0; c < d; c++)
                oi[c] += p * vj[c];
        }
    }
}

void orc_sdpa(const float* q, const float* k, const float* v, int heads, int seq,
              int head_dim, float* out, int num_threads)
{
    const float scale = 1.f / sqrtf((float)head_dim);
    const size_t plane = (size_t)seq * head_dim;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(num_threads > 0 ? num_threads : 1)
#endif
    for (int h = 0; h < heads; h++) {
        float* logits = (float*)malloc(sizeof(float) * (size_t)seq);
        sdpa_head(q + h * plane, k + h * plane, v + h * plane, seq, head_dim, scale,
                  out + h * plane, logits);
        free(logits);
    }
    (void)num_threads;
}

int orc_awa_forward(const orc_awa_params* p,
                    const float* video_norm_q, const float* video_norm_k,
                    const float* text_norm_q, const float* text_norm_k,
                    const float* rope_freqs,
                    const int* video_shapes, const int* text_lengths, int batch,
                    const float* video_q, const float* video_k, const float* video_v,
                    long video_stride,
                    const float* text_q, const float* text_k, const float* text_v,
                    long text_stride,
                    float* out_video, float* out_text,
                    const int* window_subset, int num_subset, int num_threads)
{
    /* Argument checks (adaptive_window_attention.cpp:769-772, 813-814). */
    if (!p || p->heads <= 0 || p->head_dim <= 0 || p->rope_pairs_per_axis * 6 > p->head_dim ||
        !video_norm_q || !video_norm_k || !text_norm_q || !text_norm_k || !rope_freqs ||
        batch <= 0)
        return -1;
    const int heads = p->heads, d = p->head_dim, inner = heads * d;
    int nwin = 0, lv = 0, lt = 0;
    for (int s = 0; s < batch; s++) {
        if (text_lengths[s] <= 0)
            return -1;
        lt += text_lengths[s];
    }
    int ret = orc_plan_count(video_shapes, batch, p->target_windows, p->shifted, &nwin, &lv);
    if (ret != 0)
        return ret;
    orc_slice* windows = (orc_slice*)malloc(sizeof(orc_slice) * (size_t)nwin);
    int* counts = (int*)malloc(sizeof(int) * (size_t)batch);
    int* indices = (int*)malloc(sizeof(int) * (size_t)lv);
    int* positions = (int*)malloc(sizeof(int) * 3 * (size_t)lv);
    int* text_offsets = (int*)malloc(sizeof(int) * (size_t)batch);
    if (!windows || !counts || !indices || !positions || !text_offsets) {
        ret = -100;
        goto done;
    }
    ret = orc_plan_build(video_shapes, batch, p->target_windows, p->shifted, windows, nwin,
                         counts, indices, NULL, positions);
    if (ret != 0)
        goto done;

    /* Outputs zero-filled (:838-845); text offsets (:863-865). */
    memset(out_video, 0, sizeof(float) * (size_t)lv * inner);
    memset(out_text, 0, sizeof(float) * (size_t)lt * inner);
    text_offsets[0] = 0;
    for (int s = 1; s < batch; s++)
        text_offsets[s] = text_offsets[s - 1] + text_lengths[s - 1];

    const int n_iter = window_subset ? num_subset : nwin;
    for (int it = 0; it < n_iter && ret == 0; it++) {        /* window loop :873-975 */
        const int wi = window_subset ? window_subset[it] : it;
        if (wi < 0 || wi >= nwin) {
            ret = -1;
            break;
        }
        const orc_slice* win = &windows[wi];
        const int sample = win->sample_index;
        const int text_length = text_lengths[sample];
        const int seq = win->token_count + text_length;
        const size_t plane = (size_t)seq * d;
        float* query = (float*)malloc(sizeof(float) * plane * heads);   /* :880-884 */
        float* key = (float*)malloc(sizeof(float) * plane * heads);
        float* value = (float*)malloc(sizeof(float) * plane * heads);
        float* context = (float*)malloc(sizeof(float) * plane * heads);
        if (!query || !key || !value || !context) {
            free(query); free(key); free(value); free(context);
            ret = -100;
            break;
        }
        /* Video tokens (:886-906): gather by plan index, RMSNorm q/k, RoPE at
         * (lt + text_length, lh, lw). */
        for (int local = 0; local < win->token_count; local++) {
            const int part = win->partition_offset + local;
            const int src = indices[part];
            const float* sq = video_q + (size_t)src * video_stride;
            const float* sk = video_k + (size_t)src * video_stride;
            const float* sv = video_v + (size_t)src * video_stride;
            int pos[3] = {positions[part * 3] + text_length, positions[part * 3 + 1],
                          positions[part * 3 + 2]};
            for (int h = 0; h < heads; h++) {
                float* q = query + h * plane + (size_t)local * d;
                float* k = key + h * plane + (size_t)local * d;
                float* v = value + h * plane + (size_t)local * d;
                orc_rms_norm(sq + h * d, video_norm_q, d, p->epsilon, q);
                orc_rms_norm(sk + h * d, video_norm_k, d, p->epsilon, k);
                memcpy(v, sv + h * d, sizeof(float) * d);
                orc_apply_mm_rope(q, d, rope_freqs, p->rope_pairs_per_axis, pos);
                orc_apply_mm_rope(k, d, rope_freqs, p->rope_pairs_per_axis, pos);
            }
        }
        /* Text tokens of the sample, redone per window (:908-927). */
        for (int tt = 0; tt < text_length; tt++) {
            const int src = text_offsets[sample] + tt;
            const int dst = win->token_count + tt;
            const float* sq = text_q + (size_t)src * text_stride;
            const float* sk = text_k + (size_t)src * text_stride;
            const float* sv = text_v + (size_t)src * text_stride;
            int pos[3] = {tt, tt, tt};
            for (int h = 0; h < heads; h++) {
                float* q = query + h * plane + (size_t)dst * d;
                float* k = key + h * plane + (size_t)dst * d;
                float* v = value + h * plane + (size_t)dst * d;
                orc_rms_norm(sq + h * d, text_norm_q, d, p->epsilon, q);
                orc_rms_norm(sk + h * d, text_norm_k, d, p->epsilon, k);
                memcpy(v, sv + h * d, sizeof(float) * d);
                orc_apply_mm_rope(q, d, rope_freqs, p->rope_pairs_per_axis, pos);
                orc_apply_mm_rope(k, d, rope_freqs, p->rope_pairs_per_axis, pos);
            }
        }
        if (p->official_bf16_attention) {                              /* :929-938 */
            for (size_t i = 0; i < plane * heads; i++) {
                query[i] = orc_round_bf16(query[i]);
                key[i] = orc_round_bf16(key[i]);
                value[i] = orc_round_bf16(value[i]);
            }
        }
        orc_sdpa(query, key, value, heads, seq, d, context, num_threads);   /* :939-945 */
        if (p->official_bf16_attention)                                  /* :946-952 */
            for (size_t i = 0; i < plane * heads; i++)
                context[i] = orc_round_bf16(context[i]);
        /* Video scatter back to source order (:954-961). */
        for (int local = 0; local < win->token_count; local++) {
            const int src = indices[win->partition_offset + local];
            float* o = out_video + (size_t)src * inner;
            for (int h = 0; h < heads; h++)
                memcpy(o + h * d, context + h * plane + (size_t)local * d, sizeof(float) * d);
        }
        /* Text mean-pool over the sample's windows, in window order (:963-974). */
        const float pool_scale = 1.f / counts[sample];
        for (int tt = 0; tt < text_length; tt++) {
            float* o = out_text + (size_t)(text_offsets[sample] + tt) * inner;
            const int ctx = win->token_count + tt;
            for (int h = 0; h < heads; h++) {
                const float* in = context + h * plane + (size_t)ctx * d;
                for (int c = 0; c < d; c++)
                    o[h * d + c] += in[c] * pool_scale;
            }
        }
        free(query); free(key); free(value); free(context);
    }
done:
    free(windows); free(counts); free(indices); free(positions); free(text_offsets);
    return ret;
}

static float gelu_erf(float x) { return 0.5f * x * (1.f + erff(x * 0.70710678118654752f)); }

void orc_linear(const float* x, int m, int k, const float* w, const float* bias, int n,
                int activation, float* y, const int* rows, int num_rows, int num_threads)
{
    const int out_rows = rows ? num_rows : m;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(num_threads > 0 ? num_threads : 1)
#endif
    for (int r = 0; r < out_rows; r++) {
        const int row = rows ? rows[r] : r;
        const float* xr = x + (size_t)row * k;
        float* yr = y + (size_t)r * n;
        for (int j = 0; j < n; j++) {
            const float* wj = w + (size_t)j * k;
            float acc = 0.f;
            for (int c = 0; c < k; c++)
                acc += xr[c] * wj[c];
            if (bias)
                acc += bias[j];
            yr[j] = activation == 1 ? gelu_erf(acc) : acc;
        }
    }
    (void)num_threads;
}

/* ---- DiT frontend and tail -------------------------------------------------- */

/* seedvr2_dit.cpp:167-230 */
int orc_patchify_video(const float* source, long tokens, const int* shapes, int batch,
                       float* destination)
{
    long expected = 0;
    for (int b = 0; b < batch; b++) {
        const int t = shapes[3 * b], h = shapes[3 * b + 1], w = shapes[3 * b + 2];
        if (t <= 0 || h <= 0 || w <= 0 || h % 2 != 0 || w % 2 != 0)
            return -1;
        expected += (long)t * h * w;
    }
    if (expected != tokens)
        return -1;
    long in_off = 0, out_row = 0;
    for (int b = 0; b < batch; b++) {
        const int t = shapes[3 * b], h = shapes[3 * b + 1], w = shapes[3 * b + 2];
        for (int f = 0; f < t; f++)
            for (int py = 0; py < h / 2; py++)
                for (int px = 0; px < w / 2; px++) {
                    float* out = destination + (out_row++) * 132;
                    for (int y = 0; y < 2; y++)
                        for (int x = 0; x < 2; x++) {
                            const long tok = in_off + ((long)f * h + py * 2 + y) * w + px * 2 + x;
                            memcpy(out + (y * 2 + x) * 33, source + tok * 33, 33 * sizeof(float));
                        }
                }
        in_off += (long)t * h * w;
    }
    return 0;
}

/* seedvr2_dit.cpp:232-253 */
void orc_timestep_embedding(const float* timesteps, int count, float* embedding)
{
    const int half_dim = 128;
    for (int s = 0; s < count; s++) {
        float* out = embedding + (long)s * 2 * half_dim;
        for (int i = 0; i < half_dim; i++) {
            const float exponent = -logf(10000.f) * i / half_dim;
            const float phase = timesteps[s] * expf(exponent);
            out[i] = sinf(phase);
            out[i + half_dim] = cosf(phase);
        }
    }
}

/* seedvr2_dit.cpp:255-326 */
int orc_unpatchify_prediction(const float* source, long patches, const int* shapes, int batch,
                              float* destination)
{
    long expected = 0;
    for (int b = 0; b < batch; b++) {
        const int t = shapes[3 * b], h = shapes[3 * b + 1], w = shapes[3 * b + 2];
        if (t <= 0 || h <= 0 || w <= 0 || h % 2 != 0 || w % 2 != 0)
            return -1;
        expected += (long)t * (h / 2) * (w / 2);
    }
    if (expected != patches)
        return -1;
    long patch_off = 0, out_off = 0;
    for (int b = 0; b < batch; b++) {
        const int t = shapes[3 * b], h = shapes[3 * b + 1], w = shapes[3 * b + 2];
        const int ph = h / 2, pw = w / 2;
        for (int f = 0; f < t; f++)
            for (int py = 0; py < ph; py++)
                for (int px = 0; px < pw; px++) {
                    const float* in = source + (patch_off + ((long)f * ph + py) * pw + px) * 64;
                    for (int y = 0; y < 2; y++)
                        for (int x = 0; x < 2; x++) {
                            const long tok = out_off + ((long)f * h + py * 2 + y) * w + px * 2 + x;
                            memcpy(destination + tok * 16, in + (y * 2 + x) * 16, 16 * sizeof(float));
                        }
                }
        patch_off += (long)t * ph * pw;
        out_off += (long)t * h * w;
    }
    return 0;
}

/* seedvr2_pipeline.cpp:171-210 */
void orc_apply_cfg(const float* positive, const float* negative, long count, float scale,
                   float rescale, float* output)
{
    for (long i = 0; i < count; i++)
        output[i] = negative[i] + scale * (positive[i] - negative[i]);
    if (rescale == 0.f || count < 2)
        return;
    double pos_mean = 0.0, cfg_mean = 0.0;
    for (long i = 0; i < count; i++) {
        pos_mean += positive[i];
        cfg_mean += output[i];
    }
    pos_mean /= count;
    cfg_mean /= count;
    double pos_var = 0.0, cfg_var = 0.0;
    for (long i = 0; i < count; i++) {
        const double p = positive[i] - pos_mean;
        const double c = output[i] - cfg_mean;
        pos_var += p * p;
        cfg_var += c * c;
    }
    const double pos_std = sqrt(pos_var / (count - 1));
    const double cfg_std = sqrt(cfg_var / (count - 1));
    if (cfg_std == 0.0)
        return;
    const float factor = (float)(rescale * pos_std / cfg_std + (1.f - rescale));
    for (long i = 0; i < count; i++)
        output[i] *= factor;
}

/* seedvr2_pipeline.cpp:575-588 */
void orc_euler_step(float* latent, long channel_stride, const float* prediction, long tokens,
                    float delta)
{
    for (long t = 0; t < tokens; t++)
        for (int c = 0; c < 16; c++) {
            const float step = delta * prediction[t * 16 + c];
            latent[c * channel_stride + t] += step;
        }
}

/* seedvr2_pipeline.cpp:296-317 */
void orc_video_tokens(const float* latent, const float* condition, long channel_stride,
                      long tokens, float* destination)
{
    for (long t = 0; t < tokens; t++) {
        float* row = destination + t * 33;
        for (int c = 0; c < 16; c++) {
            row[c] = latent[c * channel_stride + t];
            row[c + 16] = condition[c * channel_stride + t];
        }
        row[32] = 1.f;
    }
}

/* decomposed_conv3d.cpp:605-755: padded frame p of the sequence [prefix |
 * input] comes from the memory (p < memory_frames), from input frame 0
 * (p < head_frames without memory) or from input frame p - prefix. */
static const float* conv3d_source_frame(const float* input, long in_cstep, int frames,
                                        const float* memory, int memory_frames, long mem_cstep,
                                        int prefix, int padded_index, int plane, long* cstep)
{
    if (memory && padded_index < prefix) {
        if (padded_index >= memory_frames)
            return NULL;
        *cstep = mem_cstep;
        return memory + (long)padded_index * plane;
    }
    const int source = padded_index < prefix ? 0 : padded_index - prefix;
    if (source < 0 || source >= frames)
        return NULL;
    *cstep = in_cstep;
    return input + (long)source * plane;
}

int orc_decomposed_conv3d(const orc_conv3d* cfg, const float* input, int frames, int height,
                          int width, long in_cstep, const float* memory, int memory_frames,
                          long mem_cstep, const float* weights, const float* bias, float* output,
                          long out_cstep, float* next_memory, long next_cstep, int num_threads)
{
    const orc_conv3d c = *cfg;
    if (c.num_output <= 0 || c.num_input <= 0 || c.kernel_w <= 0 || c.kernel_h <= 0 ||
        c.kernel_t <= 0 || c.stride_t <= 0 || c.dilation_t <= 0 || c.stride_w <= 0 ||
        c.stride_h <= 0 || c.dilation_w <= 0 || c.dilation_h <= 0 || c.groups != 1 ||
        c.head_frames < 0 || frames <= 0)
        return -1;
    const int use_memory = memory != NULL && memory_frames > 0;
    const int prefix = use_memory ? memory_frames : c.head_frames;
    const int padded_t = frames + prefix;
    const int extent = c.dilation_t * (c.kernel_t - 1) + 1;
    if (padded_t < extent)
        return -1;
    const int out_t = (padded_t - extent) / c.stride_t + 1;
    const int ow = (width + 2 * c.pad_w - c.dilation_w * (c.kernel_w - 1) - 1) / c.stride_w + 1;
    const int oh = (height + 2 * c.pad_h - c.dilation_h * (c.kernel_h - 1) - 1) / c.stride_h + 1;
    if (ow <= 0 || oh <= 0)
        return -1;
    const int plane = height * width, oplane = oh * ow;
    const long wtap = (long)c.num_output * c.num_input * c.kernel_h * c.kernel_w;
    const float* mem = use_memory ? memory : NULL;
    for (int o = 0; o < out_t; o++)
        for (int tap = 0; tap < c.kernel_t; tap++) {
            long cs = 0;
            if (!conv3d_source_frame(input, in_cstep, frames, mem, memory_frames, mem_cstep,
                                     prefix, o * c.stride_t + tap * c.dilation_t, plane, &cs))
                return -1;
        }
    for (int co = 0; co < c.num_output; co++)
        for (int o = 0; o < out_t; o++)
            memset(output + co * out_cstep + (long)o * oplane, 0, sizeof(float) * oplane);
#pragma omp parallel for schedule(dynamic, 1) num_threads(num_threads > 0 ? num_threads : 1)
    for (int co = 0; co < c.num_output; co++) {
        for (int o = 0; o < out_t; o++) {
            float* out = output + co * out_cstep + (long)o * oplane;
            for (int tap = 0; tap < c.kernel_t; tap++) {
                long cs = 0;
                const float* src = conv3d_source_frame(input, in_cstep, frames, mem, memory_frames,
                                                       mem_cstep, prefix,
                                                       o * c.stride_t + tap * c.dilation_t,
                                                       plane, &cs);
                const float* wt = weights + tap * wtap + (long)co * c.num_input * c.kernel_h * c.kernel_w;
                for (int y = 0; y < oh; y++)
                    for (int x = 0; x < ow; x++) {
                        /* the tap's ncnn Convolution: bias (tap 0 only) plus
                         * the zero-padded window sum */
                        double acc = (tap == 0 && bias) ? bias[co] : 0.0;
                        for (int ci = 0; ci < c.num_input; ci++)
                            for (int ky = 0; ky < c.kernel_h; ky++) {
                                const int yi = y * c.stride_h + ky * c.dilation_h - c.pad_h;
                                if (yi < 0 || yi >= height)
                                    continue;
                                for (int kx = 0; kx < c.kernel_w; kx++) {
                                    const int xi = x * c.stride_w + kx * c.dilation_w - c.pad_w;
                                    if (xi < 0 || xi >= width)
                                        continue;
                                    acc += (double)wt[((long)ci * c.kernel_h + ky) * c.kernel_w + kx] *
                                           src[ci * cs + (long)yi * width + xi];
                                }
                            }
                        out[(long)y * ow + x] += (float)acc;
                    }
            }
        }
    }
    const int cache = c.kernel_t - c.stride_t;
    if (next_memory && cache > 0) {
        if (cache > padded_t)
            return -1;
        for (int f = 0; f < cache; f++) {
            long cs = 0;
            const float* src = conv3d_source_frame(input, in_cstep, frames, mem, memory_frames,
                                                   mem_cstep, prefix, padded_t - cache + f, plane,
                                                   &cs);
            if (!src)
                return -1;
            for (int ci = 0; ci < c.num_input; ci++)
                memcpy(next_memory + ci * next_cstep + (long)f * plane, src + ci * cs,
                       sizeof(float) * plane);
        }
    }
    return out_t;
}

/* vae_chunked_mha.cpp:223-235 with ncnn MultiHeadAttention's semantics */
void orc_mha(const float* x, int seq, int qdim, int embed, int heads, float scale,
             const float* wq, const float* bq, const float* wk, const float* bk, const float* wv,
             const float* bv, const float* wo, const float* bo, const int* rows, int count,
             float* out, int num_threads)
{
    const int d = embed / heads;
    double* k = (double*)malloc(sizeof(double) * (size_t)seq * embed);
    double* v = (double*)malloc(sizeof(double) * (size_t)seq * embed);
#pragma omp parallel for schedule(static) num_threads(num_threads > 0 ? num_threads : 1)
    for (int t = 0; t < seq; t++)
        for (int e = 0; e < embed; e++) {
            double sk = bk[e], sv = bv[e];
            for (int c = 0; c < qdim; c++) {
                sk += (double)wk[(size_t)e * qdim + c] * x[(size_t)t * qdim + c];
                sv += (double)wv[(size_t)e * qdim + c] * x[(size_t)t * qdim + c];
            }
            k[(size_t)t * embed + e] = sk;
            v[(size_t)t * embed + e] = sv;
        }
    const int n = rows ? count : seq;
#pragma omp parallel for schedule(dynamic, 1) num_threads(num_threads > 0 ? num_threads : 1)
    for (int i = 0; i < n; i++) {
        const int r = rows ? rows[i] : i;
        double* q = (double*)malloc(sizeof(double) * embed);
        double* o = (double*)malloc(sizeof(double) * embed);
        double* p = (double*)malloc(sizeof(double) * seq);
        for (int e = 0; e < embed; e++) {
            double s = bq[e];
            for (int c = 0; c < qdim; c++)
                s += (double)wq[(size_t)e * qdim + c] * x[(size_t)r * qdim + c];
            q[e] = s;
        }
        for (int h = 0; h < heads; h++) {
            double mx = -INFINITY;
            for (int t = 0; t < seq; t++) {
                double s = 0.0;
                for (int j = 0; j < d; j++)
                    s += q[h * d + j] * k[(size_t)t * embed + h * d + j];
                p[t] = s * scale;
                if (p[t] > mx)
                    mx = p[t];
            }
            double sum = 0.0;
            for (int t = 0; t < seq; t++) {
                p[t] = exp(p[t] - mx);
                sum += p[t];
            }
            for (int j = 0; j < d; j++) {
                double acc = 0.0;
                for (int t = 0; t < seq; t++)
                    acc += p[t] * v[(size_t)t * embed + h * d + j];
                o[h * d + j] = acc / sum;
            }
        }
        for (int c = 0; c < qdim; c++) {
            double s = bo[c];
            for (int e = 0; e < embed; e++)
                s += (double)wo[(size_t)c * embed + e] * o[e];
            out[(size_t)i * qdim + c] = (float)s;
        }
        free(q);
        free(o);
        free(p);
    }
    free(k);
    free(v);
}

/* vae_upsample3d.cpp:270-318 */
void orc_vae_pixel_shuffle(const float* packed, int channels, int frames, int h, int w,
                           long packed_cstep, int tr, int sr, int remove_head, float* out,
                           long out_cstep)
{
    const int ow = w * sr, oh = h * sr;
    const int out_t = frames * tr - (remove_head ? 1 : 0);
    for (int c = 0; c < channels; c++)
        for (int f = 0; f < frames; f++)
            for (int z = 0; z < tr; z++) {
                const int st = f * tr + z;
                if (remove_head && st == 1)
                    continue;
                const int ot = remove_head && st > 1 ? st - 1 : st;
                if (ot >= out_t)
                    continue;
                for (int yo = 0; yo < sr; yo++)
                    for (int xo = 0; xo < sr; xo++) {
                        const int pc = ((yo * sr + xo) * tr + z) * channels + c;
                        const float* src = packed + pc * packed_cstep + (long)f * h * w;
                        float* dst = out + c * out_cstep + (long)ot * oh * ow;
                        for (int y = 0; y < h; y++)
                            for (int x = 0; x < w; x++)
                                dst[(long)(y * sr + yo) * ow + x * sr + xo] = src[(long)y * w + x];
                    }
            }
}

/* ---- DiT block norm and AdaSingle modulation (seedvr2_dit.cpp:441-448) --- */

void orc_ada_in(const float* x, int dim, float eps, const int* sample_rows, int batch,
                const float* shift_a, const float* scale_a, const float* shift_b,
                const float* scale_b, float* out) {
    long row = 0;
    for (int b = 0; b < batch; ++b) {
        const float* sa = shift_a + (long)b * dim;
        const float* ca = scale_a + (long)b * dim;
        for (int i = 0; i < sample_rows[b]; ++i, ++row) {
            const float* xr = x + row * dim;
            float* yr = out + row * dim;
            double ss = 0.0;
            for (int c = 0; c < dim; ++c) ss += (double)xr[c] * xr[c];
            const float ms = (float)(ss / dim);
            const float rs = 1.0f / sqrtf(ms + eps);
            for (int c = 0; c < dim; ++c) {
                const float sc = ca[c] + (scale_b ? scale_b[c] : 0.0f);
                const float sh = sa[c] + (shift_b ? shift_b[c] : 0.0f);
                const float n = xr[c] * rs;
                const float m = n * sc;
                yr[c] = m + sh;
            }
        }
    }
}

void orc_ada_out(float* x, const float* y, int dim, const int* sample_rows, int batch,
                 const float* gate_a, const float* gate_b) {
    long row = 0;
    for (int b = 0; b < batch; ++b) {
        const float* ga = gate_a + (long)b * dim;
        for (int i = 0; i < sample_rows[b]; ++i, ++row) {
            float* xr = x + row * dim;
            const float* yr = y + row * dim;
            for (int c = 0; c < dim; ++c) {
                const float g = ga[c] + (gate_b ? gate_b[c] : 0.0f);
                const float p = yr[c] * g;
                xr[c] = xr[c] + p;
            }
        }
    }
}
