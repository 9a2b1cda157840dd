// extern "C" boundary of the window-attention hot path (include/seedvr2_hip.h).
#include <limits.h>
#include <string.h>

#include <algorithm>
#include <new>
#include <string>
#include <vector>

#include "awa_kernels.h"
#include "awa_plan.h"
#include "block_kernels.h"
#include "conv3d_kernels.h"
#include "graph_ops_kernels.h"
#include "mha_kernels.h"
#include "pipeline_kernels.h"
#include "seedvr2_hip.h"
#include "stream_scratch.h"

namespace {

thread_local std::string g_last_error;

int fail_hip(hipError_t e, const char* what) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    return S2_ERR_DEVICE;
}

int fail(int code, const char* what) {
    g_last_error = what;
    return code;
}

#define S2_HIP(call)                                  \
    do {                                              \
        hipError_t e_ = (call);                       \
        if (e_ != hipSuccess) return fail_hip(e_, #call); \
    } while (0)

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

bool valid_config(const s2_awa_config* c) {
    return c && c->heads > 0 && (c->head_dim == 64 || c->head_dim == 128) &&
           c->rope_pairs_per_axis >= 0 && c->rope_pairs_per_axis * 6 <= c->head_dim &&
           c->target_windows[0] > 0 && c->target_windows[1] > 0 && c->target_windows[2] > 0;
}

}  // namespace

namespace {

// Per-thread stage timing of s2_awa_forward (s2_awa_stage_timing).
struct StageTimer {
    bool on = false;
    bool created = false;
    bool recorded = false;
    hipEvent_t ev[5] = {};
};

StageTimer& stage_timer() {
    thread_local StageTimer t;
    return t;
}

bool dtype_ok(s2_dtype t) { return t == S2_DTYPE_F32 || t == S2_DTYPE_BF16 || t == S2_DTYPE_F16; }
size_t dtype_bytes(s2_dtype t) { return t == S2_DTYPE_F32 ? 4 : 2; }

bool aligned(const void* p, size_t a) { return ((uintptr_t)p) % a == 0; }

// VAEChunkedMHA configuration checks of the reference load_param
// (vae_chunked_mha.cpp:124-128); the GEMMs need 16-byte operand rows.
bool mha_config_ok(const s2_mha_config* c) {
    return c && c->embed_dim > 0 && c->num_heads > 0 && c->embed_dim % c->num_heads == 0 &&
           c->qdim > 0 && c->qdim % 8 == 0 && (c->embed_dim / c->num_heads) % 8 == 0;
}

// Byte layout of the prepared MHA weights: bf16 wq (scaled), wk, wv, wo,
// then fp32 bq (scaled), bk, bv, bo, each 256-byte aligned.
struct MhaWeights {
    size_t wq, wk, wv, wo, bq, bk, bv, bo, total;
};

MhaWeights mha_layout(const s2_mha_config* c) {
    MhaWeights m;
    const size_t mat = align256((size_t)c->embed_dim * c->qdim * 2);
    m.wq = 0;
    m.wk = m.wq + mat;
    m.wv = m.wk + mat;
    m.wo = m.wv + mat;
    m.bq = m.wo + mat;
    m.bk = m.bq + align256((size_t)c->embed_dim * 4);
    m.bv = m.bk + align256((size_t)c->embed_dim * 4);
    m.bo = m.bv + align256((size_t)c->embed_dim * 4);
    m.total = m.bo + align256((size_t)c->qdim * 4);
    return m;
}

// Workspace of a forward: staged x and the per-head buffers.
struct MhaWork {
    int lp;   // seq rounded up to 64: the k extent of the P V product
    size_t xp, q, k, vt, s, p, oh, o, total;
};

MhaWork mha_work(const s2_mha_config* c, int seq) {
    MhaWork w;
    const int d = c->embed_dim / c->num_heads;
    w.lp = (seq + 63) / 64 * 64;
    w.xp = 0;
    w.q = w.xp + align256((size_t)w.lp * c->qdim * 2);
    w.k = w.q + align256((size_t)w.lp * d * 2);
    w.vt = w.k + align256((size_t)w.lp * d * 2);
    w.s = w.vt + align256((size_t)d * w.lp * 2);
    w.p = w.s + align256((size_t)seq * seq * 4);
    w.oh = w.p + align256((size_t)seq * w.lp * 2);
    w.o = w.oh + align256((size_t)seq * d * 2);
    w.total = w.o + (c->num_heads > 1 ? align256((size_t)seq * c->embed_dim * 2) : 0);
    return w;
}

// DecomposedConv3D configuration checks of the reference load_model
// (decomposed_conv3d.cpp:442-446), plus groups == 1 and a spatial window of
// at most 32 positions (the kernel keeps one bit per position).
bool conv3d_config_ok(const s2_conv3d_config* c) {
    return c && c->num_output > 0 && c->num_input > 0 && c->kernel_w > 0 && c->kernel_h > 0 &&
           c->kernel_t > 0 && c->stride_t > 0 && c->dilation_t > 0 && c->stride_w > 0 &&
           c->stride_h > 0 && c->dilation_w > 0 && c->dilation_h > 0 && c->groups == 1 &&
           c->head_frames >= 0 && c->pad_w >= 0 && c->pad_h >= 0 &&
           c->kernel_w * c->kernel_h <= 32;
}

s2::Conv3dShape conv3d_shape(const s2_conv3d_config* c) {
    s2::Conv3dShape s;
    s.cin = c->num_input;
    s.cout = c->num_output;
    s.cpad = s2::conv3d_cpad(c->num_input);
    s.kt = c->kernel_t;
    s.kh = c->kernel_h;
    s.kw = c->kernel_w;
    s.st = c->stride_t;
    s.sh = c->stride_h;
    s.sw = c->stride_w;
    s.dt = c->dilation_t;
    s.dh = c->dilation_h;
    s.dw = c->dilation_w;
    s.ph = c->pad_h;
    s.pw = c->pad_w;
    return s;
}

// Output extent of forward (decomposed_conv3d.cpp:621-634); false where the
// reference returns -1.
bool conv3d_out(const s2_conv3d_config* c, int frames, int height, int width, int memory_frames,
                int* to, int* ho, int* wo) {
    if (!conv3d_config_ok(c) || frames <= 0 || height <= 0 || width <= 0 || memory_frames < 0)
        return false;
    const int prefix = memory_frames > 0 ? memory_frames : c->head_frames;
    const long padded = (long)frames + prefix;
    const long extent = (long)c->dilation_t * (c->kernel_t - 1) + 1;
    if (padded < extent) return false;
    *to = (int)((padded - extent) / c->stride_t + 1);
    *ho = (height + 2 * c->pad_h - c->dilation_h * (c->kernel_h - 1) - 1) / c->stride_h + 1;
    *wo = (width + 2 * c->pad_w - c->dilation_w * (c->kernel_w - 1) - 1) / c->stride_w + 1;
    return *ho > 0 && *wo > 0;
}

// Validates video sample shapes as the reference's patchify/unpatchify do
// (seedvr2_dit.cpp:181-191, 270-283): positive, even height and width.
// Returns the token and patch totals.
bool video_shapes_ok(const int* shapes, int batch, long* tokens, long* patches) {
    if (!shapes || batch <= 0) return false;
    long nt = 0, np = 0;
    for (int b = 0; b < batch; ++b) {
        const int t = shapes[3 * b], h = shapes[3 * b + 1], w = shapes[3 * b + 2];
        if (t <= 0 || h <= 0 || w <= 0 || h % 2 != 0 || w % 2 != 0) return false;
        nt += (long)t * h * w;
        np += (long)t * (h / 2) * (w / 2);
    }
    *tokens = nt;
    *patches = np;
    return true;
}

}  // namespace

extern "C" {

const char* s2_last_error(void) { return g_last_error.c_str(); }

int s2_device_count(int* count) {
    if (!count) return S2_ERR_INVALID;
    *count = 0;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return S2_OK;
    }
    for (int i = 0; i < n; ++i) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, i) == hipSuccess &&
            strncmp(prop.gcnArchName, "gfx950", 6) == 0)
            ++*count;
    }
    return S2_OK;
}

int s2_malloc(void** ptr, size_t bytes) {
    if (!ptr) return S2_ERR_INVALID;
    *ptr = nullptr;
    if (bytes == 0) return S2_OK;
    hipError_t e = hipMalloc(ptr, bytes);
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) {
        fail_hip(e, "hipMalloc");
        return S2_ERR_ALLOC;
    }
    if (e != hipSuccess) return fail_hip(e, "hipMalloc");
    return S2_OK;
}

int s2_free(void* ptr) {
    if (ptr) S2_HIP(hipFree(ptr));
    return S2_OK;
}

int s2_memcpy_h2d(void* dst, const void* src, size_t bytes, s2_stream_t stream) {
    if (bytes == 0) return S2_OK;
    S2_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream));
    return S2_OK;
}

int s2_memcpy_d2h(void* dst, const void* src, size_t bytes, s2_stream_t stream) {
    if (bytes == 0) return S2_OK;
    S2_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream));
    return S2_OK;
}

int s2_memcpy_d2d(void* dst, const void* src, size_t bytes, s2_stream_t stream) {
    if (bytes == 0) return S2_OK;
    S2_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, (hipStream_t)stream));
    return S2_OK;
}

int s2_stream_synchronize(s2_stream_t stream) {
    S2_HIP(hipStreamSynchronize((hipStream_t)stream));
    return S2_OK;
}

// ---- ncnn built-in layers of exported graphs --------------------------------

namespace {

bool view_ok(const void* p, int rows, int cols, long stride) {
    return p && rows > 0 && cols > 0 && stride >= cols;
}

}  // namespace

int s2_binary_op(int op, const void* a, s2_dtype a_dtype, int a_rows, int a_cols, long a_stride,
                 const void* b, s2_dtype b_dtype, int b_rows, int b_cols, long b_stride,
                 float b_scalar, void* y, s2_dtype y_dtype, int rows, int cols, long y_stride,
                 s2_stream_t stream) {
    if (op < 0 || op > 11) return fail(S2_ERR_INVALID, "binary op type 0..11");
    if (rows <= 0 || cols <= 0 || !y || y_stride < cols)
        return fail(S2_ERR_INVALID, "output shape or stride");
    if (!dtype_ok(a_dtype) || !dtype_ok(y_dtype) || (b && !dtype_ok(b_dtype)))
        return fail(S2_ERR_INVALID, "unsupported dtype");
    auto bcast_ok = [&](int r, int c, long stride, const void* p) {
        return p && (r == rows || r == 1) && (c == cols || c == 1) && stride >= c;
    };
    if (!bcast_ok(a_rows, a_cols, a_stride, a) || (b && !bcast_ok(b_rows, b_cols, b_stride, b)))
        return fail(S2_ERR_INVALID, "operand shapes do not broadcast to the output");
    s2::BinaryArgs p = {};
    p.op = op;
    p.a = a;
    p.a_kind = (int)a_dtype;
    p.a_rs = a_rows == 1 ? 0 : a_stride;
    p.a_cs = a_cols == 1 ? 0 : 1;
    p.b = b;
    p.b_kind = b ? (int)b_dtype : 0;
    p.b_rs = b && b_rows != 1 ? b_stride : 0;
    p.b_cs = b && b_cols != 1 ? 1 : 0;
    p.b_scalar = b_scalar;
    p.y = y;
    p.y_kind = (int)y_dtype;
    p.y_rs = y_stride;
    p.rows = rows;
    p.cols = cols;
    S2_HIP(s2::launch_binary(p, (hipStream_t)stream));
    return S2_OK;
}

int s2_unary_op(int op, const void* x, s2_dtype x_dtype, void* y, s2_dtype y_dtype, size_t count,
                s2_stream_t stream) {
    if (!((op >= 0 && op <= 19) || op == 100 || op == 101))
        return fail(S2_ERR_INVALID, "unary op type 0..19, 100 sigmoid or 101 swish");
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype)) return fail(S2_ERR_INVALID, "unsupported dtype");
    if (count == 0) return S2_OK;
    if (!x || !y) return fail(S2_ERR_INVALID, "null operand");
    S2_HIP(s2::launch_unary(op, x, (int)x_dtype, y, (int)y_dtype, count, (hipStream_t)stream));
    return S2_OK;
}

int s2_reduce(int op, float coeff, int axis, const void* x, s2_dtype x_dtype, int rows, int cols,
              long x_stride, void* y, s2_dtype y_dtype, s2_stream_t stream) {
    if (op < 0 || op > 10) return fail(S2_ERR_INVALID, "reduction op type 0..10");
    if (axis != 0 && axis != 1) return fail(S2_ERR_INVALID, "reduction axis 0 (columns) or 1 (rows)");
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype)) return fail(S2_ERR_INVALID, "unsupported dtype");
    if (!view_ok(x, rows, cols, x_stride) || !y) return fail(S2_ERR_INVALID, "operand shape or stride");
    S2_HIP(s2::launch_reduce(op, coeff, axis, x, (int)x_dtype, x_stride, rows, cols, y, (int)y_dtype,
                             (hipStream_t)stream));
    return S2_OK;
}

int s2_rms_norm(const void* x, s2_dtype x_dtype, int rows, int cols, long x_stride,
                const float* gamma, float epsilon, void* y, s2_dtype y_dtype, long y_stride,
                s2_stream_t stream) {
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype)) return fail(S2_ERR_INVALID, "unsupported dtype");
    if (!view_ok(x, rows, cols, x_stride) || !view_ok(y, rows, cols, y_stride))
        return fail(S2_ERR_INVALID, "operand shape or stride");
    if (!(epsilon >= 0.f)) return fail(S2_ERR_INVALID, "epsilon must be >= 0");
    S2_HIP(s2::launch_rms_norm(x, (int)x_dtype, x_stride, rows, cols, gamma, epsilon, y, (int)y_dtype,
                               y_stride, (hipStream_t)stream));
    return S2_OK;
}

int s2_copy_2d(const void* src, s2_dtype src_dtype, long src_stride, void* dst, s2_dtype dst_dtype,
               long dst_stride, int rows, int cols, s2_stream_t stream) {
    if (!dtype_ok(src_dtype) || !dtype_ok(dst_dtype)) return fail(S2_ERR_INVALID, "unsupported dtype");
    if (rows == 0 || cols == 0) return S2_OK;
    if (!view_ok(src, rows, cols, src_stride) || !view_ok(dst, rows, cols, dst_stride))
        return fail(S2_ERR_INVALID, "operand shape or stride");
    S2_HIP(s2::launch_copy2d(src, (int)src_dtype, src_stride, dst, (int)dst_dtype, dst_stride, rows, cols,
                             (hipStream_t)stream));
    return S2_OK;
}

int s2_stream_wait(s2_stream_t waiter, s2_stream_t producer) {
    if (waiter == producer) return S2_OK;
    hipEvent_t ev;
    S2_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    hipError_t e = hipEventRecord(ev, (hipStream_t)producer);
    if (e == hipSuccess) e = hipStreamWaitEvent((hipStream_t)waiter, ev, 0);
    // the wait holds what it needs: the event may go now
    const hipError_t d = hipEventDestroy(ev);
    S2_HIP(e);
    S2_HIP(d);
    return S2_OK;
}

int s2_stream_scratch_acquire(s2_stream_t stream) {
    S2_HIP(s2::stream_scratch_acquire((hipStream_t)stream));
    return S2_OK;
}

int s2_stream_scratch_release(s2_stream_t stream) {
    S2_HIP(s2::stream_scratch_release((hipStream_t)stream));
    return S2_OK;
}

int s2_awa_plan_windows(const int* video_shapes, int batch, const int target_windows[3],
                        int shifted, s2_window_slice* windows, int max_windows,
                        int* num_windows, int* sample_window_count, int* video_tokens) {
    std::vector<s2_window_slice> w;
    std::vector<int> counts;
    int tokens = 0;
    const int ret = s2::build_window_slices(video_shapes, batch, target_windows, shifted != 0, w,
                                            counts, tokens);
    if (ret != S2_OK) return fail(ret, "invalid window plan shapes");
    if (num_windows) *num_windows = (int)w.size();
    if (video_tokens) *video_tokens = tokens;
    if (sample_window_count) std::copy(counts.begin(), counts.end(), sample_window_count);
    if (windows) {
        if ((int)w.size() > max_windows) return fail(S2_ERR_INVALID, "window buffer too small");
        std::copy(w.begin(), w.end(), windows);
    }
    return S2_OK;
}

int s2_awa_plan_create(const s2_awa_config* config, const int* video_shapes,
                       const int* text_lengths, int batch, s2_awa_plan** out) {
    if (!out) return S2_ERR_INVALID;
    *out = nullptr;
    if (!valid_config(config) || !video_shapes || !text_lengths || batch <= 0)
        return fail(S2_ERR_INVALID, "invalid attention configuration");
    for (int b = 0; b < batch; ++b)
        if (text_lengths[b] <= 0) return fail(S2_ERR_INVALID, "text length must be positive");

    s2_awa_plan* plan = new (std::nothrow) s2_awa_plan();
    if (!plan) return S2_ERR_ALLOC;
    plan->config = *config;
    plan->batch = batch;
    plan->video_shapes.assign(video_shapes, video_shapes + 3 * batch);
    plan->text_lengths.assign(text_lengths, text_lengths + batch);
    int ret = s2::build_window_slices(video_shapes, batch, config->target_windows,
                                      config->shifted != 0, plan->windows,
                                      plan->sample_window_count, plan->video_tokens);
    if (ret != S2_OK) {
        delete plan;
        return fail(ret, "invalid window plan shapes");
    }
    plan->num_windows = (int)plan->windows.size();
    const int heads = config->heads, d = config->head_dim, inner = heads * d;

    // Per-sample offsets.
    std::vector<int> text_off(batch), tok_off(batch), first_win(batch);
    for (int b = 0, to = 0, vo = 0, fw = 0; b < batch; ++b) {
        text_off[b] = to;
        tok_off[b] = vo;
        first_win[b] = fw;
        to += text_lengths[b];
        vo += video_shapes[3 * b] * video_shapes[3 * b + 1] * video_shapes[3 * b + 2];
        fw += plan->sample_window_count[b];
    }
    plan->text_tokens = text_off[batch - 1] + text_lengths[batch - 1];

    // Window records, padded segments, text partial rows, prologue chunks.
    std::vector<s2::ChunkRef> chunks;
    long seg = 0;
    int tpart = 0, rope_pos = 1, grow = 0;
    plan->win_meta.resize(plan->num_windows);
    for (int i = 0; i < plan->num_windows; ++i) {
        const s2_window_slice& s = plan->windows[i];
        s2::WinMeta& m = plan->win_meta[i];
        const int b = s.sample_index;
        m.sample = b;
        m.t0 = s.t0; m.h0 = s.h0; m.w0 = s.w0;
        m.et = s.t1 - s.t0; m.eh = s.h1 - s.h0; m.ew = s.w1 - s.w0;
        m.part_off = s.partition_offset;
        m.n_video = s.token_count;
        m.text_len = text_lengths[b];
        m.seq = s.token_count + m.text_len;
        m.seg_off = (int)seg;
        m.text_off = text_off[b];
        m.grid_h = video_shapes[3 * b + 1];
        m.grid_w = video_shapes[3 * b + 2];
        m.tok_off = tok_off[b];
        m.tpart_off = tpart;
        m.grow_off = grow;
        grow += (s.token_count + 1) / 2 * 2;
        // the segment holds the window's video rows only: each sample's text
        // rows are staged once, after all segments
        const int padded = (m.n_video + s2::kSegAlign - 1) / s2::kSegAlign * s2::kSegAlign;
        for (int r = 0; r < padded; r += s2::kSegAlign) chunks.push_back(s2::ChunkRef{i, r});
        seg += padded;
        tpart += m.text_len;
        rope_pos = std::max(rope_pos, m.et - 1 + m.text_len + 1);
        rope_pos = std::max(rope_pos, std::max(m.eh, m.ew));
        rope_pos = std::max(rope_pos, m.text_len);
        plan->max_window_tokens = std::max(plan->max_window_tokens, m.n_video);
    }
    // Text staging rows after the window segments: sample b's text at ts_row
    // (padded to kSegAlign), written once by the prologue's text chunks (on
    // the sample's first window) or by the fused QKV projection; the
    // attention reads every window's text keys and queries there.
    plan->seg_text = seg;
    std::vector<int> ts_row(batch), tr_off(batch);
    int tr = 0;   // text rows of the fused QKV row space, each sample's run even
    for (int b = 0; b < batch; ++b) {
        ts_row[b] = (int)seg;
        tr_off[b] = tr;
        const int padded = (text_lengths[b] + s2::kSegAlign - 1) / s2::kSegAlign * s2::kSegAlign;
        const s2::WinMeta& fw = plan->win_meta[first_win[b]];
        for (int r = 0; r < padded; r += s2::kSegAlign)
            chunks.push_back(s2::ChunkRef{first_win[b], fw.n_video + r});
        seg += padded;
        tr += (text_lengths[b] + 1) / 2 * 2;
    }
    for (s2::WinMeta& m : plan->win_meta) m.ts_row = ts_row[m.sample];
    plan->seg_total = std::max<long>(seg, 1);
    // the attention addresses a head's Q/K rows and V^T keys through one
    // buffer descriptor with 32-bit offsets
    if (plan->seg_total * config->head_dim * 2 > 0xffffffffL) {
        delete plan;
        return fail(S2_ERR_INVALID, "attention workspace rows beyond 32-bit buffer offsets");
    }
    plan->qkv_text_row = (grow + 7) / 8 * 8;
    plan->qkv_rows = plan->qkv_text_row + tr;
    plan->text_partial_rows = tpart;
    plan->rope_positions = rope_pos;
    plan->num_chunks = (int)chunks.size();

    // Attention items: (window, head) pairs, longest sequence first, dealt
    // round-robin to the XCDs; the query tiles of one pair stay consecutive
    // on one XCD so its K/V tiles are shared through that XCD's L2.
    std::vector<std::pair<int, int> > pairs;
    for (int i = 0; i < plan->num_windows; ++i)
        for (int h = 0; h < heads; ++h) pairs.emplace_back(i, h);
    std::stable_sort(pairs.begin(), pairs.end(), [&](const std::pair<int, int>& a,
                                                     const std::pair<int, int>& b) {
        return plan->win_meta[a.first].seq > plan->win_meta[b.first].seq;
    });
    std::vector<std::vector<s2::AttnItem> > lists(s2::kNumXcd);
    std::vector<long> load(s2::kNumXcd, 0);
    for (const auto& pr : pairs) {
        const s2::WinMeta& m = plan->win_meta[pr.first];
        const int tiles = (m.seq + 127) / 128;
        // the least loaded XCD takes the next pair (LPT)
        const int x = (int)(std::min_element(load.begin(), load.end()) - load.begin());
        for (int t = 0; t < tiles; ++t) lists[x].push_back({pr.first, 128 * t, pr.second, 0});
        load[x] += (long)tiles * m.seq;
    }
    size_t slots = 0;
    for (const auto& l : lists) slots = std::max(slots, l.size());
    plan->slots_per_xcd = (int)slots;
    std::vector<s2::AttnItem> items(slots * s2::kNumXcd, s2::AttnItem{-1, 0, 0, 0});
    for (int x = 0; x < s2::kNumXcd; ++x)
        std::copy(lists[x].begin(), lists[x].end(), items.begin() + (size_t)x * slots);

    std::vector<s2::SampleMeta> samples(batch);
    for (int b = 0; b < batch; ++b)
        samples[b] = {first_win[b], plan->sample_window_count[b], text_off[b], text_lengths[b],
                      1.f / plan->sample_window_count[b]};
    std::vector<int> text_sample(plan->text_tokens);
    for (int b = 0; b < batch; ++b)
        for (int t = 0; t < text_lengths[b]; ++t) text_sample[text_off[b] + t] = b;

    // Row table of the fused QKV projection: window runs in plan order, each
    // starting at its grow_off, then the text tokens from qkv_text_row.  A
    // video row holds its source token (append_slice's t,h,w walk,
    // adaptive_window_attention.cpp:462-471) and its window-local position
    // with the temporal axis offset by the text length (:901-902); a text row
    // its token and the position (i, i, i) within its sample (:915).
    const int qkv_tiles = (plan->qkv_rows + 255) / 256;
    std::vector<s2::QkvRow> qrows((size_t)qkv_tiles * 256, s2::QkvRow{-1, 0, 0, 0});
    for (int i = 0; i < plan->num_windows; ++i) {
        const s2::WinMeta& m = plan->win_meta[i];
        const int run_end = i + 1 < plan->num_windows ? plan->win_meta[i + 1].grow_off
                                                      : plan->qkv_text_row;
        for (int R = m.grow_off; R < run_end; ++R) {
            const int r = R - m.grow_off;
            s2::QkvRow& q = qrows[R];
            q.dest = m.seg_off + r;
            if (r < m.n_video) {
                const int plane = m.eh * m.ew;
                const int lt = r / plane, lh = (r - lt * plane) / m.ew, lw = r - lt * plane - lh * m.ew;
                q.src = m.tok_off + ((m.t0 + lt) * m.grid_h + (m.h0 + lh)) * m.grid_w + (m.w0 + lw);
                q.pos01 = (lt + m.text_len) | (lh << 16);
                q.pos2 = lw | (1 << 16);
            }
        }
    }
    // text runs: sample b's tokens from qkv_text_row + tr_off[b] (even), to
    // its staging rows; a run's gap row keeps the staging row that follows
    for (int b = 0; b < batch; ++b) {
        const int run = (text_lengths[b] + 1) / 2 * 2;
        for (int tt = 0; tt < run; ++tt) {
            s2::QkvRow& q = qrows[plan->qkv_text_row + tr_off[b] + tt];
            q.dest = ts_row[b] + tt;
            if (tt < text_lengths[b]) {
                q.src = text_off[b] + tt;
                q.pos01 = tt | (tt << 16);
                q.pos2 = tt | (2 << 16);
            }
        }
    }

    // One device allocation for all metadata.
    const size_t sz_w = align256(sizeof(s2::WinMeta) * plan->num_windows);
    const size_t sz_s = align256(sizeof(s2::SampleMeta) * batch);
    const size_t sz_t = align256(sizeof(int) * plan->text_tokens);
    const size_t sz_c = align256(sizeof(s2::ChunkRef) * chunks.size());
    const size_t sz_i = align256(sizeof(s2::AttnItem) * items.size());
    const size_t sz_q = align256(sizeof(s2::QkvRow) * qrows.size());
    std::vector<unsigned char> host(sz_w + sz_s + sz_t + sz_c + sz_i + sz_q, 0);
    size_t o = 0;
    memcpy(host.data() + o, plan->win_meta.data(), sizeof(s2::WinMeta) * plan->num_windows);
    o += sz_w;
    memcpy(host.data() + o, samples.data(), sizeof(s2::SampleMeta) * batch);
    o += sz_s;
    memcpy(host.data() + o, text_sample.data(), sizeof(int) * plan->text_tokens);
    o += sz_t;
    memcpy(host.data() + o, chunks.data(), sizeof(s2::ChunkRef) * chunks.size());
    o += sz_c;
    memcpy(host.data() + o, items.data(), sizeof(s2::AttnItem) * items.size());
    o += sz_i;
    memcpy(host.data() + o, qrows.data(), sizeof(s2::QkvRow) * qrows.size());

    hipError_t e = hipGetDevice(&plan->device);
    if (e == hipSuccess) e = hipMalloc(&plan->d_meta, host.size());
    if (e == hipSuccess) e = hipMemcpy(plan->d_meta, host.data(), host.size(), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        if (plan->d_meta) (void)hipFree(plan->d_meta);
        delete plan;
        return fail_hip(e, "plan upload");
    }
    unsigned char* base = (unsigned char*)plan->d_meta;
    plan->d_wins = (s2::WinMeta*)base;
    plan->d_samples = (s2::SampleMeta*)(base + sz_w);
    plan->d_text_sample = (int*)(base + sz_w + sz_s);
    plan->d_chunks = (s2::ChunkRef*)(base + sz_w + sz_s + sz_t);
    plan->d_items = (s2::AttnItem*)(base + sz_w + sz_s + sz_t + sz_c);
    plan->d_qkv_rows = (s2::QkvRow*)(base + sz_w + sz_s + sz_t + sz_c + sz_i);

    // Workspace layout: Q and K [heads][seg_total][d], V^T [heads][d][seg_total]
    // (bf16), the cos/sin table (with kRopePad entries of slack: the fused QKV
    // epilogue reads up to three entries past a row's last pair for pairs it
    // does not rotate), and fp32 text partials [rows][inner].
    const size_t qkv = align256((size_t)heads * plan->seg_total * d * 2);
    plan->off_q = 0;
    plan->off_k = qkv;
    plan->off_vt = 2 * qkv;
    plan->off_rope = 3 * qkv;
    plan->off_tpart =
        plan->off_rope +
        align256(sizeof(float2) * ((size_t)rope_pos * config->rope_pairs_per_axis + s2::kRopePad));
    plan->workspace_bytes = plan->off_tpart + align256(sizeof(float) * (size_t)tpart * inner);
    *out = plan;
    return S2_OK;
}

int s2_awa_plan_get_info(const s2_awa_plan* plan, s2_awa_plan_info* info) {
    if (!plan || !info) return S2_ERR_INVALID;
    info->batch = plan->batch;
    info->num_windows = plan->num_windows;
    info->video_tokens = plan->video_tokens;
    info->text_tokens = plan->text_tokens;
    info->workspace_bytes = plan->workspace_bytes;
    return S2_OK;
}

int s2_awa_plan_get_windows(const s2_awa_plan* plan, s2_window_slice* windows, int max_windows,
                            int* sample_window_count) {
    if (!plan) return S2_ERR_INVALID;
    if (windows) {
        if (max_windows < plan->num_windows) return fail(S2_ERR_INVALID, "window buffer too small");
        std::copy(plan->windows.begin(), plan->windows.end(), windows);
    }
    if (sample_window_count)
        std::copy(plan->sample_window_count.begin(), plan->sample_window_count.end(),
                  sample_window_count);
    return S2_OK;
}

int s2_awa_plan_destroy(s2_awa_plan* plan) {
    if (!plan) return S2_OK;
    hipError_t e = hipSuccess;
    if (plan->d_meta) e = hipFree(plan->d_meta);
    if (plan->d_rope_cache) {
        const hipError_t e2 = hipFree(plan->d_rope_cache);
        if (e == hipSuccess) e = e2;
    }
    delete plan;
    if (e != hipSuccess) return fail_hip(e, "hipFree");
    return S2_OK;
}

int s2_awa_plan_cache_rope(s2_awa_plan* plan, const float* rope_freqs, s2_stream_t stream) {
    if (!plan) return fail(S2_ERR_INVALID, "null plan");
    plan->rope_cache_src = nullptr;
    const int pairs = plan->config.rope_pairs_per_axis;
    if (!rope_freqs || pairs == 0) return S2_OK;   // cache cleared / nothing to cache
    if (!plan->d_rope_cache)
        S2_HIP(hipMalloc((void**)&plan->d_rope_cache,
                         sizeof(float2) * ((size_t)plan->rope_positions * pairs + s2::kRopePad)));
    S2_HIP(s2::launch_rope_table(rope_freqs, pairs, plan->rope_positions,
                                 (float2*)plan->d_rope_cache, (hipStream_t)stream));
    plan->rope_cache_src = rope_freqs;
    return S2_OK;
}

int s2_awa_plan_tables(const s2_awa_plan* plan, int* video_indices, int* inverse_video_indices,
                       int* local_positions, s2_stream_t stream) {
    if (!plan) return S2_ERR_INVALID;
    S2_HIP(s2::launch_awa_plan_tables(*plan, video_indices, inverse_video_indices, local_positions,
                                      (hipStream_t)stream));
    return S2_OK;
}

int s2_awa_forward(const s2_awa_plan* plan, const float* norm_weights, const float* rope_freqs,
                   const void* video_q, const void* video_k, const void* video_v,
                   long video_row_stride, const void* text_q, const void* text_k,
                   const void* text_v, long text_row_stride, s2_dtype in_dtype, void* out_video,
                   void* out_text, s2_dtype out_dtype, void* workspace, size_t workspace_bytes,
                   s2_stream_t stream) {
    if (!plan || !norm_weights || !video_q || !video_k || !video_v || !text_q || !text_k ||
        !text_v || !out_video || !out_text || !workspace)
        return fail(S2_ERR_INVALID, "null argument");
    // rows are read as 16-byte chunks
    if ((video_row_stride % 8) != 0 || (text_row_stride % 8) != 0)
        return fail(S2_ERR_INVALID, "row strides must be multiples of 8 elements");
    if ((plan->config.rope_pairs_per_axis > 0 && !rope_freqs))
        return fail(S2_ERR_INVALID, "missing rope frequencies");
    if (workspace_bytes < plan->workspace_bytes) return fail(S2_ERR_INVALID, "workspace too small");
    if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return fail(S2_ERR_INVALID, "unsupported dtype");
    const int inner = plan->config.heads * plan->config.head_dim;
    if (video_row_stride < inner || text_row_stride < inner || (video_row_stride % 8) != 0 ||
        (text_row_stride % 8) != 0)
        return fail(S2_ERR_INVALID, "row stride must be >= heads*head_dim and a multiple of 8");
    const size_t elem = dtype_bytes(in_dtype);
    const void* ins[6] = {video_q, video_k, video_v, text_q, text_k, text_v};
    for (const void* p : ins)
        if (((uintptr_t)p) % (8 * elem) != 0)
            return fail(S2_ERR_INVALID, "inputs must be aligned to 8 elements");
    if (((uintptr_t)out_video) % 16 != 0 || ((uintptr_t)out_text) % 16 != 0)
        return fail(S2_ERR_INVALID, "outputs must be 16-byte aligned");
    if (((uintptr_t)workspace) % 256 != 0) return fail(S2_ERR_INVALID, "workspace alignment");

    hipStream_t s = (hipStream_t)stream;
    unsigned char* ws = (unsigned char*)workspace;
    uint16_t* q = (uint16_t*)(ws + plan->off_q);
    uint16_t* k = (uint16_t*)(ws + plan->off_k);
    uint16_t* vt = (uint16_t*)(ws + plan->off_vt);
    const bool rope_cached = rope_freqs && rope_freqs == plan->rope_cache_src;
    float2* rope = rope_cached ? (float2*)plan->d_rope_cache : (float2*)(ws + plan->off_rope);
    float* tpart = (float*)(ws + plan->off_tpart);
    StageTimer& tm = stage_timer();
    if (tm.on) S2_HIP(hipEventRecord(tm.ev[0], s));
    if (plan->config.rope_pairs_per_axis > 0 && !rope_cached)
        S2_HIP(s2::launch_rope_table(rope_freqs, plan->config.rope_pairs_per_axis,
                                     plan->rope_positions, rope, s));
    if (tm.on) S2_HIP(hipEventRecord(tm.ev[1], s));
    S2_HIP(s2::launch_awa_prologue(*plan, video_q, video_k, video_v, video_row_stride, text_q,
                                   text_k, text_v, text_row_stride, (int)in_dtype, norm_weights, rope, q,
                                   k, vt, s));
    if (tm.on) S2_HIP(hipEventRecord(tm.ev[2], s));
    S2_HIP(s2::launch_awa_attention(*plan, q, k, vt, out_video, (int)out_dtype, tpart,
                                    norm_weights, s));
    if (tm.on) S2_HIP(hipEventRecord(tm.ev[3], s));
    S2_HIP(s2::launch_awa_text_pool(*plan, tpart, out_text, (int)out_dtype, s));
    if (tm.on) {
        S2_HIP(hipEventRecord(tm.ev[4], s));
        tm.recorded = true;
    }
    return S2_OK;
}

int s2_awa_qkv_forward(const s2_awa_plan* plan, const void* x_video, const void* x_text, int hidden,
                       const uint16_t* qkv_weight, const float* qkv_bias,
                       const float* norm_weights, const float* rope_freqs, void* out_video,
                       void* out_text, s2_dtype out_dtype, void* workspace,
                       size_t workspace_bytes, s2_stream_t stream) {
    if (!plan || !x_video || !x_text || !qkv_weight || !norm_weights || !out_video || !out_text ||
        !workspace)
        return fail(S2_ERR_INVALID, "null argument");
    const int d = plan->config.head_dim;
    const int inner = plan->config.heads * d;
    if ((d != 64 && d != 128) || inner % 256 != 0)
        return fail(S2_ERR_INVALID, "fused QKV path needs head_dim 64 or 128 and heads*head_dim % 256 == 0");
    if (hidden <= 0 || hidden % 64 != 0) return fail(S2_ERR_INVALID, "hidden must be a multiple of 64");
    if ((long)(plan->video_tokens + 1) * hidden * 2 > 0x7fffffffL ||
        (long)(plan->text_tokens + 1) * hidden * 2 > 0x7fffffffL)
        return fail(S2_ERR_INVALID, "activations beyond the 32-bit buffer offsets");
    if (plan->config.rope_pairs_per_axis > 0 && !rope_freqs)
        return fail(S2_ERR_INVALID, "missing rope frequencies");
    if (workspace_bytes < plan->workspace_bytes) return fail(S2_ERR_INVALID, "workspace too small");
    if (!dtype_ok(out_dtype)) return fail(S2_ERR_INVALID, "unsupported dtype");
    if (((uintptr_t)x_video) % 16 != 0 || ((uintptr_t)x_text) % 16 != 0 ||
        ((uintptr_t)qkv_weight) % 16 != 0 || ((uintptr_t)out_video) % 16 != 0 ||
        ((uintptr_t)out_text) % 16 != 0)
        return fail(S2_ERR_INVALID, "inputs and outputs must be 16-byte aligned");
    if (((uintptr_t)workspace) % 256 != 0) return fail(S2_ERR_INVALID, "workspace alignment");

    hipStream_t s = (hipStream_t)stream;
    unsigned char* ws = (unsigned char*)workspace;
    uint16_t* q = (uint16_t*)(ws + plan->off_q);
    uint16_t* k = (uint16_t*)(ws + plan->off_k);
    uint16_t* vt = (uint16_t*)(ws + plan->off_vt);
    const bool rope_cached = rope_freqs && rope_freqs == plan->rope_cache_src;
    float2* rope = rope_cached ? (float2*)plan->d_rope_cache : (float2*)(ws + plan->off_rope);
    float* tpart = (float*)(ws + plan->off_tpart);
    StageTimer& tm = stage_timer();
    if (tm.on) S2_HIP(hipEventRecord(tm.ev[0], s));
    if (plan->config.rope_pairs_per_axis > 0 && !rope_cached)
        S2_HIP(s2::launch_rope_table(rope_freqs, plan->config.rope_pairs_per_axis,
                                     plan->rope_positions, rope, s));
    if (tm.on) S2_HIP(hipEventRecord(tm.ev[1], s));
    S2_HIP(s2::launch_awa_qkv(*plan, (const uint16_t*)x_video, (const uint16_t*)x_text, hidden,
                              qkv_weight, qkv_bias, norm_weights, rope, q, k, vt, s));
    if (tm.on) S2_HIP(hipEventRecord(tm.ev[2], s));
    S2_HIP(s2::launch_awa_attention(*plan, q, k, vt, out_video, (int)out_dtype, tpart,
                                    norm_weights, s));
    if (tm.on) S2_HIP(hipEventRecord(tm.ev[3], s));
    S2_HIP(s2::launch_awa_text_pool(*plan, tpart, out_text, (int)out_dtype, s));
    if (tm.on) {
        S2_HIP(hipEventRecord(tm.ev[4], s));
        tm.recorded = true;
    }
    return S2_OK;
}

int s2_awa_stage_timing(int enable) {
    StageTimer& tm = stage_timer();
    if (enable && !tm.created) {
        for (hipEvent_t& e : tm.ev) S2_HIP(hipEventCreate(&e));
        tm.created = true;
    }
    tm.on = enable != 0;
    tm.recorded = false;
    return S2_OK;
}

int s2_awa_stage_times(float stage_ms[4]) {
    if (!stage_ms) return fail(S2_ERR_INVALID, "null argument");
    StageTimer& tm = stage_timer();
    if (!tm.created || !tm.recorded) return fail(S2_ERR_INVALID, "no timed forward recorded");
    S2_HIP(hipEventSynchronize(tm.ev[4]));
    for (int i = 0; i < 4; ++i) S2_HIP(hipEventElapsedTime(&stage_ms[i], tm.ev[i], tm.ev[i + 1]));
    return S2_OK;
}

int s2_cast_f32_to_bf16(const float* src, uint16_t* dst, size_t count, s2_stream_t stream) {
    if (count && (!src || !dst)) return S2_ERR_INVALID;
    S2_HIP(s2::launch_cast_f32_bf16(src, dst, count, (hipStream_t)stream));
    return S2_OK;
}

int s2_swiglu_pack_weight(const uint16_t* gate, const uint16_t* up, const float* gate_bias,
                          const float* up_bias, int n, int k, uint16_t* packed,
                          float* packed_bias, s2_stream_t stream) {
    if (!gate || !up || !packed || n <= 0 || k <= 0 || n % 128 != 0 ||
        ((gate_bias != 0) != (up_bias != 0)) || ((gate_bias != 0) != (packed_bias != 0)))
        return fail(S2_ERR_INVALID, "invalid SwiGLU weight pair");
    hipStream_t s = (hipStream_t)stream;
    const size_t rows = 128, row_bytes = (size_t)k * 2;
    for (int j = 0; j < n / 128; ++j) {
        S2_HIP(hipMemcpyAsync(packed + (size_t)(2 * j) * rows * k, gate + (size_t)j * rows * k,
                              rows * row_bytes, hipMemcpyDeviceToDevice, s));
        S2_HIP(hipMemcpyAsync(packed + (size_t)(2 * j + 1) * rows * k, up + (size_t)j * rows * k,
                              rows * row_bytes, hipMemcpyDeviceToDevice, s));
        if (gate_bias) {
            S2_HIP(hipMemcpyAsync(packed_bias + (size_t)(2 * j) * rows, gate_bias + (size_t)j * rows,
                                  rows * 4, hipMemcpyDeviceToDevice, s));
            S2_HIP(hipMemcpyAsync(packed_bias + (size_t)(2 * j + 1) * rows, up_bias + (size_t)j * rows,
                                  rows * 4, hipMemcpyDeviceToDevice, s));
        }
    }
    return S2_OK;
}

int s2_gelu(const void* x, void* y, size_t count, s2_dtype dtype, s2_stream_t stream) {
    if (count && (!x || !y)) return fail(S2_ERR_INVALID, "null argument");
    if (!dtype_ok(dtype)) return fail(S2_ERR_INVALID, "unsupported dtype");
    S2_HIP(s2::launch_gelu(x, y, count, (int)dtype, (hipStream_t)stream));
    return S2_OK;
}

int s2_cast_bf16_to_f32(const uint16_t* src, float* dst, size_t count, s2_stream_t stream) {
    if (count && (!src || !dst)) return S2_ERR_INVALID;
    S2_HIP(s2::launch_cast_bf16_f32(src, dst, count, (hipStream_t)stream));
    return S2_OK;
}

// Argument checks of the SharedLinear entry points (shared_linear.cpp:87-90
// for the widths; the alignment and k rules are this build's).
static int linear_args_ok(const void* x_video, int m_video, const void* x_text, int m_text,
                          s2_dtype x_dtype, const uint16_t* weight, int n, int k, int activation,
                          void* y_video, void* y_text, s2_dtype y_dtype) {
    if (n <= 0 || k <= 0 || m_video < 0 || m_text < 0 || !weight)
        return fail(S2_ERR_INVALID, "invalid linear shape");
    if ((m_video > 0 && (!x_video || !y_video)) || (m_text > 0 && (!x_text || !y_text)))
        return fail(S2_ERR_INVALID, "null stream pointer");
    if (k % 8 != 0) return fail(S2_ERR_INVALID, "k must be a multiple of 8");
    if (activation != S2_ACT_NONE && activation != S2_ACT_GELU && activation != S2_ACT_SWIGLU)
        return fail(S2_ERR_INVALID, "unknown activation");
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype)) return fail(S2_ERR_INVALID, "unsupported dtype");
    if (activation == S2_ACT_SWIGLU &&
        (x_dtype != S2_DTYPE_BF16 || k % 64 != 0 || n % 128 != 0 || (long)256 * k * 2 > 0x7fffffffL))
        return fail(S2_ERR_INVALID, "SwiGLU needs bf16 activations, k % 64 == 0 and n % 128 == 0");
    const size_t xe = dtype_bytes(x_dtype);
    if (((uintptr_t)x_video) % (8 * xe) || ((uintptr_t)x_text) % (8 * xe) ||
        ((uintptr_t)weight) % 16 || ((uintptr_t)y_video) % 16 || ((uintptr_t)y_text) % 16)
        return fail(S2_ERR_INVALID, "operands must be 16-byte aligned");
    return S2_OK;
}

int s2_shared_linear_forward(const void* x_video, int m_video, const void* x_text, int m_text,
                             s2_dtype x_dtype, const uint16_t* weight, const float* bias, int n,
                             int k, int activation, void* y_video, void* y_text, s2_dtype y_dtype,
                             s2_stream_t stream) {
    const int ret = linear_args_ok(x_video, m_video, x_text, m_text, x_dtype, weight, n, k,
                                   activation, y_video, y_text, y_dtype);
    if (ret != S2_OK) return ret;
    S2_HIP(s2::launch_shared_linear(x_video, m_video, x_text, m_text, (int)x_dtype, weight, bias,
                                    n, k, activation, y_video, y_text, (int)y_dtype,
                                    (hipStream_t)stream));
    return S2_OK;
}

int s2_shared_linear_forward_noalloc(const void* x_video, int m_video, const void* x_text,
                                     int m_text, s2_dtype x_dtype, const uint16_t* weight,
                                     const float* bias, int n, int k, int activation,
                                     void* y_video, void* y_text, s2_dtype y_dtype,
                                     s2_stream_t stream) {
    const int ret = linear_args_ok(x_video, m_video, x_text, m_text, x_dtype, weight, n, k,
                                   activation, y_video, y_text, y_dtype);
    if (ret != S2_OK) return ret;
    const hipError_t e = s2::launch_shared_linear_noalloc(
        x_video, m_video, x_text, m_text, (int)x_dtype, weight, bias, n, k, activation, y_video,
        y_text, (int)y_dtype, (hipStream_t)stream);
    if (e == hipErrorNotSupported)
        return fail(S2_ERR_INVALID,
                    "split-k tail needs more workgroups than the static scratch holds (256)");
    S2_HIP(e);
    return S2_OK;
}

/* ---- DiT frontend and tail, sampler step ---------------------------------- */

int s2_patchify_video(const float* video, long tokens, const int* video_shapes, int batch,
                      float* patches, s2_stream_t stream) {
    long nt = 0, np = 0;
    if (!video_shapes_ok(video_shapes, batch, &nt, &np) || nt != tokens)
        return fail(S2_ERR_INVALID, "video shapes do not match the token count");
    if (!video || !patches) return fail(S2_ERR_INVALID, "null pointer");
    if (!aligned(video, 8) || !aligned(patches, 8))
        return fail(S2_ERR_INVALID, "video and patches must be 8-byte aligned");
    long in_off = 0, out_off = 0;
    for (int b = 0; b < batch; ++b) {
        const int t = video_shapes[3 * b], h = video_shapes[3 * b + 1], w = video_shapes[3 * b + 2];
        S2_HIP(s2::launch_patchify(video + in_off * 33, t, h, w, patches + out_off * 132,
                                   (hipStream_t)stream));
        in_off += (long)t * h * w;
        out_off += (long)t * (h / 2) * (w / 2);
    }
    return S2_OK;
}

int s2_latent_patches(const float* latent, const float* condition, long channel_stride,
                      int frames, int height, int width, float* patches, s2_stream_t stream) {
    const int shape[3] = {frames, height, width};
    long nt = 0, np = 0;
    if (!video_shapes_ok(shape, 1, &nt, &np)) return fail(S2_ERR_INVALID, "invalid latent shape");
    if (channel_stride < nt) return fail(S2_ERR_INVALID, "channel stride below the token count");
    if (!latent || !condition || !patches) return fail(S2_ERR_INVALID, "null pointer");
    S2_HIP(s2::launch_latent_patches(latent, condition, channel_stride, frames, height, width,
                                     patches, (hipStream_t)stream));
    return S2_OK;
}

int s2_timestep_embedding(const float* timesteps, int count, float* embedding,
                          s2_stream_t stream) {
    if (count <= 0 || !timesteps) return fail(S2_ERR_INVALID, "no timesteps");
    if (!embedding) return fail(S2_ERR_INVALID, "null pointer");
    S2_HIP(s2::launch_timestep_embedding(timesteps, count, embedding, (hipStream_t)stream));
    return S2_OK;
}

int s2_unpatchify_prediction(const float* patches, long patch_count, const int* video_shapes,
                             int batch, float* prediction, s2_stream_t stream) {
    long nt = 0, np = 0;
    if (!video_shapes_ok(video_shapes, batch, &nt, &np) || np != patch_count)
        return fail(S2_ERR_INVALID, "video shapes do not match the patch count");
    if (!patches || !prediction) return fail(S2_ERR_INVALID, "null pointer");
    if (!aligned(patches, 16) || !aligned(prediction, 16))
        return fail(S2_ERR_INVALID, "patches and prediction must be 16-byte aligned");
    long in_off = 0, out_off = 0;
    for (int b = 0; b < batch; ++b) {
        const int t = video_shapes[3 * b], h = video_shapes[3 * b + 1], w = video_shapes[3 * b + 2];
        S2_HIP(s2::launch_unpatchify(patches + in_off * 64, t, h, w, prediction + out_off * 16,
                                     (hipStream_t)stream));
        in_off += (long)t * (h / 2) * (w / 2);
        out_off += (long)t * h * w;
    }
    return S2_OK;
}

int s2_apply_cfg(const float* positive, const float* negative, long count, float scale,
                 float rescale, float* output, s2_stream_t stream) {
    if (count < 0) return fail(S2_ERR_INVALID, "negative count");
    if (count == 0) return S2_OK;
    if (!positive || !negative || !output) return fail(S2_ERR_INVALID, "null pointer");
    if (!aligned(positive, 16) || !aligned(negative, 16) || !aligned(output, 16))
        return fail(S2_ERR_INVALID, "operands must be 16-byte aligned");
    S2_HIP(s2::launch_cfg(positive, negative, count, scale, rescale, output, (hipStream_t)stream));
    return S2_OK;
}

int s2_euler_step(float* latent, long channel_stride, const float* prediction, long tokens,
                  float delta, s2_stream_t stream) {
    if (tokens < 0 || channel_stride < tokens)
        return fail(S2_ERR_INVALID, "token count exceeds the channel stride");
    if (tokens == 0) return S2_OK;
    if (!latent || !prediction) return fail(S2_ERR_INVALID, "null pointer");
    if (!aligned(prediction, 16)) return fail(S2_ERR_INVALID, "prediction must be 16-byte aligned");
    S2_HIP(s2::launch_euler(latent, channel_stride, prediction, tokens, delta,
                            (hipStream_t)stream));
    return S2_OK;
}

int s2_denoise_update(const float* positive_patches, const float* negative_patches, int frames,
                      int height, int width, float cfg_scale, float cfg_rescale, float delta,
                      float* latent, long channel_stride, s2_stream_t stream) {
    const int shape[3] = {frames, height, width};
    long nt = 0, np = 0;
    if (!video_shapes_ok(shape, 1, &nt, &np)) return fail(S2_ERR_INVALID, "invalid latent shape");
    if (channel_stride < nt) return fail(S2_ERR_INVALID, "channel stride below the token count");
    if (!positive_patches || !latent) return fail(S2_ERR_INVALID, "null pointer");
    if (!aligned(positive_patches, 16) || !aligned(negative_patches, 16))
        return fail(S2_ERR_INVALID, "patches must be 16-byte aligned");
    S2_HIP(s2::launch_denoise_update(positive_patches, negative_patches, frames, height, width,
                                     cfg_scale, cfg_rescale, delta, latent, channel_stride,
                                     (hipStream_t)stream));
    return S2_OK;
}

/* ---- DiT block: norm and AdaSingle modulation ---------------------------- */

namespace {

// The two streams' per-sample row counts as kernel row tables; the stream
// pointers and strides are checked against the rows they must cover.
int ada_rows(int hidden, int batch, const int* video_rows, const int* text_rows,
             s2::AdaRows* rows) {
    if (hidden <= 0 || hidden % 4 != 0 || hidden > s2::kAdaMaxDim)
        return fail(S2_ERR_INVALID, "hidden size must be a positive multiple of 4, at most 4096");
    if (batch <= 0 || batch > s2::kAdaMaxBatch)
        return fail(S2_ERR_INVALID, "batch must be 1..64");
    if (!video_rows) return fail(S2_ERR_INVALID, "null row counts");
    memset(rows, 0, sizeof(*rows));
    rows->batch = batch;
    long v = 0, t = 0;
    for (int b = 0; b < batch; ++b) {
        const int tr = text_rows ? text_rows[b] : 0;
        if (video_rows[b] < 0 || tr < 0) return fail(S2_ERR_INVALID, "negative row count");
        v += video_rows[b];
        t += tr;
        if (v + t > INT_MAX) return fail(S2_ERR_INVALID, "too many rows");
        rows->end[b] = (int)v;
        rows->end[s2::kAdaMaxBatch + b] = (int)t;
    }
    rows->video_rows = (int)v;
    rows->text_rows = (int)t;
    return S2_OK;
}

// a stream of `n` rows: pointer, row stride (elements) and alignment
bool ada_stream_ok(const void* p, int n, long stride, int hidden, s2_dtype dt) {
    if (n == 0) return true;
    return p && stride >= hidden && stride % 4 == 0 && aligned(p, dt == S2_DTYPE_F32 ? 16 : 8);
}

bool ada_vec_ok(const float* p) { return !p || aligned(p, 16); }

}  // namespace

int s2_dit_ada_in(int hidden, float epsilon, int batch, const int* video_rows,
                  const int* text_rows, const void* x_video, const void* x_text, s2_dtype x_dtype,
                  long x_stride, const float* shift, const float* scale, const float* video_shift,
                  const float* video_scale, const float* text_shift, const float* text_scale,
                  void* out_video, void* out_text, s2_dtype out_dtype, long out_stride,
                  s2_stream_t stream) {
    s2::AdaInArgs a = {};
    const int rc = ada_rows(hidden, batch, video_rows, text_rows, &a.rows);
    if (rc != S2_OK) return rc;
    if (!dtype_ok(x_dtype) || !dtype_ok(out_dtype)) return fail(S2_ERR_INVALID, "unsupported dtype");
    if (!(epsilon >= 0.f)) return fail(S2_ERR_INVALID, "epsilon must be >= 0");
    const int nv = a.rows.video_rows, nt = a.rows.text_rows;
    if (!ada_stream_ok(x_video, nv, x_stride, hidden, x_dtype) ||
        !ada_stream_ok(x_text, nt, x_stride, hidden, x_dtype) ||
        !ada_stream_ok(out_video, nv, out_stride, hidden, out_dtype) ||
        !ada_stream_ok(out_text, nt, out_stride, hidden, out_dtype))
        return fail(S2_ERR_INVALID, "stream pointer, row stride (>= hidden, multiple of 4) or alignment");
    if (!shift || !scale || !aligned(shift, 16) || !aligned(scale, 16) || !ada_vec_ok(video_shift) ||
        !ada_vec_ok(video_scale) || !ada_vec_ok(text_shift) || !ada_vec_ok(text_scale))
        return fail(S2_ERR_INVALID, "modulation vectors must be non-null (shift, scale) and 16-byte aligned");
    a.x[0] = x_video;
    a.x[1] = x_text;
    a.x_stride = x_stride;
    a.x_kind = (int)x_dtype;
    a.out[0] = out_video;
    a.out[1] = out_text;
    a.out_stride = out_stride;
    a.out_kind = (int)out_dtype;
    a.dim = hidden;
    a.eps = epsilon;
    a.shift_a = shift;
    a.scale_a = scale;
    a.shift_b[0] = video_shift;
    a.shift_b[1] = text_shift;
    a.scale_b[0] = video_scale;
    a.scale_b[1] = text_scale;
    S2_HIP(s2::launch_ada_in(a, (hipStream_t)stream));
    return S2_OK;
}

int s2_dit_ada_out(int hidden, int batch, const int* video_rows, const int* text_rows,
                   const void* x_video, const void* x_text, s2_dtype x_dtype, long x_stride,
                   const void* y_video, const void* y_text, s2_dtype y_dtype, long y_stride,
                   const float* gate, const float* video_gate, const float* text_gate,
                   void* out_video, void* out_text, long out_stride, s2_stream_t stream) {
    s2::AdaOutArgs a = {};
    const int rc = ada_rows(hidden, batch, video_rows, text_rows, &a.rows);
    if (rc != S2_OK) return rc;
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype)) return fail(S2_ERR_INVALID, "unsupported dtype");
    const int nv = a.rows.video_rows, nt = a.rows.text_rows;
    if (!ada_stream_ok(x_video, nv, x_stride, hidden, x_dtype) ||
        !ada_stream_ok(x_text, nt, x_stride, hidden, x_dtype) ||
        !ada_stream_ok(y_video, nv, y_stride, hidden, y_dtype) ||
        !ada_stream_ok(y_text, nt, y_stride, hidden, y_dtype) ||
        !ada_stream_ok(out_video, nv, out_stride, hidden, x_dtype) ||
        !ada_stream_ok(out_text, nt, out_stride, hidden, x_dtype))
        return fail(S2_ERR_INVALID, "stream pointer, row stride (>= hidden, multiple of 4) or alignment");
    // in place needs the output rows to be the input rows
    if ((out_video == x_video && nv > 0 && out_stride != x_stride) ||
        (out_text == x_text && nt > 0 && out_stride != x_stride))
        return fail(S2_ERR_INVALID, "in-place output must keep the residual's row stride");
    if (!gate || !aligned(gate, 16) || !ada_vec_ok(video_gate) || !ada_vec_ok(text_gate))
        return fail(S2_ERR_INVALID, "gate vectors must be non-null (gate) and 16-byte aligned");
    a.x[0] = x_video;
    a.x[1] = x_text;
    a.x_stride = x_stride;
    a.x_kind = (int)x_dtype;
    a.y[0] = y_video;
    a.y[1] = y_text;
    a.y_stride = y_stride;
    a.y_kind = (int)y_dtype;
    a.out[0] = out_video;
    a.out[1] = out_text;
    a.out_stride = out_stride;
    a.dim = hidden;
    a.gate_a = gate;
    a.gate_b[0] = video_gate;
    a.gate_b[1] = text_gate;
    S2_HIP(s2::launch_ada_out(a, (hipStream_t)stream));
    return S2_OK;
}

int s2_shared_linear_residual(const void* x_video, int m_video, const void* x_text, int m_text,
                              const uint16_t* weight, const float* bias, int n, int k, int batch,
                              const int* video_rows, const int* text_rows, const void* res_video,
                              const void* res_text, s2_dtype res_dtype, const float* gate,
                              const float* video_gate, const float* text_gate, void* out_video,
                              void* out_text, s2_stream_t stream) {
    s2::LinearResidual r = {};
    const int rc = ada_rows(n, batch, video_rows, text_rows, &r.rows);
    if (rc != S2_OK) return rc;
    if (r.rows.video_rows != m_video || r.rows.text_rows != m_text)
        return fail(S2_ERR_INVALID, "row counts do not sum to m_video / m_text");
    if (!weight || k <= 0 || k % 64 != 0 || n % 8 != 0 || (long)256 * k * 2 > 0x7fffffffL)
        return fail(S2_ERR_INVALID, "weight, k (multiple of 64) or n (multiple of 8)");
    if (!dtype_ok(res_dtype)) return fail(S2_ERR_INVALID, "unsupported dtype");
    const bool vid = m_video > 0, txt = m_text > 0;
    if ((vid && (!x_video || !res_video || !out_video)) || (txt && (!x_text || !res_text || !out_text)))
        return fail(S2_ERR_INVALID, "null stream pointer");
    if ((vid && (!aligned(x_video, 16) || !aligned(res_video, 16) || !aligned(out_video, 16))) ||
        (txt && (!aligned(x_text, 16) || !aligned(res_text, 16) || !aligned(out_text, 16))) ||
        !aligned(weight, 16))
        return fail(S2_ERR_INVALID, "operands must be 16-byte aligned");
    if (!gate || !aligned(gate, 16) || !ada_vec_ok(video_gate) || !ada_vec_ok(text_gate))
        return fail(S2_ERR_INVALID, "gate vectors must be non-null (gate) and 16-byte aligned");
    r.x[0] = res_video;
    r.x[1] = res_text;
    r.out[0] = out_video;
    r.out[1] = out_text;
    r.x_kind = (int)res_dtype;
    r.gate = gate;
    r.gate_s[0] = video_gate;
    r.gate_s[1] = text_gate;
    S2_HIP(s2::launch_shared_linear_residual((const uint16_t*)x_video, m_video,
                                             (const uint16_t*)x_text, m_text, weight, bias, n, k,
                                             r, (hipStream_t)stream));
    return S2_OK;
}

int s2_dit_ada_out_in(int hidden, int batch, const int* video_rows, const int* text_rows,
                      const void* x_video, const void* x_text, s2_dtype x_dtype, long x_stride,
                      const void* y_video, const void* y_text, s2_dtype y_dtype, long y_stride,
                      const float* gate, const float* video_gate, const float* text_gate,
                      void* out_video, void* out_text, long out_stride, float epsilon,
                      const float* shift, const float* scale, const float* video_shift,
                      const float* video_scale, const float* text_shift, const float* text_scale,
                      void* h_video, void* h_text, s2_dtype h_dtype, long h_stride,
                      s2_stream_t stream) {
    s2::AdaOutArgs a = {};
    const int rc = ada_rows(hidden, batch, video_rows, text_rows, &a.rows);
    if (rc != S2_OK) return rc;
    if (!dtype_ok(x_dtype) || !dtype_ok(y_dtype) || !dtype_ok(h_dtype))
        return fail(S2_ERR_INVALID, "unsupported dtype");
    if (!(epsilon >= 0.f)) return fail(S2_ERR_INVALID, "epsilon must be >= 0");
    const int nv = a.rows.video_rows, nt = a.rows.text_rows;
    if (!ada_stream_ok(x_video, nv, x_stride, hidden, x_dtype) ||
        !ada_stream_ok(x_text, nt, x_stride, hidden, x_dtype) ||
        !ada_stream_ok(y_video, nv, y_stride, hidden, y_dtype) ||
        !ada_stream_ok(y_text, nt, y_stride, hidden, y_dtype) ||
        !ada_stream_ok(out_video, nv, out_stride, hidden, x_dtype) ||
        !ada_stream_ok(out_text, nt, out_stride, hidden, x_dtype) ||
        !ada_stream_ok(h_video, nv, h_stride, hidden, h_dtype) ||
        !ada_stream_ok(h_text, nt, h_stride, hidden, h_dtype))
        return fail(S2_ERR_INVALID, "stream pointer, row stride (>= hidden, multiple of 4) or alignment");
    if ((out_video == x_video && nv > 0 && out_stride != x_stride) ||
        (out_text == x_text && nt > 0 && out_stride != x_stride))
        return fail(S2_ERR_INVALID, "in-place output must keep the residual's row stride");
    if (!gate || !aligned(gate, 16) || !ada_vec_ok(video_gate) || !ada_vec_ok(text_gate) ||
        !shift || !scale || !aligned(shift, 16) || !aligned(scale, 16) || !ada_vec_ok(video_shift) ||
        !ada_vec_ok(video_scale) || !ada_vec_ok(text_shift) || !ada_vec_ok(text_scale))
        return fail(S2_ERR_INVALID, "modulation vectors must be non-null (gate, shift, scale) and 16-byte aligned");
    a.x[0] = x_video;
    a.x[1] = x_text;
    a.x_stride = x_stride;
    a.x_kind = (int)x_dtype;
    a.y[0] = y_video;
    a.y[1] = y_text;
    a.y_stride = y_stride;
    a.y_kind = (int)y_dtype;
    a.out[0] = out_video;
    a.out[1] = out_text;
    a.out_stride = out_stride;
    a.dim = hidden;
    a.gate_a = gate;
    a.gate_b[0] = video_gate;
    a.gate_b[1] = text_gate;
    a.norm = 1;
    a.h[0] = h_video;
    a.h[1] = h_text;
    a.h_stride = h_stride;
    a.h_kind = (int)h_dtype;
    a.eps = epsilon;
    a.shift_a = shift;
    a.scale_a = scale;
    a.shift_b[0] = video_shift;
    a.shift_b[1] = text_shift;
    a.scale_b[0] = video_scale;
    a.scale_b[1] = text_scale;
    S2_HIP(s2::launch_ada_out(a, (hipStream_t)stream));
    return S2_OK;
}

/* ---- DecomposedConv3D ---------------------------------------------------- */

int s2_conv3d_output_shape(const s2_conv3d_config* config, int frames, int height, int width,
                           int memory_frames, int out_shape[3]) {
    int to = 0, ho = 0, wo = 0;
    if (!out_shape || !conv3d_out(config, frames, height, width, memory_frames, &to, &ho, &wo))
        return fail(S2_ERR_INVALID, "invalid DecomposedConv3D configuration or input shape");
    out_shape[0] = to;
    out_shape[1] = ho;
    out_shape[2] = wo;
    return S2_OK;
}

int s2_conv3d_packed_weight_bytes(const s2_conv3d_config* config, size_t* bytes) {
    if (!bytes || !conv3d_config_ok(config)) return fail(S2_ERR_INVALID, "invalid configuration");
    const s2::Conv3dShape s = conv3d_shape(config);
    *bytes = (size_t)s.cout * s2::conv3d_kp(s) * 2;
    return S2_OK;
}

int s2_conv3d_pack_weights(const s2_conv3d_config* config, const float* weights, void* packed,
                           s2_stream_t stream) {
    if (!conv3d_config_ok(config)) return fail(S2_ERR_INVALID, "invalid configuration");
    if (!weights || !packed) return fail(S2_ERR_INVALID, "null pointer");
    S2_HIP(s2::launch_conv3d_pack_weights(weights, conv3d_shape(config), (uint16_t*)packed,
                                          (hipStream_t)stream));
    return S2_OK;
}

int s2_conv3d_memory_bytes(const s2_conv3d_config* config, int height, int width, size_t* bytes,
                           int* frames) {
    if (!bytes || !frames || !conv3d_config_ok(config) || height <= 0 || width <= 0)
        return fail(S2_ERR_INVALID, "invalid configuration");
    const int cache = std::max(config->kernel_t - config->stride_t, 0);
    *frames = cache;
    if (s2::conv3d_narrow(conv3d_shape(config)))   // partial sums of two output frames
        *bytes = (size_t)2 * config->num_output * height * width * 4;
    else
        *bytes = (size_t)cache * height * width * s2::conv3d_cpad(config->num_input) * 2;
    return S2_OK;
}

int s2_conv3d_workspace_bytes(const s2_conv3d_config* config, int frames, int height, int width,
                              int memory_frames, size_t* bytes) {
    return s2_conv3d_workspace_bytes_padded(config, frames, height, width, 0, 0, memory_frames,
                                            bytes);
}

int s2_conv3d_workspace_bytes_padded(const s2_conv3d_config* config, int frames, int height,
                                     int width, int pad_right, int pad_bottom, int memory_frames,
                                     size_t* bytes) {
    int to, ho, wo;
    if (pad_right < 0 || pad_bottom < 0) return fail(S2_ERR_INVALID, "negative padding");
    // the output extent (and the partial tiles) follow the padded frames,
    // the staged frames the unpadded input
    if (!bytes || !conv3d_out(config, frames, height + pad_bottom, width + pad_right,
                              memory_frames, &to, &ho, &wo))
        return fail(S2_ERR_INVALID, "invalid DecomposedConv3D configuration or input shape");
    if (s2::conv3d_narrow(conv3d_shape(config))) {
        // a copy of the memory, for a forward that rewrites it in place
        if (pad_right || pad_bottom)
            return fail(S2_ERR_INVALID, "layers of at most 3 output channels take no extra padding");
        *bytes = align256((size_t)2 * config->num_output * height * width * 4);
        return S2_OK;
    }
    *bytes = align256((size_t)(frames + memory_frames) * height * width *
                      s2::conv3d_cpad(config->num_input) * 2);
    // fp32 partial tiles when the k loop is split into ranges
    const s2::Conv3dShape s = conv3d_shape(config);
    const long mo = (long)to * ho * wo;
    const int splits = s2::conv3d_k_split(s, mo, wo);
    if (splits > 1) *bytes += align256((size_t)splits * s.cout * mo * 4);
    return S2_OK;
}

int s2_conv3d_forward(const s2_conv3d_config* config, const void* packed_weights,
                      const float* bias, const void* input, s2_dtype in_dtype, int frames,
                      int height, int width, long in_cstep, const void* memory, int memory_frames,
                      void* output, s2_dtype out_dtype, long out_cstep, void* next_memory,
                      void* workspace, size_t workspace_bytes, s2_stream_t stream) {
    return s2_conv3d_forward_padded(config, packed_weights, bias, input, in_dtype, frames, height,
                                    width, in_cstep, 0, 0, memory, memory_frames, output,
                                    out_dtype, out_cstep, next_memory, workspace,
                                    workspace_bytes, stream);
}

int s2_conv3d_forward_padded(const s2_conv3d_config* config, const void* packed_weights,
                             const float* bias, const void* input, s2_dtype in_dtype, int frames,
                             int height, int width, long in_cstep, int pad_right, int pad_bottom,
                             const void* memory, int memory_frames, void* output,
                             s2_dtype out_dtype, long out_cstep, void* next_memory,
                             void* workspace, size_t workspace_bytes, s2_stream_t stream) {
    const int mem = memory ? memory_frames : 0;
    int to, ho, wo;
    if (pad_right < 0 || pad_bottom < 0) return fail(S2_ERR_INVALID, "negative padding");
    // the zero padding on the right and bottom only lengthens the output: the
    // kernel already reads every pixel outside the image as zero
    if (!conv3d_out(config, frames, height + pad_bottom, width + pad_right, mem, &to, &ho, &wo))
        return fail(S2_ERR_INVALID, "invalid DecomposedConv3D configuration or input shape");
    if (memory && memory_frames <= 0) return fail(S2_ERR_INVALID, "memory without frames");
    if (!packed_weights || !input || !output) return fail(S2_ERR_INVALID, "null pointer");
    if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return fail(S2_ERR_INVALID, "unsupported dtype");
    const long plane_in = (long)height * width;
    if (in_cstep < (long)frames * plane_in || in_cstep % 4 != 0 || !aligned(input, 16))
        return fail(S2_ERR_INVALID, "input channel stride or alignment");
    if (out_cstep < (long)to * ho * wo) return fail(S2_ERR_INVALID, "output channel stride");
    const s2::Conv3dShape s = conv3d_shape(config);
    if (s2::conv3d_narrow(s)) {
        if (pad_right || pad_bottom)
            return fail(S2_ERR_INVALID, "layers of at most 3 output channels take no extra padding");
        if (mem && mem != 2) return fail(S2_ERR_INVALID, "the memory holds 2 frames");
        if ((memory && !aligned(memory, 4)) || (next_memory && !aligned(next_memory, 4)))
            return fail(S2_ERR_INVALID, "memory alignment");
        const int prefix = mem > 0 ? mem : config->head_frames;
        const size_t mem_bytes = (size_t)2 * s.cout * plane_in * 4;
        // workgroups of different output frames run at once when there are
        // more than kNarrowSlots of them (with the memory's two): a memory
        // rewritten in place is read from a copy then
        const float* mem_in = (const float*)memory;
        if (mem && next_memory && to + 2 > s2::kNarrowSlots &&
            (const uint8_t*)next_memory < (const uint8_t*)memory + mem_bytes &&
            (const uint8_t*)memory < (const uint8_t*)next_memory + mem_bytes) {
            if (!workspace || !aligned(workspace, 256) || workspace_bytes < mem_bytes)
                return fail(S2_ERR_INVALID, "workspace too small");
            S2_HIP(hipMemcpyAsync(workspace, memory, mem_bytes, hipMemcpyDeviceToDevice,
                                  (hipStream_t)stream));
            mem_in = (const float*)workspace;
        }
        S2_HIP(s2::launch_conv3d_narrow(s, input, (int)in_dtype, in_cstep, frames, height, width,
                                        prefix, mem, to, (const uint16_t*)packed_weights, bias,
                                        output, (int)out_dtype, out_cstep, mem_in,
                                        (float*)next_memory, (hipStream_t)stream));
        return S2_OK;
    }
    if (!workspace) return fail(S2_ERR_INVALID, "null pointer");
    if (!aligned(workspace, 256)) return fail(S2_ERR_INVALID, "workspace alignment");
    const size_t frame_elems = (size_t)plane_in * s.cpad;
    const size_t frame_bytes = frame_elems * 2;
    if ((size_t)(mem + frames) * frame_bytes > workspace_bytes)
        return fail(S2_ERR_INVALID, "workspace too small");
    const int prefix = mem > 0 ? mem : config->head_frames;
    const int padded = frames + prefix;
    const int cache = config->kernel_t - config->stride_t;
    const bool want_memory = next_memory && cache > 0;
    if (want_memory && cache > padded) return fail(S2_ERR_INVALID, "too few frames for the memory");
    const long max_span = (long)(0x7fffffffL / (long)frame_bytes);
    if (max_span < (long)(config->kernel_t - 1) * config->dilation_t + 1)
        return fail(S2_ERR_INVALID, "one output frame reads more than 2 GiB of staged input");
    hipStream_t st = (hipStream_t)stream;

    // Padded frame p is frame v = max(p - shift, 0) of [memory | input].  The
    // kernel reads the memory frames straight from `memory` when each 8-row
    // DMA group stays inside one output frame; otherwise they are copied in
    // front of the staged input.
    const int shift = prefix - mem;
    const bool direct = mem > 0 && (long)mem <= max_span &&
                        (s2::conv3d_halo_ok(s, wo) || (s.cpad >= 64 && ((long)ho * wo) % 8 == 0));
    const int kmem = direct ? mem : 0;
    const int lead = mem - kmem;
    uint16_t* staged = (uint16_t*)workspace;
    if (lead > 0)
        S2_HIP(hipMemcpyAsync(staged, memory, (size_t)lead * frame_bytes, hipMemcpyDeviceToDevice, st));
    // The next memory is the last `cache` padded frames.  The staging pass
    // writes the input frames among them (all of them, or the last `frames`
    // after cache - frames earlier ones, copied below), unless the kernel
    // still has to read `memory` and next_memory overlaps it.
    const uint8_t* mlo = (const uint8_t*)memory;
    const uint8_t* nlo = (const uint8_t*)next_memory;
    const bool overlap = memory && next_memory && nlo < mlo + (size_t)mem * frame_bytes &&
                         mlo < nlo + (size_t)std::max(cache, 0) * frame_bytes;
    const bool tail_in_stage = want_memory && (kmem == 0 || !overlap);
    const int early = std::max(cache - frames, 0);   // next-memory frames from before the input
    S2_HIP(s2::launch_conv3d_stage(input, (int)in_dtype, in_cstep, s.cin, (long)frames * plane_in,
                                   s.cpad, staged + (size_t)lead * frame_elems,
                                   tail_in_stage ? (uint16_t*)next_memory + (size_t)early * frame_elems
                                                 : nullptr,
                                   (long)std::max(frames - cache, 0) * plane_in, st));
    // fp32 partial tiles of a k loop split into ranges, after the staged
    // frames, when the workspace holds them (s2_conv3d_workspace_bytes counts
    // them; a smaller workspace runs the whole k loop per tile instead)
    float* part = nullptr;
    {
        const size_t need = align256((size_t)(mem + frames) * frame_bytes);
        const long mo = (long)to * ho * wo;
        const int splits = s2::conv3d_k_split(s, mo, wo);
        if (splits > 1 && workspace_bytes >= need + (size_t)splits * s.cout * mo * 4)
            part = (float*)((uint8_t*)workspace + need);
    }
    auto vframe = [&](long p) { return (int)std::max(p - shift, 0L); };
    const long reach = (long)(config->kernel_t - 1) * config->dilation_t;
    for (int t0 = 0; t0 < to;) {
        // as many output frames as keep the staged frames they read under 2 GiB
        const int lo = std::max(vframe((long)t0 * config->stride_t) - kmem, 0);
        int n = 1;
        while (t0 + n < to &&
               vframe((long)(t0 + n) * config->stride_t + reach) - kmem - lo + 1 <= max_span)
            ++n;
        const int hi = vframe((long)(t0 + n - 1) * config->stride_t + reach) - kmem;
        const size_t span = hi >= lo ? (size_t)(hi - lo + 1) * frame_bytes : 0;
        S2_HIP(s2::launch_conv3d(s, (const uint16_t*)memory, kmem, (size_t)kmem * frame_bytes,
                                 staged + (size_t)lo * frame_elems, span, lo, shift, height, width,
                                 ho, wo, t0, n, (const uint16_t*)packed_weights, bias, output,
                                 (int)out_dtype, out_cstep, part, st));
        t0 += n;
    }
    if (want_memory) {
        // frames in ascending order: frame f comes from v >= f, so a memory
        // buffer reused as next_memory is read before it is overwritten
        for (int f = 0; f < (tail_in_stage ? early : cache); ++f) {
            const int v = vframe((long)padded - cache + f);
            const uint8_t* src = v < kmem ? mlo + (size_t)v * frame_bytes
                                          : (const uint8_t*)(staged + (size_t)(v - kmem) * frame_elems);
            uint8_t* dst = (uint8_t*)next_memory + (size_t)f * frame_bytes;
            if (src != dst)
                S2_HIP(hipMemcpyAsync(dst, src, frame_bytes, hipMemcpyDeviceToDevice, st));
        }
    }
    return S2_OK;
}

/* ---- VAEChunkedMHA ------------------------------------------------------- */

int s2_mha_weight_bytes(const s2_mha_config* config, size_t* bytes) {
    if (!bytes || !mha_config_ok(config)) return fail(S2_ERR_INVALID, "invalid MHA configuration");
    *bytes = mha_layout(config).total;
    return S2_OK;
}

int s2_mha_prepare_weights(const s2_mha_config* config, const float* wq, const float* bq,
                           const float* wk, const float* bk, const float* wv, const float* bv,
                           const float* wo, const float* bo, void* prepared,
                           s2_stream_t stream) {
    if (!mha_config_ok(config)) return fail(S2_ERR_INVALID, "invalid MHA configuration");
    if (!wq || !bq || !wk || !bk || !wv || !bv || !wo || !bo || !prepared)
        return fail(S2_ERR_INVALID, "null pointer");
    if (!aligned(prepared, 256)) return fail(S2_ERR_INVALID, "prepared weights alignment");
    const MhaWeights m = mha_layout(config);
    uint8_t* base = (uint8_t*)prepared;
    hipStream_t st = (hipStream_t)stream;
    const long mat = (long)config->embed_dim * config->qdim;
    S2_HIP(s2::launch_mha_weight(wq, mat, config->scale, (uint16_t*)(base + m.wq), st));
    S2_HIP(s2::launch_mha_weight(wk, mat, 1.f, (uint16_t*)(base + m.wk), st));
    S2_HIP(s2::launch_mha_weight(wv, mat, 1.f, (uint16_t*)(base + m.wv), st));
    S2_HIP(s2::launch_mha_weight(wo, mat, 1.f, (uint16_t*)(base + m.wo), st));
    S2_HIP(s2::launch_mha_bias(bq, config->embed_dim, config->scale, (float*)(base + m.bq), st));
    S2_HIP(s2::launch_mha_bias(bk, config->embed_dim, 1.f, (float*)(base + m.bk), st));
    S2_HIP(s2::launch_mha_bias(bv, config->embed_dim, 1.f, (float*)(base + m.bv), st));
    S2_HIP(s2::launch_mha_bias(bo, config->qdim, 1.f, (float*)(base + m.bo), st));
    return S2_OK;
}

int s2_mha_workspace_bytes(const s2_mha_config* config, int seq, size_t* bytes) {
    if (!bytes || !mha_config_ok(config) || seq <= 0)
        return fail(S2_ERR_INVALID, "invalid MHA configuration or sequence");
    *bytes = mha_work(config, seq).total;
    return S2_OK;
}

int s2_mha_forward(const s2_mha_config* config, const void* prepared, const void* x,
                   s2_dtype in_dtype, int seq, void* out, s2_dtype out_dtype, void* workspace,
                   size_t workspace_bytes, s2_stream_t stream) {
    if (!mha_config_ok(config) || seq <= 0)
        return fail(S2_ERR_INVALID, "invalid MHA configuration or sequence");
    if (!prepared || !x || !out || !workspace) return fail(S2_ERR_INVALID, "null pointer");
    if (!dtype_ok(in_dtype) || !dtype_ok(out_dtype)) return fail(S2_ERR_INVALID, "unsupported dtype");
    if (!aligned(x, 16) || !aligned(out, 16) || !aligned(workspace, 256) || !aligned(prepared, 256))
        return fail(S2_ERR_INVALID, "operand alignment");
    const MhaWork w = mha_work(config, seq);
    if (workspace_bytes < w.total) return fail(S2_ERR_INVALID, "workspace too small");
    const MhaWeights m = mha_layout(config);
    const int E = config->embed_dim, H = config->num_heads, D = E / H, Q = config->qdim;
    const uint8_t* wb = (const uint8_t*)prepared;
    uint8_t* ws = (uint8_t*)workspace;
    const uint16_t* wq = (const uint16_t*)(wb + m.wq);
    const uint16_t* wk = (const uint16_t*)(wb + m.wk);
    const uint16_t* wv = (const uint16_t*)(wb + m.wv);
    const uint16_t* wo = (const uint16_t*)(wb + m.wo);
    const float* bq = (const float*)(wb + m.bq);
    const float* bk = (const float*)(wb + m.bk);
    const float* bv = (const float*)(wb + m.bv);
    const float* bo = (const float*)(wb + m.bo);
    uint16_t* xp = (uint16_t*)(ws + w.xp);
    uint16_t* q = (uint16_t*)(ws + w.q);
    uint16_t* k = (uint16_t*)(ws + w.k);
    uint16_t* vt = (uint16_t*)(ws + w.vt);
    float* sc = (float*)(ws + w.s);
    uint16_t* p = (uint16_t*)(ws + w.p);
    uint16_t* oh = (uint16_t*)(ws + w.oh);
    uint16_t* o = H > 1 ? (uint16_t*)(ws + w.o) : oh;
    hipStream_t st = (hipStream_t)stream;
    constexpr int kBF = (int)S2_DTYPE_BF16, kF32 = (int)S2_DTYPE_F32;
    // x as bf16 rows, padded with zero rows to the 64-multiple extent of P V
    S2_HIP(s2::launch_mha_stage(x, (int)in_dtype, seq, w.lp, Q, xp, st));
    for (int h = 0; h < H; ++h) {
        const long wo_h = (long)h * D * Q;
        // q_h = x Wq_h^T + bq_h (scale folded in), k_h likewise: [lp][D]
        S2_HIP(s2::launch_shared_linear(xp, w.lp, nullptr, 0, kBF, wq + wo_h, bq + h * D, D, Q,
                                        S2_ACT_NONE, q, nullptr, kBF, st));
        S2_HIP(s2::launch_shared_linear(xp, w.lp, nullptr, 0, kBF, wk + wo_h, bk + h * D, D, Q,
                                        S2_ACT_NONE, k, nullptr, kBF, st));
        // v_h^T without its bias = Wv_h x^T: [D][lp], zero columns past seq
        S2_HIP(s2::launch_shared_linear(wv + wo_h, D, nullptr, 0, kBF, xp, nullptr, w.lp, Q,
                                        S2_ACT_NONE, vt, nullptr, kBF, st));
        // S = q_h k_h^T (already scaled): [seq][seq] fp32
        S2_HIP(s2::launch_shared_linear(q, seq, nullptr, 0, kBF, k, nullptr, seq, D, S2_ACT_NONE,
                                        sc, nullptr, kF32, st));
        S2_HIP(s2::launch_mha_softmax(sc, seq, seq, seq, w.lp, p, st));
        // o_h = P v_h + bv_h (the rows of P sum to one): [seq][D]
        S2_HIP(s2::launch_shared_linear(p, seq, nullptr, 0, kBF, vt, bv + h * D, D, w.lp,
                                        S2_ACT_NONE, oh, nullptr, kBF, st));
        if (H > 1) S2_HIP(s2::launch_mha_interleave(oh, seq, D, E, h, o, st));
    }
    // out = o Wo^T + bo: [seq][qdim]
    S2_HIP(s2::launch_shared_linear(o, seq, nullptr, 0, kBF, wo, bo, Q, E, S2_ACT_NONE, out,
                                    nullptr, (int)out_dtype, st));
    return S2_OK;
}

/* ---- VAEUpsample3D shuffle -------------------------------------------------- */

int s2_vae_pixel_shuffle(const void* packed, s2_dtype dtype, int channels, int frames,
                         int height, int width, long packed_cstep, int temporal_ratio,
                         int spatial_ratio, int remove_head, void* output, long out_cstep,
                         s2_stream_t stream) {
    if (channels <= 0 || frames <= 0 || height <= 0 || width <= 0 || temporal_ratio <= 0 ||
        spatial_ratio <= 0 || !dtype_ok(dtype))
        return fail(S2_ERR_INVALID, "invalid shuffle shape");
    const int out_t = frames * temporal_ratio - (remove_head ? 1 : 0);
    if (out_t <= 0) return fail(S2_ERR_INVALID, "no output frames");
    if (packed_cstep < (long)frames * height * width ||
        out_cstep < (long)out_t * height * spatial_ratio * width * spatial_ratio)
        return fail(S2_ERR_INVALID, "channel stride");
    if (!packed || !output) return fail(S2_ERR_INVALID, "null pointer");
    S2_HIP(s2::launch_vae_shuffle(packed, (int)dtype, packed_cstep, channels, frames, height,
                                  width, temporal_ratio, spatial_ratio, remove_head ? 1 : 0,
                                  output, out_cstep, (hipStream_t)stream));
    return S2_OK;
}

}  // extern "C"
