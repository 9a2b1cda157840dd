// Window-plan data shared by the host plan builder and the gfx950 kernels.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <vector>

#include "seedvr2_hip.h"

namespace s2 {

// Per-window record the kernels read (one 64-byte line per window).  The
// per-token gather/scatter index is recomputed from these integers on the
// device: partition-local token r of a window maps to
//   lt = r / (eh*ew), lh = (r / ew) % eh, lw = r % ew
//   source = tok_off + ((t0+lt)*grid_h + h0+lh)*grid_w + w0+lw
// which is append_slice's t,h,w row-major walk
// (adaptive_window_attention.cpp:462-471).
struct WinMeta {
    int sample;
    int t0, h0, w0;
    int et, eh, ew;       // window extents t1-t0, h1-h0, w1-w0
    int part_off;         // WindowSlice::partition_offset
    int n_video;          // WindowSlice::token_count
    int seq;              // n_video + text_len (the SDPA sequence length)
    int seg_off;          // first row of this window's padded Q/K/V segment
    int text_off;         // first text row of the sample
    int text_len;
    int grid_h, grid_w;   // sample token grid h, w
    int tok_off;          // first video row of the sample
    int tpart_off;        // first row of this window's text partials
    int grow_off;         // first row of this window's video tokens in the row space of
                          // the fused QKV projection (even; see s2_awa_plan::qkv_text_row)
    int ts_row;           // first workspace row of the sample's text tokens (staged once
                          // per sample, a multiple of kSegAlign)
};
static_assert(sizeof(WinMeta) == 76, "WinMeta layout");

// Per-sample record for the text mean-pool.
struct SampleMeta {
    int first_window;
    int num_windows;
    int text_off;
    int text_len;
    float pool_scale;     // 1.f / num_windows (adaptive_window_attention.cpp:963)
};

// One attention work item: (window, 128-row query tile, head).
struct AttnItem {
    int window;
    int q_row0;
    int head;
    int pad_;
};

// A window's segment (its video rows) and a sample's text staging rows are
// padded to this multiple: whole 32-key tiles and 64-row prologue chunks.
constexpr int kSegAlign = 64;

// Entries of slack after a cos/sin table: a reader may fetch the three
// entries after any (position, pair) entry without using them.
constexpr int kRopePad = 4;

// MI355X has 8 XCDs; workgroups are dealt to them round-robin.
constexpr int kNumXcd = 8;

// One row of the fused QKV projection's row space: its source row (video or
// text token; -1 for a gap or padding row), its workspace row, its RoPE
// position and its kind (0 none, 1 video, 2 text).  A row of a window's run
// past the window's tokens (a gap) keeps the workspace row that follows the
// window's video rows, so that V^T key pairs stay contiguous.
struct QkvRow {
    int src;
    int dest;
    int pos01;   // position axis 0 | axis 1 << 16
    int pos2;    // position axis 2 | kind << 16
};

// One prologue work item: 64 rows of one window's sequence -- video rows of
// the window (row0 < n_video), or text rows of its sample (row0 >= n_video,
// written once per sample to the staging rows).
struct ChunkRef {
    int window;
    int row0;
};

// Host window list (restates adaptive_window_attention.cpp:565-655).
int build_window_slices(const int* video_shapes, int batch, const int target_windows[3],
                        bool shifted, std::vector<s2_window_slice>& windows,
                        std::vector<int>& sample_window_count, int& video_tokens);

}  // namespace s2

// The opaque plan handle behind s2_awa_plan*.
struct s2_awa_plan {
    s2_awa_config config;
    int batch = 0;
    int num_windows = 0;
    int video_tokens = 0;
    int text_tokens = 0;
    int device = 0;
    std::vector<int> video_shapes;          // [batch][3]
    std::vector<int> text_lengths;          // [batch]
    std::vector<s2_window_slice> windows;
    std::vector<int> sample_window_count;
    std::vector<s2::WinMeta> win_meta;
    // device metadata, one allocation
    void* d_meta = nullptr;
    s2::WinMeta* d_wins = nullptr;
    s2::SampleMeta* d_samples = nullptr;
    int* d_text_sample = nullptr;           // [text_tokens] -> sample
    s2::ChunkRef* d_chunks = nullptr;               // prologue chunks {window, row0}
    s2::AttnItem* d_items = nullptr;        // [kNumXcd][slots_per_xcd]
    int num_chunks = 0;
    int slots_per_xcd = 0;
    int max_window_tokens = 0;
    int rope_positions = 0;                 // rows of the cos/sin table
    long seg_total = 0;                     // row pitch of the Q/K/V^T workspace: the padded
                                            // window segments (video rows), then the
                                            // samples' padded text staging rows
    long seg_text = 0;                      // first text staging row (each text token's
                                            // Q/K/V^T is written there once)
    // Row space of the fused QKV projection (s2_awa_qkv_forward): the video
    // tokens in window order, each window's run starting at an even row
    // (WinMeta::grow_off), then from qkv_text_row (a multiple of 8) to
    // qkv_rows the text tokens, each sample's run starting at an even row.
    int qkv_text_row = 0;
    int qkv_rows = 0;
    s2::QkvRow* d_qkv_rows = nullptr;       // [qkv_rows rounded up to 256]
    int text_partial_rows = 0;
    // (cos, sin) pairs [rope_positions][pairs] of the frequencies at
    // rope_cache_src, filled by s2_awa_plan_cache_rope; forwards given that
    // pointer read it instead of recomputing the table in their workspace
    float* d_rope_cache = nullptr;
    const float* rope_cache_src = nullptr;
    // workspace layout (byte offsets)
    size_t off_q = 0, off_k = 0, off_vt = 0, off_rope = 0, off_tpart = 0;
    size_t workspace_bytes = 0;
};
