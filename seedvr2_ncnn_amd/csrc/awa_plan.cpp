// Host window list of the adaptive 3-D window plan.
//
// Restates build_adaptive_window_plan (src/seedvr2/adaptive_window_attention.cpp:
// 565-655).  The reference walks three nested loops (w outer, h, t inner) and
// skips empty windows inside them; an empty bound on one axis empties every
// window in that row, so the walk is the same as taking the product of three
// per-axis lists of non-empty (lo, hi) bounds in w, h, t order, which is how
// it is written here.  Only O(windows) work happens on the host; the
// per-token index tables are computed on the device from these bounds.
#include <algorithm>
#include <cmath>
#include <utility>

#include "awa_plan.h"

namespace s2 {
namespace {

// Window extent on one axis: ceil(size / target) (:434-437, :586-588).
int ceil_div(int extent, int window) { return (extent + window - 1) / window; }

// Non-empty window bounds along one axis of length n with extent e.
//   regular: [i*e, min((i+1)*e, n)) for i < ceil(n/e)                (:601-606)
//   shifted, e < n: shift s = 0.5, count ceil((n-s)/e)+1, bounds
//     [max(int((i-s)*e), 0), min(int((i-s+1)*e), n)) with C truncation  (:592-598, :611-613)
//   shifted, e >= n: one window [0, n).
void axis_bounds(int n, int e, bool shifted, std::vector<std::pair<int, int> >& out) {
    out.clear();
    if (!shifted) {
        for (int i = 0, count = ceil_div(n, e); i < count; ++i) {
            const int lo = i * e;
            const int hi = std::min(lo + e, n);
            if (hi > lo) out.emplace_back(lo, hi);
        }
        return;
    }
    const double s = e < n ? 0.5 : 0.0;
    const int count = s > 0.0 ? static_cast<int>(std::ceil((n - s) / e)) + 1 : 1;
    for (int i = 0; i < count; ++i) {
        const int lo = std::max(static_cast<int>((i - s) * e), 0);
        const int hi = std::min(static_cast<int>((i - s + 1.0) * e), n);
        if (hi > lo) out.emplace_back(lo, hi);
    }
}

}  // namespace

int build_window_slices(const int* video_shapes, int batch, const int target_windows[3],
                        bool shifted, std::vector<s2_window_slice>& windows,
                        std::vector<int>& sample_window_count, int& video_tokens) {
    windows.clear();
    sample_window_count.clear();
    video_tokens = 0;
    if (batch <= 0 || !video_shapes || !target_windows) return S2_ERR_INVALID;
    if (target_windows[0] <= 0 || target_windows[1] <= 0 || target_windows[2] <= 0)
        return S2_ERR_INVALID;
    std::vector<std::pair<int, int> > bt, bh, bw;
    long long offset = 0;
    for (int sample = 0; sample < batch; ++sample) {
        const int t = video_shapes[3 * sample + 0];
        const int h = video_shapes[3 * sample + 1];
        const int w = video_shapes[3 * sample + 2];
        if (t <= 0 || h <= 0 || w <= 0) return S2_ERR_INVALID;
        // Resolution-adaptive extents (:583-588): the grid is rescaled to
        // about 3600 tokens per frame, rounded half-to-even like Python round().
        const double scale = std::sqrt(3600.0 / static_cast<double>(h * w));
        const int resized_h = static_cast<int>(std::nearbyint(h * scale));
        const int resized_w = static_cast<int>(std::nearbyint(w * scale));
        const int et = ceil_div(std::min(t, 30), target_windows[0]);
        const int eh = ceil_div(resized_h, target_windows[1]);
        const int ew = ceil_div(resized_w, target_windows[2]);
        if (et <= 0 || eh <= 0 || ew <= 0) return S2_ERR_INVALID;
        axis_bounds(t, et, shifted, bt);
        axis_bounds(h, eh, shifted, bh);
        axis_bounds(w, ew, shifted, bw);
        int count = 0;
        for (const auto& xw : bw)
            for (const auto& xh : bh)
                for (const auto& xt : bt) {
                    s2_window_slice s;
                    s.sample_index = sample;
                    s.t0 = xt.first; s.t1 = xt.second;
                    s.h0 = xh.first; s.h1 = xh.second;
                    s.w0 = xw.first; s.w1 = xw.second;
                    s.partition_offset = static_cast<int>(offset);
                    s.token_count = (s.t1 - s.t0) * (s.h1 - s.h0) * (s.w1 - s.w0);
                    offset += s.token_count;
                    windows.push_back(s);
                    ++count;
                }
        sample_window_count.push_back(count);
        const long long tokens = static_cast<long long>(t) * h * w;
        video_tokens += static_cast<int>(tokens);
        if (static_cast<long long>(video_tokens) > 0x7fffffffLL) return S2_ERR_INVALID;
    }
    // The windows tile each sample exactly once (the reference's permutation
    // check, :642-653): the per-axis bounds are contiguous and cover [0, n).
    if (offset != video_tokens) return S2_ERR_PLAN;
    return S2_OK;
}

}  // namespace s2
