// Device-side window index math shared by the attention and the fused QKV
// projection kernels: partition-local token r of a window -> its window-local
// (t, h, w) coordinates and its source token, in append_slice's t,h,w
// row-major order (src/seedvr2/adaptive_window_attention.cpp:462-471).
#pragma once

#include <hip/hip_runtime.h>

#include "awa_plan.h"

namespace s2 {

struct TokenCoord {
    int lt, lh, lw;
    long src;
};

// a / b for 0 <= a < 2^22, b > 0: the fp32 quotient is within one of the
// true one, and one correction step makes it exact (cheaper than the
// integer division sequence)
__device__ __forceinline__ int div_small(int a, int b) {
    int q = (int)((float)a * __builtin_amdgcn_rcpf((float)b));
    const int r = a - q * b;
    q += (r >= b) - (r < 0);
    return q;
}

__device__ __forceinline__ TokenCoord window_token(const WinMeta& w, int r) {
    TokenCoord c;
    const int plane = w.eh * w.ew;
    c.lt = div_small(r, plane);
    const int rem = r - c.lt * plane;
    c.lh = div_small(rem, w.ew);
    c.lw = rem - c.lh * w.ew;
    c.src = (long)w.tok_off +
            ((long)(w.t0 + c.lt) * w.grid_h + (w.h0 + c.lh)) * w.grid_w + (w.w0 + c.lw);
    return c;
}

}  // namespace s2
