"""An independent Python statement of SeedVR2's adaptive window plan, used to
pin the C oracle (not a transcription of it: window bounds come from the
closed integer form below, the walk is a product of per-axis lists).

For an axis of n tokens with window extent e:
  regular: windows [i*e, min((i+1)*e, n)) for i = 0 .. ceil(n/e)-1
  shifted (e < n): the grid is offset by half a window, so window i covers
      [max(floor((2i-1)e/2), 0), min(floor((2i+1)e/2), n)),  i = 0 .. ceil((2n-1)/(2e))
      (for i = 0 the lower bound is clamped to 0, which equals C's truncation
      of -e/2 toward zero followed by max(., 0)); empty windows are dropped
  shifted (e >= n): one window [0, n)
The extent is ceil(min(t,30)/Tt) on t, ceil(round(h*s)/Th) and
ceil(round(w*s)/Tw) with s = sqrt(3600/(h*w)) and round half to even.
Windows are listed w outer, h, t inner; tokens in a window t,h,w row-major.
"""
from __future__ import annotations

import math

import numpy as np


def axis_windows(n: int, e: int, shifted: bool):
    if not shifted or e >= n:
        count = -(-n // e) if not shifted else 1
        out = [(i * e, min((i + 1) * e, n)) for i in range(count)]
    else:
        count = -(-(2 * n - 1) // (2 * e)) + 1
        out = []
        for i in range(count):
            lo = 0 if i == 0 else ((2 * i - 1) * e) // 2
            hi = min(((2 * i + 1) * e) // 2, n)
            out.append((lo, hi))
    return [(lo, hi) for lo, hi in out if hi > lo]


def extents(t, h, w, target):
    s = math.sqrt(3600.0 / (h * w))
    rh = round(h * s)   # Python round: half to even
    rw = round(w * s)
    return (-(-min(t, 30) // target[0]), -(-rh // target[1]), -(-rw // target[2]))


def plan(video_shapes, target, shifted):
    windows, counts, indices, positions = [], [], [], []
    offset = 0
    for b, (t, h, w) in enumerate(video_shapes):
        et, eh, ew = extents(t, h, w, target)
        n0 = len(windows)
        for (w0, w1) in axis_windows(w, ew, shifted):
            for (h0, h1) in axis_windows(h, eh, shifted):
                for (t0, t1) in axis_windows(t, et, shifted):
                    part = len(indices)
                    tt, hh, ww = np.meshgrid(np.arange(t0, t1), np.arange(h0, h1), np.arange(w0, w1),
                                             indexing="ij")
                    src = offset + (tt * h + hh) * w + ww
                    indices.extend(src.ravel().tolist())
                    positions.extend(np.stack([tt - t0, hh - h0, ww - w0], -1).reshape(-1, 3).tolist())
                    windows.append((b, t0, t1, h0, h1, w0, w1, part, (t1 - t0) * (h1 - h0) * (w1 - w0)))
        counts.append(len(windows) - n0)
        offset += t * h * w
    idx = np.asarray(indices, np.int32)
    inv = np.full(offset, -1, np.int32)
    inv[idx] = np.arange(len(idx), dtype=np.int32)
    return (np.asarray(windows, np.int32).reshape(-1, 9), np.asarray(counts, np.int32), idx, inv,
            np.asarray(positions, np.int32).reshape(-1, 3))
