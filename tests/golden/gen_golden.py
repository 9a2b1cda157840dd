"""Writes the committed fixtures under tests/golden/ from the CPU oracle.

The reference ships no golden vectors for this path, so the fixtures are
produced by the oracle (pinned by tests/test_oracle.py and tests/test_plan.py)
and freeze its results so that later changes to either side are caught:

  plans.json       window lists and SHA-256 of video_indices,
                   inverse_video_indices and local_positions (little-endian
                   int32) for the benchmark grids, regular and shifted
  awa_tiny.npz     one small full-numeric AdaptiveWindowAttention case
                   (grids 2x4x6 + 1x3x5, 1 head x 64, 10 rope pairs, fp32)
  linear_tiny.npz  one small SharedLinear case with bias and GELU

Run: python tests/golden/gen_golden.py
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

import oracle  # noqa: E402
from common import make_awa_inputs, oracle_awa  # noqa: E402

PLAN_CASES = [
    ("grid_1x32x32_target_1x8x8", [(1, 32, 32)], (1, 8, 8)),
    ("grid_1x64x64_target_4x3x3", [(1, 64, 64)], (4, 3, 3)),
    ("grid_6x45x80_target_4x3x3", [(6, 45, 80)], (4, 3, 3)),
    ("batch_grid_5x9x16_2x30x17", [(5, 9, 16), (2, 30, 17)], (4, 3, 3)),
]


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a, dtype="<i4").tobytes()).hexdigest()


def plan_record(shapes, target, shifted):
    p = oracle.plan(shapes, target, shifted)
    return {
        "video_shapes": [list(s) for s in shapes],
        "target_windows": list(target),
        "shifted": int(shifted),
        "windows": p.windows.tolist(),
        "sample_window_count": p.sample_window_count.tolist(),
        "sha256_video_indices": sha(p.video_indices),
        "sha256_inverse_video_indices": sha(p.inverse_video_indices),
        "sha256_local_positions": sha(p.local_positions),
    }


def main():
    plans = {}
    for name, shapes, target in PLAN_CASES:
        for shifted in (0, 1):
            plans[f"{name}_{'shifted' if shifted else 'regular'}"] = plan_record(shapes, target, shifted)
    with open(os.path.join(HERE, "plans.json"), "w") as f:
        json.dump(plans, f, indent=1)

    shapes, text_lengths = [(2, 4, 6), (1, 3, 5)], [3, 2]
    heads, d, pairs, target = 1, 64, 10, (2, 2, 3)
    case = make_awa_inputs(2024, shapes, text_lengths, heads, d, pairs)
    out = {}
    for shifted in (0, 1):
        ov, ot = oracle_awa(case, heads, d, target, shifted, 1e-5, pairs, shapes, text_lengths, threads=1)
        out[f"out_video_{shifted}"] = ov
        out[f"out_text_{shifted}"] = ot
    np.savez(os.path.join(HERE, "awa_tiny.npz"), video=case["video"], text=case["text"],
             norms=case["norms"], freqs=case["freqs"], video_shapes=np.asarray(shapes, np.int32),
             text_lengths=np.asarray(text_lengths, np.int32),
             config=np.asarray([heads, d, pairs, *target], np.int32), **out)

    g = np.random.default_rng(7)
    xv = g.standard_normal((37, 24)).astype(np.float32)
    xt = g.standard_normal((5, 24)).astype(np.float32)
    w = (0.2 * g.standard_normal((40, 24))).astype(np.float32)
    b = (0.1 * g.standard_normal(40)).astype(np.float32)
    np.savez(os.path.join(HERE, "linear_tiny.npz"), x_video=xv, x_text=xt, weight=w, bias=b,
             y_video=oracle.linear(xv, w, b, 1), y_text=oracle.linear(xt, w, b, 1))


if __name__ == "__main__":
    main()
