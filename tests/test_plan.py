"""Window plan (build_adaptive_window_plan, adaptive_window_attention.cpp:565-655):
the oracle against closed forms and an independent model, then the product's
host plan (C-ABI s2_awa_plan_windows) and the layer-level
seedvr2::build_adaptive_window_plan against the oracle, bit-exact.  All CPU."""
import hashlib
import itertools
import json
import os

import numpy as np
import pytest

import oracle
import plan_model
from common import harness_plan
from seedvr2_ncnn_amd import capi

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a, dtype="<i4").tobytes()).hexdigest()


# ---- closed forms at the benchmark grids ------------------------------------

def _sizes(p, axis):
    lo, hi = {0: (1, 2), 1: (3, 4), 2: (5, 6)}[axis]
    return [int(w[hi] - w[lo]) for w in p.windows]


def test_grid_32x32_target_1x8x8_is_16_windows_of_8x8():
    p = oracle.plan([(1, 32, 32)], (1, 8, 8), 0)
    assert len(p.windows) == 16 and set(p.windows[:, 8]) == {64}


def test_grid_64x64_window_sets():
    reg = oracle.plan([(1, 64, 64)], (4, 3, 3), 0)
    assert len(reg.windows) == 16 and set(reg.windows[:, 8]) == {400, 80, 16}
    assert sorted(set(_sizes(reg, 1))) == [4, 20]
    sh = oracle.plan([(1, 64, 64)], (4, 3, 3), 1)
    assert len(sh.windows) == 16 and set(sh.windows[:, 8]) == {100, 140, 196, 200, 280, 400}


def test_grid_6x45x80_regular_and_shifted():
    reg = oracle.plan([(6, 45, 80)], (4, 3, 3), 0)
    assert len(reg.windows) == 27 and set(reg.windows[:, 8]) == {810, 780}
    assert set(_sizes(reg, 0)) == {2} and set(_sizes(reg, 1)) == {15} and set(_sizes(reg, 2)) == {27, 26}
    sh = oracle.plan([(6, 45, 80)], (4, 3, 3), 1)
    assert len(sh.windows) == 64
    # per-axis slices t {1,2,2,1}, h {7,15,15,8}, w {13,27,27,13}
    ts = [int(w[2] - w[1]) for w in sh.windows[:4]]
    hs = [int(w[4] - w[3]) for w in sh.windows[0:16:4]]
    ws = [int(w[6] - w[5]) for w in sh.windows[0:64:16]]
    assert (ts, hs, ws) == ([1, 2, 2, 1], [7, 15, 15, 8], [13, 27, 27, 13])
    assert set(sh.windows[:, 8]) == {91, 104, 182, 189, 195, 208, 216, 378, 390, 405, 432, 810}


def test_loop_order_is_w_outer_then_h_then_t():
    p = oracle.plan([(6, 45, 80)], (4, 3, 3), 0)
    keys = [(w[5], w[3], w[1]) for w in p.windows]
    assert keys == sorted(keys)


# ---- brute force against the independent model ---------------------------------

SMALL = list(itertools.product([1, 2, 5], [1, 3, 8, 13], [1, 4, 11, 21]))
TARGETS = [(1, 1, 1), (4, 3, 3), (2, 5, 2), (1, 8, 8)]


def _check_same(a, b):
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1], b[1])
    np.testing.assert_array_equal(a[2], b[2])
    np.testing.assert_array_equal(a[3], b[3])
    np.testing.assert_array_equal(a[4], b[4])


@pytest.mark.parametrize("shifted", [0, 1])
def test_oracle_plan_equals_independent_model(shifted):
    for shape in SMALL:
        for target in TARGETS:
            p = oracle.plan([shape], target, shifted)
            m = plan_model.plan([shape], target, shifted)
            _check_same((p.windows, p.sample_window_count, p.video_indices, p.inverse_video_indices,
                         p.local_positions), m)


def test_oracle_plan_is_a_permutation_with_batches():
    shapes = [(3, 17, 29), (1, 8, 8), (7, 45, 80)]
    for shifted in (0, 1):
        p = oracle.plan(shapes, (4, 3, 3), shifted)
        lv = sum(t * h * w for t, h, w in shapes)
        assert p.windows[:, 8].sum() == lv
        assert np.array_equal(np.sort(p.video_indices), np.arange(lv))
        assert np.array_equal(p.inverse_video_indices[p.video_indices], np.arange(lv))
        assert p.sample_window_count.sum() == len(p.windows)


def test_oracle_rejects_bad_shapes():
    with pytest.raises(ValueError):
        oracle.plan([(0, 4, 4)], (4, 3, 3), 0)
    with pytest.raises(ValueError):
        oracle.plan([(1, 4, 4)], (0, 3, 3), 0)


# ---- product plans vs the oracle, bit-exact -------------------------------------

PRODUCT_CASES = [([s], t) for s in SMALL[::3] for t in TARGETS] + [
    ([(1, 32, 32)], (1, 8, 8)), ([(1, 64, 64)], (4, 3, 3)), ([(6, 45, 80)], (4, 3, 3)),
    ([(21, 90, 160)], (4, 3, 3)), ([(45, 30, 17)], (4, 3, 3)),
    ([(3, 17, 29), (1, 8, 8), (7, 45, 80)], (4, 3, 3)),
]


@pytest.mark.parametrize("shifted", [0, 1])
def test_capi_host_windows_equal_oracle(shifted):
    for shapes, target in PRODUCT_CASES:
        p = oracle.plan(shapes, target, shifted)
        wins, counts, tokens = capi.plan_windows(shapes, target, shifted)
        np.testing.assert_array_equal(np.asarray(wins, np.int32).reshape(-1, 9), p.windows)
        np.testing.assert_array_equal(counts, p.sample_window_count)
        assert tokens == len(p.video_indices)


@pytest.mark.parametrize("shifted", [0, 1])
def test_layer_build_adaptive_window_plan_equals_oracle(shifted):
    for shapes, target in PRODUCT_CASES:
        p = oracle.plan(shapes, target, shifted)
        h = harness_plan(shapes, target, shifted)
        _check_same(h, (p.windows, p.sample_window_count, p.video_indices, p.inverse_video_indices,
                        p.local_positions))


def test_capi_plan_rejects_bad_shapes():
    with pytest.raises(capi.S2Error) as e:
        capi.plan_windows([(1, 0, 4)], (4, 3, 3), 0)
    assert e.value.code == capi.S2_ERR_INVALID
    with pytest.raises(capi.S2Error):
        capi.plan_windows([(1, 4, 4)], (4, -1, 3), 1)


# ---- committed fixtures ------------------------------------------------------------

def _golden():
    with open(os.path.join(GOLDEN, "plans.json")) as f:
        return json.load(f)


def test_fixture_plans_match_oracle_and_product():
    for name, rec in _golden().items():
        shapes = [tuple(s) for s in rec["video_shapes"]]
        p = oracle.plan(shapes, rec["target_windows"], rec["shifted"])
        assert p.windows.tolist() == rec["windows"], name
        assert p.sample_window_count.tolist() == rec["sample_window_count"], name
        assert sha(p.video_indices) == rec["sha256_video_indices"], name
        assert sha(p.inverse_video_indices) == rec["sha256_inverse_video_indices"], name
        assert sha(p.local_positions) == rec["sha256_local_positions"], name
        wins, counts, _ = capi.plan_windows(shapes, rec["target_windows"], rec["shifted"])
        assert [list(w) for w in wins] == rec["windows"], name
        h = harness_plan(shapes, rec["target_windows"], rec["shifted"])
        assert sha(h[2]) == rec["sha256_video_indices"], name
        assert sha(h[3]) == rec["sha256_inverse_video_indices"], name
        assert sha(h[4]) == rec["sha256_local_positions"], name
