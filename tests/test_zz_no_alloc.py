"""s2_shared_linear_forward_noalloc: the SharedLinear forward with its split-k
scratch in a static device array instead of an allocation.  Same kernels
and split decisions as s2_shared_linear_forward, so the outputs are equal bit
for bit; they also meet the path's bar against the oracle (max-abs <= 2e-2,
cosine >= 0.9999).  Two calls in a row, the second smaller, both with a
split tail, so the second reuses what the first left in the array."""
import os

import numpy as np
import pytest

import oracle
from common import assert_close, bf16_round
from seedvr2_ncnn_amd import capi

pytestmark = pytest.mark.gpu
THREADS = min(16, os.cpu_count() or 1)

# (video rows, text rows, k, n, activation): the 720p out projection (860
# tiles: the last 82 split in three, 246 workgroups share them), then a
# smaller GEMM (36 tiles, each split in two) with GELU.
CALLS = [(21600, 64, 2560, 2560, 0), (2936, 64, 1024, 768, 1)]


def _inputs(seed, mv, mt, k, n):
    g = np.random.default_rng(seed)
    xv = bf16_round(g.standard_normal((mv, k), dtype=np.float32))
    xt = bf16_round(g.standard_normal((mt, k), dtype=np.float32))
    w = (0.02 * g.standard_normal((n, k), dtype=np.float32))
    b = (0.02 * g.standard_normal(n)).astype(np.float32)
    return g, xv, xt, w, b


def test_noalloc_matches_allocating_entry_point_twice():
    import torch
    assert capi.device_count() >= 1
    for i, (mv, mt, k, n, act) in enumerate(CALLS):
        print(f"noalloc call {i}: m={mv}+{mt} k={k} n={n} act={act}", flush=True)
        g, xv, xt, w, b = _inputs(100 + i, mv, mt, k, n)
        tv = torch.from_numpy(xv).cuda().to(torch.bfloat16)
        tt = torch.from_numpy(xt).cuda().to(torch.bfloat16)
        wb = capi.cast_f32_to_bf16(torch.from_numpy(w).cuda())
        tb = torch.from_numpy(b).cuda()
        got_v, got_t = capi.shared_linear(tv, tt, wb, tb, act, out_dtype=torch.float32,
                                          noalloc=True)
        ref_v, ref_t = capi.shared_linear(tv, tt, wb, tb, act, out_dtype=torch.float32)
        torch.cuda.synchronize()
        got_v, got_t = got_v.cpu().numpy(), got_t.cpu().numpy()
        np.testing.assert_array_equal(got_v, ref_v.cpu().numpy())
        np.testing.assert_array_equal(got_t, ref_t.cpu().numpy())
        rows = np.concatenate([np.arange(0, 2), g.integers(0, mv, 24),
                               np.arange(mv - 2, mv)]).astype(np.int32)
        assert_close(got_v[rows], oracle.linear(xv, w, b, act, rows=rows, threads=THREADS),
                     f"call {i} video rows")
        assert_close(got_t, oracle.linear(xt, w, b, act, threads=THREADS), f"call {i} text")


def test_noalloc_bf16_output_and_single_stream():
    """bf16 outputs, video stream only, no split (a full last wave): still
    equal to the allocating entry point."""
    import torch
    mv, k, n = 256 * 64, 512, 1024   # 64 x 4 = 256 tiles: one full wave
    g, xv, _, w, b = _inputs(7, mv, 0, k, n)
    tv = torch.from_numpy(xv).cuda().to(torch.bfloat16)
    wb = capi.cast_f32_to_bf16(torch.from_numpy(w).cuda())
    tb = torch.from_numpy(b).cuda()
    got, _ = capi.shared_linear(tv, None, wb, tb, 1, noalloc=True)
    ref, _ = capi.shared_linear(tv, None, wb, tb, 1)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.view(torch.int16).cpu().numpy(),
                                  ref.view(torch.int16).cpu().numpy())
