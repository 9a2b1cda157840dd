"""The DiT block's norm and AdaSingle modulation on the GPU (s2_dit_ada_in,
s2_dit_ada_out; the block graph's modulation inputs,
src/seedvr2/seedvr2_dit.cpp:441-448, 734-738) against the CPU oracle.

ada_in sums the squares in fp32 on the device (double in the oracle), so
fp32 outputs are compared at the path's bar (max-abs <= 2e-2, cosine >=
0.9999) and within 2e-6 of the output scale, and 16-bit outputs within one
bf16 / fp16 rounding of each value.  ada_out performs the same fp32 operations in the
same order as the oracle and is compared bit-exact.  Row counts are chosen
so that workgroups of 16 rows straddle sample and stream boundaries, and
include empty samples."""
import numpy as np
import pytest

import oracle
from common import assert_close

pytestmark = pytest.mark.gpu

CASES = [
    # hidden, video rows per sample, text rows per sample
    (2560, [37, 0, 129], [5, 3, 0]),
    (3072, [70], [64]),
    (96, [1, 2, 3, 4], [4, 3, 2, 1]),
    (1000, [16, 16], None),
    (4096, [9, 23], [7, 0]),
]


def _torch():
    import torch
    return torch


def _data(hidden, vr, tr, seed):
    g = np.random.default_rng(seed)
    b = len(vr)
    nv, nt = sum(vr), sum(tr or [])
    xv = (g.standard_normal((nv, hidden)) * g.uniform(0.2, 5, (nv, 1))).astype(np.float32)
    xt = (g.standard_normal((nt, hidden)) * g.uniform(0.2, 5, (nt, 1))).astype(np.float32)
    mod = {k: (g.standard_normal((b, hidden)) * 0.5 + (1.0 if k == "scale" else 0.0)).astype(np.float32)
           for k in ("shift", "scale", "gate")}
    own = {f"{s}_{k}": (0.1 * g.standard_normal(hidden)).astype(np.float32)
           for s in ("video", "text") for k in ("shift", "scale", "gate")}
    return xv, xt, mod, own


def _dev(a, dtype=None):
    torch = _torch()
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


def _stored(a, dtype):
    """the values a tensor of `dtype` holds for a"""
    torch = _torch()
    return torch.from_numpy(a).to(dtype).float().numpy()


@pytest.mark.parametrize("hidden,vr,tr", CASES)
@pytest.mark.parametrize("x_dt,out_dt", [("f32", "bf16"), ("bf16", "f32"), ("f16", "f16"),
                                         ("f32", "f32")])
def test_ada_in_matches_oracle(hidden, vr, tr, x_dt, out_dt):
    torch = _torch()
    from seedvr2_ncnn_amd import capi
    dts = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
    xv, xt, mod, own = _data(hidden, vr, tr, hidden + len(vr))
    xv, xt = _stored(xv, dts[x_dt]), _stored(xt, dts[x_dt])
    use_own = hidden != 1000   # one case without the block's own vectors
    ov, ot = capi.ada_in(_dev(xv, dts[x_dt]), _dev(xt, dts[x_dt]) if tr else None, vr, tr,
                         _dev(mod["shift"]), _dev(mod["scale"]),
                         *([_dev(own[k]) for k in ("video_shift", "video_scale", "text_shift",
                                                   "text_scale")] if use_own else []),
                         eps=1e-5, out_dtype=dts[out_dt])
    torch.cuda.synchronize()
    for stream, x, rows, out in (("video", xv, vr, ov), ("text", xt, tr, ot)):
        if not rows or sum(rows) == 0:
            continue
        ref = oracle.ada_in(x, rows, mod["shift"], mod["scale"],
                            own[f"{stream}_shift"] if use_own else None,
                            own[f"{stream}_scale"] if use_own else None, eps=1e-5)
        got = out.float().cpu().numpy()
        assert got.shape == ref.shape
        if out_dt == "f32":
            assert_close(got, ref)
            bound = 2e-6 * max(1.0, float(np.abs(ref).max()))
        else:
            bound = (2.0 ** -8 if out_dt == "bf16" else 2.0 ** -11) * np.abs(ref) + 1e-6
        assert np.all(np.abs(got - ref) <= bound), float(np.max(np.abs(got - ref) - bound))


@pytest.mark.parametrize("hidden,vr,tr", CASES)
@pytest.mark.parametrize("x_dt,y_dt", [("f32", "bf16"), ("f32", "f32"), ("bf16", "bf16"),
                                       ("f16", "f32")])
def test_ada_out_is_bit_exact(hidden, vr, tr, x_dt, y_dt):
    torch = _torch()
    from seedvr2_ncnn_amd import capi
    dts = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
    xv, xt, mod, own = _data(hidden, vr, tr, 7 * hidden + len(vr))
    g = np.random.default_rng(hidden)
    yv = _stored(g.standard_normal(xv.shape).astype(np.float32), dts[y_dt])
    yt = _stored(g.standard_normal(xt.shape).astype(np.float32), dts[y_dt])
    xv, xt = _stored(xv, dts[x_dt]), _stored(xt, dts[x_dt])
    use_own = hidden != 96
    xv_d, xt_d = _dev(xv, dts[x_dt]), (_dev(xt, dts[x_dt]) if tr else None)
    ov, ot = capi.ada_out(xv_d, xt_d, _dev(yv, dts[y_dt]), _dev(yt, dts[y_dt]) if tr else None,
                          vr, tr, _dev(mod["gate"]),
                          *([_dev(own["video_gate"]), _dev(own["text_gate"])] if use_own else []))
    torch.cuda.synchronize()
    assert ov.data_ptr() == xv_d.data_ptr()   # in place by default
    for stream, x, y, rows, out in (("video", xv, yv, vr, ov), ("text", xt, yt, tr, ot)):
        if not rows or sum(rows) == 0:
            continue
        ref = oracle.ada_out(x, y, rows, mod["gate"], own[f"{stream}_gate"] if use_own else None)
        ref = _stored(ref, dts[x_dt])
        np.testing.assert_array_equal(out.float().cpu().numpy(), ref)


def test_ada_in_strided_rows_and_separate_output():
    """row views into wider buffers (the fused QKV-style strides) and an
    output stride that differs from the input's"""
    torch = _torch()
    from seedvr2_ncnn_amd import capi
    hidden, vr, tr = 256, [33, 18], [6, 6]
    xv, xt, mod, own = _data(hidden, vr, tr, 99)
    big_v = _dev(np.concatenate([xv, np.zeros_like(xv)], 1))
    big_t = _dev(np.concatenate([xt, np.zeros_like(xt)], 1))
    out_v = torch.zeros((sum(vr), 3 * hidden), dtype=torch.bfloat16, device="cuda")
    out_t = torch.zeros((sum(tr), 3 * hidden), dtype=torch.bfloat16, device="cuda")
    capi.ada_in(big_v[:, :hidden], big_t[:, :hidden], vr, tr, _dev(mod["shift"]),
                _dev(mod["scale"]), out_video=out_v[:, hidden:2 * hidden],
                out_text=out_t[:, hidden:2 * hidden])
    torch.cuda.synchronize()
    for x, rows, out in ((xv, vr, out_v), (xt, tr, out_t)):
        o = out.float().cpu().numpy()
        assert np.all(o[:, :hidden] == 0) and np.all(o[:, 2 * hidden:] == 0)
        ref = oracle.ada_in(x, rows, mod["shift"], mod["scale"])
        assert np.all(np.abs(o[:, hidden:2 * hidden] - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-6)


@pytest.mark.parametrize("hidden,vr,tr", CASES)
@pytest.mark.parametrize("x_dt,y_dt,h_dt", [("f32", "bf16", "bf16"), ("bf16", "bf16", "f32"),
                                            ("f16", "f32", "f16")])
def test_fused_out_in_equals_the_two_passes(hidden, vr, tr, x_dt, y_dt, h_dt):
    """s2_dit_ada_out_in gives bit for bit what s2_dit_ada_out followed by
    s2_dit_ada_in gives, and h matches the oracle composite"""
    torch = _torch()
    from seedvr2_ncnn_amd import capi
    dts = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
    xv, xt, mod, own = _data(hidden, vr, tr, 3 * hidden + len(vr))
    g = np.random.default_rng(hidden + 1)
    yv = _stored(g.standard_normal(xv.shape).astype(np.float32), dts[y_dt])
    yt = _stored(g.standard_normal(xt.shape).astype(np.float32), dts[y_dt])
    xv, xt = _stored(xv, dts[x_dt]), _stored(xt, dts[x_dt])
    nt = sum(tr or [])
    y_d = (_dev(yv, dts[y_dt]), _dev(yt, dts[y_dt]) if nt else None)
    vecs = {k: _dev(v) for k, v in own.items()}
    m = {k: _dev(v) for k, v in mod.items()}

    # two passes
    x2 = (_dev(xv, dts[x_dt]), _dev(xt, dts[x_dt]) if nt else None)
    capi.ada_out(*x2, *y_d, vr, tr, m["gate"], vecs["video_gate"], vecs["text_gate"])
    h2 = capi.ada_in(*x2, vr, tr, m["shift"], m["scale"], vecs["video_shift"], vecs["video_scale"],
                     vecs["text_shift"], vecs["text_scale"], out_dtype=dts[h_dt])
    # one pass
    x1 = (_dev(xv, dts[x_dt]), _dev(xt, dts[x_dt]) if nt else None)
    _, _, hv1, ht1 = capi.ada_out_in(*x1, *y_d, vr, tr, m["gate"], m["shift"], m["scale"],
                                     vecs["video_gate"], vecs["text_gate"], vecs["video_shift"],
                                     vecs["video_scale"], vecs["text_shift"], vecs["text_scale"],
                                     h_dtype=dts[h_dt])
    torch.cuda.synchronize()
    assert torch.equal(x1[0], x2[0]) and torch.equal(hv1, h2[0])
    if nt:
        assert torch.equal(x1[1], x2[1]) and torch.equal(ht1, h2[1])
    for stream, x, y, rows, h in (("video", xv, yv, vr, hv1), ("text", xt, yt, tr, ht1)):
        if not rows or sum(rows) == 0:
            continue
        res = _stored(oracle.ada_out(x, y, rows, mod["gate"], own[f"{stream}_gate"]), dts[x_dt])
        ref = oracle.ada_in(res, rows, mod["shift"], mod["scale"], own[f"{stream}_shift"],
                            own[f"{stream}_scale"])
        got = h.float().cpu().numpy()
        tol = {"f32": 2e-6 * max(1.0, float(np.abs(ref).max())), "bf16": 2.0 ** -8 * np.abs(ref) + 1e-6,
               "f16": 2.0 ** -11 * np.abs(ref) + 1e-6}[h_dt]
        assert np.all(np.abs(got - ref) <= tol)
