"""DiT frontend/tail and the sampler step on the GPU against the CPU oracle:
patchify (src/seedvr2/seedvr2_dit.cpp:167-230), the latent/condition video
tokens of SeedVR2Pipeline::predict (src/seedvr2/seedvr2_pipeline.cpp:296-317),
the timestep embedding (seedvr2_dit.cpp:232-253), unpatchify (:255-326), CFG
(seedvr2_pipeline.cpp:171-210) and the Euler update (:575-588).

Permutations, CFG without rescale and the Euler update are bit-exact.  The
embedding is within 1 ulp (the device rounds sin/cos correctly; the C
library's sinf/cosf are not always correctly rounded).  With rescale the
guidance factor comes from fp64 sums in another order than the reference's
serial loop, so the rescaled values may differ in the last bit of the
factor: relative error <= 3e-7."""
import numpy as np
import pytest

import oracle
from seedvr2_ncnn_amd import capi

pytestmark = pytest.mark.gpu

# (t, h, w) samples: tiny, odd patch counts, one patch row wider than a
# 32-patch tile, the 720p latent grid, and a mixed batch
SHAPES = [[(1, 2, 2)], [(2, 4, 6)], [(3, 10, 130)], [(6, 90, 160)],
          [(3, 10, 14), (1, 8, 8), (2, 2, 70)]]


def _cuda(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _ulps(a, b):
    ai = a.view(np.int32).astype(np.int64)
    bi = b.view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(ai & 0x7fffffff), ai)
    bi = np.where(bi < 0, -(bi & 0x7fffffff), bi)
    return np.abs(ai - bi)


@pytest.mark.parametrize("shapes", SHAPES)
def test_patchify_bit_exact(shapes):
    g = np.random.default_rng(sum(h * w for _, h, w in shapes))
    tokens = sum(t * h * w for t, h, w in shapes)
    src = g.standard_normal((tokens, 33)).astype(np.float32)
    code, ref = oracle.patchify_video(src, shapes)
    assert code == 0
    got = _host(capi.patchify_video(_cuda(src), shapes))
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("shapes", SHAPES)
def test_unpatchify_bit_exact(shapes):
    g = np.random.default_rng(3 + sum(t * w for t, _, w in shapes))
    patches = sum(t * (h // 2) * (w // 2) for t, h, w in shapes)
    src = g.standard_normal((patches, 64)).astype(np.float32)
    code, ref = oracle.unpatchify_prediction(src, shapes)
    assert code == 0
    got = _host(capi.unpatchify_prediction(_cuda(src), shapes))
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("shape", [(1, 2, 2), (2, 4, 6), (3, 10, 130), (6, 90, 160), (1, 6, 64)])
def test_latent_patches_bit_exact(shape):
    t, h, w = shape
    tokens = t * h * w
    stride = (tokens + 3) // 4 * 4 + 4          # an ncnn cstep with padding
    g = np.random.default_rng(tokens)
    lat = g.standard_normal((16, stride)).astype(np.float32)
    cond = g.standard_normal((16, stride)).astype(np.float32)
    code, ref = oracle.patchify_video(oracle.video_tokens(lat, cond, tokens), [shape])
    assert code == 0
    got = _host(capi.latent_patches(_cuda(lat), _cuda(cond), t, h, w, stride))
    assert np.array_equal(got, ref)


def test_timestep_embedding_within_one_ulp():
    steps = 50
    ts = [1000.0 * (steps - s) / steps for s in range(steps)]      # the sampler's schedule
    ts += [0.0, 1.0, 0.5, 999.9, 1000.0, 123.456, 7.0, 3.0e-3]
    ts += list(np.linspace(0, 1000, 17, dtype=np.float32))         # 75 rows: two launches
    ref = oracle.timestep_embedding(np.asarray(ts, np.float32))
    got = _host(capi.timestep_embedding(ts))
    assert got.shape == (len(ts), 256)
    assert int(_ulps(got, ref).max()) <= 1
    assert np.mean(got == ref) > 0.95
    assert np.array_equal(got[steps, :128], np.zeros(128, np.float32))
    assert np.array_equal(got[steps, 128:], np.ones(128, np.float32))


CFG_COUNTS = [1, 3, 4096, 4099, 21600 * 64, 1000003]


@pytest.mark.parametrize("count", CFG_COUNTS)
@pytest.mark.parametrize("scale,rescale", [(6.5, 0.0), (1.0, 0.0), (6.5, 0.7), (3.0, 1.0)])
def test_apply_cfg(count, scale, rescale):
    g = np.random.default_rng(count + int(scale * 10 + rescale * 100))
    pos = g.standard_normal(count).astype(np.float32)
    neg = (0.8 * pos + 0.3 * g.standard_normal(count)).astype(np.float32)
    ref = oracle.apply_cfg(pos, neg, scale, rescale)
    got = _host(capi.apply_cfg(_cuda(pos), _cuda(neg), scale, rescale))
    if rescale == 0.0 or count < 2:
        assert np.array_equal(got, ref)
    else:
        rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)
        assert float(rel.max()) <= 3e-7


def test_apply_cfg_zero_spread_and_nan():
    pos = np.full(5000, 2.0, np.float32)
    neg = np.full(5000, 1.0, np.float32)
    got = _host(capi.apply_cfg(_cuda(pos), _cuda(neg), 4.0, 0.7))
    assert np.array_equal(got, oracle.apply_cfg(pos, neg, 4.0, 0.7))
    pos[123] = np.nan                      # a NaN reaches the statistics: all NaN
    got = _host(capi.apply_cfg(_cuda(pos), _cuda(neg), 4.0, 0.7))
    ref = oracle.apply_cfg(pos, neg, 4.0, 0.7)
    assert np.isnan(ref).all() and np.isnan(got).all()


@pytest.mark.parametrize("tokens", [1, 255, 257, 86400])
def test_euler_step_bit_exact(tokens):
    g = np.random.default_rng(tokens)
    stride = (tokens + 3) // 4 * 4 + 8
    lat = g.standard_normal((16, stride)).astype(np.float32)
    pred = g.standard_normal((tokens, 16)).astype(np.float32)
    delta = np.float32((980.0 - 1000.0) / 1000.0)
    ref = oracle.euler_step(lat, pred, delta)
    d_lat = _cuda(lat)
    capi.euler_step(d_lat, stride, _cuda(pred), delta)
    assert np.array_equal(_host(d_lat), ref)


@pytest.mark.parametrize("shape", [(2, 4, 6), (3, 10, 130), (6, 90, 160)])
@pytest.mark.parametrize("mode", ["positive", "cfg", "rescale"])
def test_denoise_update(shape, mode):
    t, h, w = shape
    tokens = t * h * w
    patches = tokens // 4
    stride = (tokens + 3) // 4 * 4
    g = np.random.default_rng(tokens + len(mode))
    lat = g.standard_normal((16, stride)).astype(np.float32)
    pos = g.standard_normal((patches, 64)).astype(np.float32)
    neg = (0.9 * pos + 0.2 * g.standard_normal((patches, 64))).astype(np.float32)
    scale, rescale = {"positive": (1.0, 0.0), "cfg": (6.5, 0.0), "rescale": (6.5, 0.7)}[mode]
    delta = np.float32(-0.02)
    # the reference's sequence: unpatchify each prediction, CFG unless
    # cfg_scale == 1, Euler update
    _, pp = oracle.unpatchify_prediction(pos, [shape])
    pred = pp
    if mode != "positive":
        _, pn = oracle.unpatchify_prediction(neg, [shape])
        pred = oracle.apply_cfg(pp.ravel(), pn.ravel(), scale, rescale).reshape(pp.shape)
    ref = oracle.euler_step(lat, pred, delta)
    d_lat = _cuda(lat)
    capi.denoise_update(_cuda(pos), None if mode == "positive" else _cuda(neg), t, h, w, scale,
                        rescale, delta, d_lat, stride)
    got = _host(d_lat)
    if mode != "rescale":
        assert np.array_equal(got, ref)
    else:
        step = np.abs(delta * pred.T)
        bound = 2 * np.spacing(np.abs(ref[:, :tokens])) + 3e-7 * step
        assert np.all(np.abs(got[:, :tokens] - ref[:, :tokens]) <= bound)
        assert np.array_equal(got[:, tokens:], lat[:, tokens:])


def test_fused_tail_equals_unfused_entry_points():
    t, h, w = 2, 6, 70
    tokens = t * h * w
    stride = tokens + 4
    g = np.random.default_rng(11)
    lat = g.standard_normal((16, stride)).astype(np.float32)
    pos = g.standard_normal((tokens // 4, 64)).astype(np.float32)
    neg = g.standard_normal((tokens // 4, 64)).astype(np.float32)
    d_pos, d_neg = _cuda(pos), _cuda(neg)
    a = _cuda(lat)
    capi.denoise_update(d_pos, d_neg, t, h, w, 5.0, 0.0, -0.1, a, stride)
    b = _cuda(lat)
    pp = capi.unpatchify_prediction(d_pos, [(t, h, w)])
    pn = capi.unpatchify_prediction(d_neg, [(t, h, w)])
    capi.euler_step(b, stride, capi.apply_cfg(pp, pn, 5.0, 0.0), -0.1)
    assert np.array_equal(_host(a), _host(b))
