"""CPU pinning of the oracle's DiT frontend/tail functions (patchify, timestep
embedding, unpatchify, classifier-free guidance, Euler step) against numpy
closed forms; the reference is src/seedvr2/seedvr2_dit.cpp:167-326 and
src/seedvr2/seedvr2_pipeline.cpp:171-210, 575-588."""
import numpy as np
import pytest

import oracle


def _patchify_np(src, shapes):
    out, off = [], 0
    for t, h, w in shapes:
        g = src[off:off + t * h * w].reshape(t, h // 2, 2, w // 2, 2, 33)
        out.append(g.transpose(0, 1, 3, 2, 4, 5).reshape(t * (h // 2) * (w // 2), 132))
        off += t * h * w
    return np.concatenate(out)


def _unpatchify_np(src, shapes):
    out, off = [], 0
    for t, h, w in shapes:
        n = t * (h // 2) * (w // 2)
        g = src[off:off + n].reshape(t, h // 2, w // 2, 2, 2, 16)
        out.append(g.transpose(0, 1, 3, 2, 4, 5).reshape(t * h * w, 16))
        off += n
    return np.concatenate(out)


SHAPES = [[(1, 2, 2)], [(2, 4, 6)], [(6, 90, 160)], [(3, 10, 14), (1, 8, 8), (2, 2, 30)]]


@pytest.mark.parametrize("shapes", SHAPES)
def test_patchify_matches_reshape(shapes):
    g = np.random.default_rng(len(shapes) * 31 + shapes[0][1])
    tokens = sum(t * h * w for t, h, w in shapes)
    src = g.standard_normal((tokens, 33)).astype(np.float32)
    code, out = oracle.patchify_video(src, shapes)
    assert code == 0
    assert np.array_equal(out, _patchify_np(src, shapes))


@pytest.mark.parametrize("shapes", SHAPES)
def test_unpatchify_matches_reshape_and_inverts_patch_layout(shapes):
    g = np.random.default_rng(len(shapes) * 37 + shapes[0][2])
    tokens = sum(t * h * w for t, h, w in shapes)
    patches = sum(t * (h // 2) * (w // 2) for t, h, w in shapes)
    src = g.standard_normal((patches, 64)).astype(np.float32)
    code, out = oracle.unpatchify_prediction(src, shapes)
    assert code == 0 and out.shape == (tokens, 16)
    assert np.array_equal(out, _unpatchify_np(src, shapes))
    # tokens laid out as 16-channel patches come back unchanged
    tok = g.standard_normal((tokens, 16)).astype(np.float32)
    pat = np.concatenate([_patchify_np(np.pad(tok, ((0, 0), (0, 17))), shapes)[:, k * 33:k * 33 + 16]
                          for k in range(4)], axis=1)
    code, back = oracle.unpatchify_prediction(pat, shapes)
    assert code == 0 and np.array_equal(back, tok)


def test_patchify_rejects_odd_or_mismatched_shapes():
    src = np.zeros((2 * 3 * 4, 33), np.float32)
    assert oracle.patchify_video(src, [(2, 3, 4)])[0] == -1          # odd h
    assert oracle.patchify_video(src[:-1], [(2, 4, 3)])[0] == -1     # odd w
    assert oracle.patchify_video(np.zeros((10, 33), np.float32), [(1, 4, 4)])[0] == -1
    assert oracle.unpatchify_prediction(np.zeros((3, 64), np.float32), [(1, 4, 4)])[0] == -1


def test_timestep_embedding_closed_form():
    ts = np.array([0.0, 1.0, 37.5, 500.0, 1000.0], np.float32)
    out = oracle.timestep_embedding(ts)
    i = np.arange(128)
    phase = ts[:, None].astype(np.float64) * np.exp(-np.log(10000.0) * i / 128)
    ref = np.concatenate([np.sin(phase), np.cos(phase)], axis=1)
    # fp32 phase: one rounding of a value up to 1000 moves sin/cos by < 1e-4
    assert np.max(np.abs(out - ref)) < 2e-4
    assert np.array_equal(out[0, :128], np.zeros(128, np.float32))
    assert np.array_equal(out[0, 128:], np.ones(128, np.float32))


@pytest.mark.parametrize("scale,rescale", [(0.0, 0.0), (6.5, 0.0), (6.5, 0.7), (3.0, 1.0)])
def test_apply_cfg_closed_form(scale, rescale):
    g = np.random.default_rng(int(scale * 10 + rescale * 100))
    pos = g.standard_normal(4000).astype(np.float32)
    neg = (0.8 * pos + 0.3 * g.standard_normal(4000)).astype(np.float32)
    out = oracle.apply_cfg(pos, neg, scale, rescale)
    cfg = neg + np.float32(scale) * (pos - neg)          # fp32, as the reference
    if rescale != 0.0:
        pd, cd = pos.astype(np.float64), cfg.astype(np.float64)
        factor = np.float32(rescale * pd.std(ddof=1) / cd.std(ddof=1) + (1.0 - rescale))
        cfg = cfg * factor
    if rescale == 0.0:
        # no reduction involved: one fp32 subtract, multiply and add, unfused
        assert np.array_equal(out, cfg)
    else:
        assert np.max(np.abs(out - cfg) / np.maximum(np.abs(cfg), 1e-3)) < 1e-6
    if scale == 0.0:
        assert np.array_equal(out, neg)


def test_apply_cfg_zero_spread_is_not_rescaled():
    pos = np.full(100, 2.0, np.float32)
    neg = np.full(100, 1.0, np.float32)
    out = oracle.apply_cfg(pos, neg, 4.0, 0.7)
    assert np.array_equal(out, np.full(100, 5.0, np.float32))


def test_euler_step_closed_form():
    g = np.random.default_rng(5)
    tokens, stride = 1000, 1008          # channel rows padded, as an ncnn cstep
    lat = g.standard_normal((16, stride)).astype(np.float32)
    pred = g.standard_normal((tokens, 16)).astype(np.float32)
    delta = np.float32(-0.04)
    out = oracle.euler_step(lat, pred, delta)
    ref = lat.copy()
    ref[:, :tokens] = lat[:, :tokens] + (delta * pred.T)
    assert np.array_equal(out, ref)


def test_video_tokens_transpose_of_planes():
    g = np.random.default_rng(6)
    tokens, stride = 300, 304
    lat = g.standard_normal((16, stride)).astype(np.float32)
    cond = g.standard_normal((16, stride)).astype(np.float32)
    out = oracle.video_tokens(lat, cond, tokens)
    ref = np.concatenate([lat[:, :tokens].T, cond[:, :tokens].T, np.ones((tokens, 1), np.float32)], 1)
    assert np.array_equal(out, ref)
