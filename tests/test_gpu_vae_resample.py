"""VAEDownsample3D and VAEUpsample3D on the GPU (src/seedvr2/vae_downsample3d.cpp:98-172,
vae_upsample3d.cpp:191-321) against the oracle's restatements: right/bottom
zero padding then DecomposedConv3D; upscale DecomposedConv3D, depth-to-space
shuffle over time and space, post DecomposedConv3D.  The convolutions run in
bf16 with fp32 accumulation; the bar is the path's (max-abs <= 2e-2, cosine
>= 0.9999)."""
import numpy as np
import pytest

import oracle
from common import Layer, assert_close, set_vae_memory_state

pytestmark = pytest.mark.gpu


def _conv(g, cin, cout, k=(3, 3, 3), s=(1, 1, 1), p=(1, 1), head=2):
    cfg = oracle.conv3d_config(num_output=cout, num_input=cin, kernel_t=k[0], kernel_h=k[1],
                               kernel_w=k[2], stride_t=s[0], stride_h=s[1], stride_w=s[2],
                               pad_h=p[0], pad_w=p[1], head_frames=head, bias_term=1)
    w = (g.standard_normal((k[0], cout, cin, k[1], k[2])) / np.sqrt(cin * k[0] * k[1] * k[2]))
    b = 0.1 * g.standard_normal(cout)
    return cfg, w.astype(np.float32), b.astype(np.float32)


def _conv_blobs(cfg, w, b):
    fields = [getattr(cfg, n) for n, _ in oracle.Conv3dConfig._fields_]
    return [np.asarray(fields, np.float32), b, w]


def _downsample(g, c, cout, pr, pb):
    cfg, w, b = _conv(g, c, cout, s=(1, 2, 2), p=(0, 0))
    layer = Layer("ExportDownsample3D", "", weights=[np.asarray([c, pr, pb], np.float32)] +
                  _conv_blobs(cfg, w, b))
    assert layer.create_code == 0 and layer.create_pipeline() == 0
    return layer, (cfg, w, b)


def _upsample(g, c, tr, sr):
    ratio = tr * sr * sr
    post = _conv(g, c, c)
    up = _conv(g, c, c * ratio)
    cfg_blob = np.asarray([c, tr, sr, 1 if tr == 2 else 0], np.float32)
    layer = Layer("ExportUpsample3D", "",
                  weights=[cfg_blob] + _conv_blobs(*post) + _conv_blobs(*up))
    assert layer.create_code == 0 and layer.create_pipeline() == 0
    return layer, post, up


@pytest.mark.parametrize("device", [False, True])
@pytest.mark.parametrize("pr,pb", [(1, 1), (1, 0)])
def test_downsample(device, pr, pb):
    import torch
    g = np.random.default_rng(pr * 2 + pb)
    c, f, h, w = 32, 3, 10, 14
    layer, (cfg, wt, b) = _downsample(g, c, 48, pr, pb)
    x = g.standard_normal((c, f, h, w)).astype(np.float32)
    if device:
        x = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    set_vae_memory_state(0)
    ref = oracle.vae_downsample3d(cfg, wt, b, x, pr, pb)
    code, got = layer.forward_planar(x, (w, h, f, c), tuple(reversed(ref.shape[1:])) + (48,),
                                     device=device, dtype=torch.bfloat16 if device else None)
    assert code == 0
    assert_close(got, ref)


@pytest.mark.parametrize("device", [False, True])
@pytest.mark.parametrize("h,w", [(2, 9), (5, 2)])
def test_downsample_input_valid_only_after_padding(device, h, w):
    """A frame two rows (or columns) wide is narrower than a 3 x 3 window
    without padding until the bottom (right) zero padding lengthens it to 3;
    the workspace and the output follow the padded extent
    (vae_downsample3d.cpp:145-172).  64 -> 128 channels over 3 taps: the few
    output tiles split the k loop into ranges."""
    import torch
    g = np.random.default_rng(40 + h)
    c, f = 64, 3
    cfg, wt, b = _conv(g, c, 128, s=(1, 1, 1), p=(0, 0))
    layer = Layer("ExportDownsample3D", "", weights=[np.asarray([c, 1, 1], np.float32)] +
                  _conv_blobs(cfg, wt, b))
    assert layer.create_code == 0 and layer.create_pipeline() == 0
    x = g.standard_normal((c, f, h, w)).astype(np.float32)
    if device:
        x = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    set_vae_memory_state(0)
    ref = oracle.vae_downsample3d(cfg, wt, b, x, 1, 1)
    code, got = layer.forward_planar(x, (w, h, f, c), tuple(reversed(ref.shape[1:])) + (128,),
                                     device=device, dtype=torch.bfloat16 if device else None)
    assert code == 0
    assert_close(got, ref)


@pytest.mark.parametrize("device", [False, True])
@pytest.mark.parametrize("tr,sr", [(2, 2), (1, 2), (2, 1)])
def test_upsample(device, tr, sr):
    import torch
    g = np.random.default_rng(tr * 10 + sr)
    c, f, h, w = 16, 3, 6, 8
    layer, post, up = _upsample(g, c, tr, sr)
    x = g.standard_normal((c, f, h, w)).astype(np.float32)
    if device:
        x = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    set_vae_memory_state(0)
    ref = oracle.vae_upsample3d(*post, *up, x, c, tr, sr, remove_head=(tr == 2))
    code, got = layer.forward_planar(x, (w, h, f, c), tuple(reversed(ref.shape[1:])) + (c,),
                                     device=device, dtype=torch.bfloat16 if device else None)
    assert code == 0
    assert_close(got, ref)


def test_upsample_memory_chains_slices():
    """A first slice (INITIALIZING: the shuffled time 1 is dropped) and a
    second (ACTIVE: kept, both convolutions continue their memory) equal the
    unsplit run."""
    g = np.random.default_rng(5)
    c, h, w = 16, 6, 8
    layer, post, up = _upsample(g, c, 2, 2)
    x = g.standard_normal((c, 3, h, w)).astype(np.float32)
    full = oracle.vae_upsample3d(*post, *up, x, c, 2, 2, remove_head=True)
    outs = []
    for state, (a, b_) in ((1, (0, 2)), (2, (2, 3))):
        set_vae_memory_state(state)
        n_out = (b_ - a) * 2 - (1 if state == 1 else 0)
        code, out = layer.forward_planar(x[:, a:b_], (w, h, b_ - a, c), (w * 2, h * 2, n_out, c))
        assert code == 0
        outs.append(out)
    set_vae_memory_state(0)
    assert_close(np.concatenate(outs, axis=1), full)


def test_resample_rejects_bad_blobs():
    g = np.random.default_rng(6)
    layer, _ = _downsample(g, 8, 8, 1, 1)
    set_vae_memory_state(0)
    x = np.zeros((4, 2, 6, 6), np.float32)
    assert layer.forward_planar(x, (6, 6, 2, 4), (3, 3, 2, 8))[0] == -1   # wrong channels
    # config blobs the reference refuses: no padding; a temporal ratio of 3
    bad = Layer("ExportDownsample3D", "", weights=[np.asarray([8, 0, 0], np.float32)])
    assert bad.create_code == -1
    bad = Layer("ExportUpsample3D", "", weights=[np.asarray([8, 3, 2, 0], np.float32)])
    assert bad.create_code == -1
