"""CPU pinning of the oracle's DecomposedConv3D (src/seedvr2/decomposed_conv3d.cpp:605-755)
against torch's float64 conv3d over the temporally padded input, and of its
temporal memory against the unsplit run."""
import numpy as np
import pytest
import torch

import oracle


def _torch_conv3d(cfg, x, weights, bias, prefix_frames):
    """conv3d of [prefix | x] in float64; weights [kt, Cout, Cin, kh, kw]."""
    xp = torch.from_numpy(np.concatenate([prefix_frames, x], axis=1)).double()[None]
    w = torch.from_numpy(weights).double().permute(1, 2, 0, 3, 4)
    b = torch.from_numpy(bias).double() if bias is not None else None
    y = torch.nn.functional.conv3d(xp, w, b, stride=(cfg.stride_t, cfg.stride_h, cfg.stride_w),
                                   padding=(0, cfg.pad_h, cfg.pad_w),
                                   dilation=(cfg.dilation_t, cfg.dilation_h, cfg.dilation_w))
    return y[0].numpy()


CASES = [
    # cin, cout, frames, h, w, (kt, kh, kw), strides (t, h, w), dilation (t, h, w), pad (h, w), head
    (4, 6, 3, 5, 7, (3, 3, 3), (1, 1, 1), (1, 1, 1), (1, 1), 2),
    (3, 8, 5, 6, 6, (3, 3, 3), (1, 2, 2), (1, 1, 1), (1, 1), 2),
    (5, 4, 4, 7, 9, (2, 3, 1), (2, 1, 1), (1, 2, 1), (2, 0), 1),
    (8, 8, 2, 4, 4, (1, 1, 1), (1, 1, 1), (1, 1, 1), (0, 0), 0),
    (2, 3, 6, 5, 4, (3, 3, 3), (1, 1, 1), (2, 1, 1), (1, 1), 4),
]


@pytest.mark.parametrize("cin,cout,frames,h,w,k,s,d,p,head", CASES)
@pytest.mark.parametrize("with_bias", [True, False])
def test_matches_torch_conv3d_over_padded_input(cin, cout, frames, h, w, k, s, d, p, head, with_bias):
    g = np.random.default_rng(cin * 100 + cout * 10 + frames)
    cfg = oracle.conv3d_config(num_output=cout, num_input=cin, kernel_t=k[0], kernel_h=k[1],
                               kernel_w=k[2], stride_t=s[0], stride_h=s[1], stride_w=s[2],
                               dilation_t=d[0], dilation_h=d[1], dilation_w=d[2], pad_h=p[0],
                               pad_w=p[1], head_frames=head, bias_term=int(with_bias))
    x = g.standard_normal((cin, frames, h, w)).astype(np.float32)
    wts = (0.3 * g.standard_normal((k[0], cout, cin, k[1], k[2]))).astype(np.float32)
    bias = g.standard_normal(cout).astype(np.float32) if with_bias else None
    code, out, _ = oracle.decomposed_conv3d(cfg, x, wts, bias, cstep_pad=4)
    ref = _torch_conv3d(cfg, x, wts, bias, np.repeat(x[:, :1], head, axis=1))
    assert code == ref.shape[1]
    assert out.shape == ref.shape
    # each tap rounded to fp32, the taps summed in fp32
    assert np.max(np.abs(out - ref)) <= 1e-5 * max(1.0, np.max(np.abs(ref)))


def test_one_by_one_kernel_is_a_pixel_matmul():
    g = np.random.default_rng(1)
    cfg = oracle.conv3d_config(num_output=5, num_input=7, kernel_t=1, kernel_h=1, kernel_w=1)
    x = g.standard_normal((7, 2, 3, 4)).astype(np.float32)
    wts = g.standard_normal((1, 5, 7, 1, 1)).astype(np.float32)
    code, out, _ = oracle.decomposed_conv3d(cfg, x, wts)
    ref = np.einsum("oc,cthw->othw", wts[0, :, :, 0, 0].astype(np.float64), x.astype(np.float64))
    assert code == 2 and np.max(np.abs(out - ref)) < 1e-5


@pytest.mark.parametrize("split", [1, 2, 3])
def test_memory_chains_slices_into_the_unsplit_run(split):
    g = np.random.default_rng(split)
    cfg = oracle.conv3d_config(num_output=4, num_input=3, kernel_t=3, kernel_h=3, kernel_w=3,
                               pad_h=1, pad_w=1, head_frames=2)
    x = g.standard_normal((3, 5, 4, 6)).astype(np.float32)
    wts = g.standard_normal((3, 4, 3, 3, 3)).astype(np.float32)
    _, full, _ = oracle.decomposed_conv3d(cfg, x, wts)
    # first slice: head frames (no memory yet); later slices: the memory
    c1, a, mem = oracle.decomposed_conv3d(cfg, x[:, :split], wts, want_memory=True)
    c2, b, mem2 = oracle.decomposed_conv3d(cfg, x[:, split:], wts, memory=mem, want_memory=True)
    assert c1 == split and c2 == 5 - split
    assert np.array_equal(np.concatenate([a, b], axis=1), full)
    assert np.array_equal(mem2, x[:, 3:5])


def test_rejects_bad_configurations():
    x = np.zeros((2, 1, 4, 4), np.float32)
    w = np.zeros((3, 2, 2, 3, 3), np.float32)
    bad = oracle.conv3d_config(num_output=2, num_input=2, kernel_t=3, kernel_h=3, kernel_w=3,
                               head_frames=0)
    assert oracle.decomposed_conv3d(bad, x, w)[0] == -1          # too few frames
    grp = oracle.conv3d_config(num_output=2, num_input=2, kernel_t=3, kernel_h=3, kernel_w=3,
                               head_frames=2, groups=2)
    assert oracle.decomposed_conv3d(grp, x, w)[0] == -1


@pytest.mark.parametrize("tr,sr,remove", [(1, 2, False), (2, 2, True), (2, 1, True), (1, 1, False)])
def test_pixel_shuffle_is_depth_to_space(tr, sr, remove):
    g = np.random.default_rng(tr * 10 + sr)
    c, f, h, w = 3, 3, 4, 5
    packed = g.standard_normal((c * tr * sr * sr, f, h, w)).astype(np.float32)
    out = oracle.vae_pixel_shuffle(packed, c, tr, sr, remove)
    # packed channel ((yo*sr + xo)*tr + z)*c + ch -> (yo, xo, z, ch) outermost first
    t = torch.from_numpy(packed).reshape(sr, sr, tr, c, f, h, w)
    t = t.permute(3, 4, 2, 5, 0, 6, 1).reshape(c, f * tr, h * sr, w * sr)
    if remove:
        t = torch.cat([t[:, :1], t[:, 2:]], dim=1)
    assert np.array_equal(out, t.numpy())
