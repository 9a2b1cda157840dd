"""DecomposedConv3D on the GPU (src/seedvr2/decomposed_conv3d.cpp:605-755) against
the CPU oracle.

The device multiplies bf16 operands (inputs and weights rounded to nearest
even as they are staged and packed) with fp32 accumulation over the whole
kt x kh x kw x num_input window.  Two comparisons per case: against the
oracle on the unrounded fp32 operands with the path's bar (max-abs <= 2e-2,
cosine >= 0.9999), and against the oracle on the bf16-rounded operands with
a tight bound (1e-4 of the output scale) that isolates the kernel's own
arithmetic (summation order only)."""
import ctypes

import numpy as np
import pytest

import oracle
from common import assert_close, bf16_round
from seedvr2_ncnn_amd import capi

pytestmark = pytest.mark.gpu


def _cfg(cin, cout, k=(3, 3, 3), s=(1, 1, 1), d=(1, 1, 1), p=(1, 1), head=2, bias=True):
    kw = dict(num_output=cout, num_input=cin, kernel_t=k[0], kernel_h=k[1], kernel_w=k[2],
              stride_t=s[0], stride_h=s[1], stride_w=s[2], dilation_t=d[0], dilation_h=d[1],
              dilation_w=d[2], pad_h=p[0], pad_w=p[1], head_frames=head, bias_term=int(bias))
    return capi.conv3d_config(**kw), oracle.conv3d_config(**kw)


def _case(cin, cout, frames, h, w, cfgs, seed):
    g = np.random.default_rng(seed)
    cfg = cfgs[1]
    x = g.standard_normal((cin, frames, h, w)).astype(np.float32)
    fan_in = cin * cfg.kernel_t * cfg.kernel_h * cfg.kernel_w
    wts = (g.standard_normal((cfg.kernel_t, cout, cin, cfg.kernel_h, cfg.kernel_w)) /
           np.sqrt(fan_in)).astype(np.float32)
    bias = (0.1 * g.standard_normal(cout)).astype(np.float32) if cfg.bias_term else None
    return x, wts, bias


def _device(cfg, wts, bias):
    import torch
    return capi.Conv3d(cfg, torch.from_numpy(wts).cuda(),
                       torch.from_numpy(bias).cuda() if bias is not None else None)


def _run(conv, x, cstep_pad=0, dtype=None, out_dtype=None, **kw):
    import torch
    cin, frames, h, w = x.shape
    flat = x.reshape(cin, -1)
    # an ncnn cstep: the channel rounded up to 16 bytes (8 elements covers
    # the 16-bit blobs too), plus any extra padding under test
    pad = (-flat.shape[1]) % 8 + cstep_pad
    if pad:
        flat = np.concatenate([flat, np.zeros((cin, pad), np.float32)], 1)
    t = torch.from_numpy(np.ascontiguousarray(flat)).cuda()
    if dtype is not None:
        t = t.to(dtype)
    out, (to, ho, wo) = conv.forward(t, frames, h, w, out_dtype=out_dtype, **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()[:, :to * ho * wo].reshape(-1, to, ho, wo)


def _check(got, x, wts, bias, cfg_o, memory=None):
    _, ref, _ = oracle.decomposed_conv3d(cfg_o, x, wts, bias, memory=memory)
    assert got.shape == ref.shape
    assert_close(got, ref)
    _, tight, _ = oracle.decomposed_conv3d(cfg_o, bf16_round(x), bf16_round(wts), bias,
                                           memory=None if memory is None else bf16_round(memory))
    scale = max(1.0, float(np.max(np.abs(tight))))
    assert float(np.max(np.abs(got - tight))) <= 1e-4 * scale


SHAPES = [
    # cin, cout, frames, h, w, kwargs
    (128, 128, 3, 12, 20, {}),                         # 512x128 tiles, partial last tile
    (64, 256, 2, 9, 13, {}),                           # 256x256 tiles
    (16, 320, 2, 6, 10, {}),                           # cin < 64 (zero channels), ragged n
    (3, 128, 5, 16, 16, dict(s=(1, 2, 2))),            # RGB input, spatial stride 2
    (96, 72, 4, 7, 9, dict(k=(3, 1, 3), p=(0, 1))),    # ragged k window, cin not a multiple of 64
    (256, 256, 1, 8, 8, dict(k=(1, 1, 1), p=(0, 0), head=0)),   # pointwise
    (32, 40, 6, 5, 6, dict(s=(2, 1, 1), d=(2, 1, 2), p=(1, 2), head=4)),
    (128, 3, 3, 12, 20, {}),                           # RGB output: 512x32 tiles
    (64, 32, 2, 9, 13, dict(s=(1, 2, 2))),             # 32 output channels, stride 2
    (16, 16, 4, 8, 10, {}),                            # 16 in and out (latent width)
    (24, 64, 3, 7, 9, dict(k=(1, 3, 3))),              # 32-channel pixels, last k-step part empty
    (8, 130, 2, 11, 6, dict(k=(2, 3, 3), head=1)),     # 8-channel pixels, ragged n
    # 3x3 stride-1 layers on frames that fill 128-column tiles to 93% take the
    # halo kernel (4 x 128 output tiles, 128 or 32 output channels a tile)
    (128, 128, 3, 6, 120, {}),                         # ragged tile rows and columns
    (64, 3, 2, 9, 250, {}),                            # RGB output, two tile columns
    (16, 64, 2, 5, 124, dict(head=1)),                 # 16-channel pixels
    (32, 96, 3, 4, 128, dict(p=(0, 1))),               # no row padding
    (96, 128, 3, 7, 240, dict(k=(2, 3, 3), s=(2, 1, 1))),   # temporal stride 2
    (64, 200, 2, 5, 120, {}),                          # two channel tiles, the second ragged
    (256, 256, 2, 4, 128, {}),                         # 256 channels in and out
    (64, 160, 2, 10, 192, {}),                         # 64-column tiles (192 = 3 x 64)
    (128, 3, 2, 9, 320, {}),                           # RGB output in 64-column tiles
    # layers of at least 64 input channels with fewer than 256 implicit-GEMM
    # tiles split the k loop into ranges of k-steps (most small cases above
    # do too; the ranges cross window positions and temporal taps); these
    # are a latent-width frame, two temporal taps, and the 720p latent
    # layer's 114 tiles (two ranges)
    (512, 512, 1, 9, 16, {}),                          # 512 channels, 3 taps
    (64, 96, 3, 6, 10, dict(k=(2, 3, 3))),             # 2 taps
    (512, 512, 1, 90, 160, {}),                        # 114 tiles, 2 ranges
]


@pytest.mark.parametrize("cin,cout,frames,h,w,kw", SHAPES)
def test_conv3d_matches_oracle(cin, cout, frames, h, w, kw):
    cfgs = _cfg(cin, cout, **kw)
    x, wts, bias = _case(cin, cout, frames, h, w, cfgs, cin + cout + frames)
    got = _run(_device(cfgs[0], wts, bias), x)
    _check(got, x, wts, bias, cfgs[1])


# The unsplit implicit-GEMM k loop of layers with several temporal taps: one
# workgroup advances from tap to tap and runs the bias epilogue on the whole
# sum.  Small layers of at least 64 input channels split their k loop into
# ranges when the workspace holds the partial tiles; a workspace with only
# the staged frames (which the forward accepts) runs them unsplit.
@pytest.mark.parametrize("cin,cout,frames,h,w,kw", [
    (64, 128, 3, 10, 12, {}),                    # 512 x 128 tiles, 3 taps
    (64, 256, 2, 9, 13, dict(k=(2, 3, 3))),      # 256 x 256 tiles, 2 taps
    (128, 96, 3, 6, 10, dict(s=(1, 2, 2))),      # stride 2, ragged n
])
def test_conv3d_unsplit_taps_with_staged_only_workspace(cin, cout, frames, h, w, kw):
    cfgs = _cfg(cin, cout, **kw)
    x, wts, bias = _case(cin, cout, frames, h, w, cfgs, 3 * cin + cout)
    conv = _device(cfgs[0], wts, bias)
    got = _run(conv, x, staged_only_workspace=True)
    _check(got, x, wts, bias, cfgs[1])
    split = _run(conv, x)
    assert_close(split, got)


def test_conv3d_unsplit_taps_at_256_tiles():
    """A layer that fills 256 implicit-GEMM tiles never splits its k loop:
    64 -> 256 channels, 2 taps, stride (1, 2, 2) (not the halo kernel), two
    output frames of 128 x 256 pixels = 256 tiles of 256 x 256."""
    cfgs = _cfg(64, 256, k=(2, 3, 3), s=(1, 2, 2), head=1)
    x, wts, bias = _case(64, 256, 2, 256, 512, cfgs, 11)
    got = _run(_device(cfgs[0], wts, bias), x)
    assert got.shape == (256, 2, 128, 256)
    _check(got, x, wts, bias, cfgs[1])


# More than 128 outputs (256 x 256 tiles on the ping-pong schedule) with the
# memory read in place: 80 pixels a frame keep each 8-row DMA group in one
# frame; 2 + 3 frames, the second slice's memory buffer reused or not.
@pytest.mark.parametrize("reuse", [False, True])
def test_conv3d_memory_chains_256_outputs(reuse):
    cfgs = _cfg(64, 256)
    x, wts, bias = _case(64, 256, 5, 8, 10, cfgs, 13)
    conv = _device(cfgs[0], wts, bias)
    a = _run(conv, x[:, :2], keep_memory=True)
    b = _run(conv, x[:, 2:], use_memory=True, keep_memory=True, reuse_memory_buffer=reuse)
    _, ref, _ = oracle.decomposed_conv3d(cfgs[1], x, wts, bias)
    assert_close(np.concatenate([a, b], axis=1), ref)


# (10, 12): the implicit-GEMM kernel; (6, 120): the halo kernel.  A channel
# stride padded by 4 elements leaves 16-bit channel rows without 16-byte
# alignment, which the staging pass reads element by element.
@pytest.mark.parametrize("in_dtype,out_dtype", [("bf16", "bf16"), ("f16", "f32"), ("f32", "f16")])
@pytest.mark.parametrize("hw", [(10, 12), (6, 120)])
@pytest.mark.parametrize("cstep_pad", [8, 4])
def test_conv3d_16bit_blobs_and_padded_cstep(in_dtype, out_dtype, hw, cstep_pad):
    import torch
    dt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
    cfgs = _cfg(64, 128)
    x, wts, bias = _case(64, 128, 2, hw[0], hw[1], cfgs, 7)
    if in_dtype != "f32":
        x = torch.from_numpy(x).to(dt[in_dtype]).float().numpy()    # the stored values
    got = _run(_device(cfgs[0], wts, bias), x, cstep_pad=cstep_pad, dtype=dt[in_dtype],
               out_dtype=dt[out_dtype])
    _, ref, _ = oracle.decomposed_conv3d(cfgs[1], x, wts, bias)
    assert_close(got, ref)


# (64, 128, 10x12): the implicit-GEMM kernel; (64, 128, 6x120): the halo
# kernel; (128, 3): the narrow output kernel; (3, 128): the RGB input kernel
@pytest.mark.parametrize("cin,cout,hw", [(64, 128, (10, 12)), (64, 128, (6, 120)),
                                         (128, 3, (10, 256)), (3, 128, (16, 16))])
def test_conv3d_16bit_outputs_round_the_fp32_output(cin, cout, hw):
    """bf16 and fp16 outputs are the round-to-nearest-even of the fp32
    output of the same call (one rounding of the fp32 result)."""
    import torch
    cfgs = _cfg(cin, cout)
    x, wts, bias = _case(cin, cout, 2, hw[0], hw[1], cfgs, 29 + cin)
    x = bf16_round(x)
    conv = _device(cfgs[0], wts, bias)
    outs = {odt: _run(conv, x, dtype=torch.bfloat16, out_dtype=odt)
            for odt in (torch.float32, torch.bfloat16, torch.float16)}
    ref = outs[torch.float32]
    np.testing.assert_array_equal(outs[torch.bfloat16], bf16_round(ref))
    np.testing.assert_array_equal(outs[torch.float16], ref.astype(np.float16).astype(np.float32))
    _check(ref, x, wts, bias, cfgs[1])


# 6x10 frames copy the memory in front of the staged input (a DMA group of
# 8 rows can straddle two frames); 8x10 frames read it in place, except with
# 16 input channels (16-channel pixels always copy it); the halo kernel's
# 5x120 frames always read it in place
@pytest.mark.parametrize("split", [1, 2])
@pytest.mark.parametrize("hw", [(6, 10), (8, 10), (5, 120)])   # (5, 120): the halo kernel
@pytest.mark.parametrize("reuse", [False, True])
@pytest.mark.parametrize("cin", [64, 16])
def test_conv3d_memory_chains_slices(split, hw, reuse, cin):
    cfgs = _cfg(cin, 128)
    x, wts, bias = _case(cin, 128, 5, hw[0], hw[1], cfgs, 11)
    conv = _device(cfgs[0], wts, bias)
    a = _run(conv, x[:, :split], keep_memory=True)
    b = _run(conv, x[:, split:], use_memory=True, keep_memory=True, reuse_memory_buffer=reuse)
    _, ref, _ = oracle.decomposed_conv3d(cfgs[1], x, wts, bias)   # the unsplit run
    got = np.concatenate([a, b], axis=1)
    assert_close(got, ref)
    _, tight, _ = oracle.decomposed_conv3d(cfgs[1], bf16_round(x), bf16_round(wts), bias)
    assert float(np.max(np.abs(got - tight))) <= 1e-4 * max(1.0, float(np.max(np.abs(tight))))
    # a third slice of one frame: its memory mixes the old memory and the input
    c = _run(conv, x[:, 4:], use_memory=True, keep_memory=True, reuse_memory_buffer=reuse)
    _, ref3, _ = oracle.decomposed_conv3d(cfgs[1], np.concatenate([x, x[:, 4:]], 1), wts, bias)
    assert_close(c, ref3[:, 5:])


def test_conv3d_larger_frame_against_torch():
    """A VAE-shaped layer (128 -> 128, 3x3x3) on 2 frames of 90x160 against
    torch's fp32 conv3d on the CPU over the same bf16-rounded operands."""
    import torch
    cfgs = _cfg(128, 128)
    x, wts, bias = _case(128, 128, 2, 90, 160, cfgs, 3)
    got = _run(_device(cfgs[0], wts, bias), x)
    xp = np.concatenate([np.repeat(bf16_round(x)[:, :1], 2, axis=1), bf16_round(x)], axis=1)
    ref = torch.nn.functional.conv3d(
        torch.from_numpy(xp)[None], torch.from_numpy(bf16_round(wts)).permute(1, 2, 0, 3, 4),
        torch.from_numpy(bias), padding=(0, 1, 1))[0].numpy()
    assert got.shape == ref.shape
    assert float(np.max(np.abs(got - ref))) <= 1e-4 * max(1.0, float(np.max(np.abs(ref))))


# ---- the ncnn-surface layer (decomposed_conv3d.h:29-88) ------------------------

def _layer(cfg_o, wts, bias):
    from common import Layer
    fields = [getattr(cfg_o, n) for n, _ in oracle.Conv3dConfig._fields_]
    params = " ".join(f"{i}={v}" for i, v in enumerate(fields))
    blobs = [np.asarray(fields, np.float32)] + ([bias] if bias is not None else []) + [wts]
    layer = Layer("DecomposedConv3d", params, weights=blobs)
    assert layer.create_code == 0
    assert layer.create_pipeline() == 0
    return layer


@pytest.mark.parametrize("device", [False, True])
def test_layer_forward_host_and_device_blobs(device):
    import torch
    from common import set_vae_memory_state
    cfgs = _cfg(64, 128)
    x, wts, bias = _case(64, 128, 3, 10, 12, cfgs, 21)
    layer = _layer(cfgs[1], wts, bias)
    set_vae_memory_state(0)
    dt = torch.bfloat16 if device else None
    xin = torch.from_numpy(x).to(torch.bfloat16).float().numpy() if device else x
    code, got = layer.forward_planar(xin, (12, 10, 3, 64), (12, 10, 3, 128), device=device, dtype=dt)
    assert code == 0
    _, ref, _ = oracle.decomposed_conv3d(cfgs[1], xin, wts, bias)
    assert_close(got, ref)


def test_layer_memory_states_chain_slices():
    from common import set_vae_memory_state
    cfgs = _cfg(32, 64)
    x, wts, bias = _case(32, 64, 6, 8, 8, cfgs, 5)
    layer = _layer(cfgs[1], wts, bias)
    _, full, _ = oracle.decomposed_conv3d(cfgs[1], x, wts, bias)
    outs = []
    # the VAE driver's sequence: a first slice that starts the memory, then
    # slices that continue it (seedvr2_vae.cpp:424-447)
    for i, (a, b) in enumerate([(0, 2), (2, 3), (3, 6)]):
        set_vae_memory_state(1 if i == 0 else 2)
        code, out = layer.forward_planar(x[:, a:b], (8, 8, b - a, 32), (8, 8, b - a, 64))
        assert code == 0
        outs.append(out)
    assert_close(np.concatenate(outs, axis=1), full)
    # DISABLED forgets the memory: the prefix is head frames again
    set_vae_memory_state(0)
    code, out = layer.forward_planar(x[:, 3:6], (8, 8, 3, 32), (8, 8, 3, 64))
    _, ref, _ = oracle.decomposed_conv3d(cfgs[1], x[:, 3:6], wts, bias)
    assert code == 0
    assert_close(out, ref)


def test_layer_rejects_mismatched_blobs():
    from common import set_vae_memory_state
    cfgs = _cfg(32, 64)
    x, wts, bias = _case(32, 64, 2, 8, 8, cfgs, 9)
    layer = _layer(cfgs[1], wts, bias)
    set_vae_memory_state(0)
    code, _ = layer.forward_planar(x[:16], (8, 8, 2, 16), (8, 8, 2, 64))   # wrong channels
    assert code == -1
    set_vae_memory_state(1)
    assert layer.forward_planar(x, (8, 8, 2, 32), (8, 8, 2, 64))[0] == 0
    set_vae_memory_state(2)   # the memory holds 8x8 frames: a 6x8 slice is refused
    code, _ = layer.forward_planar(x[:, :, :6], (8, 6, 2, 32), (8, 6, 2, 64))
    assert code == -1
    assert layer.conv_memory(reset=True) == 0
    assert layer.forward_planar(x[:, :, :6], (8, 6, 2, 32), (8, 6, 2, 64))[0] == 0
    set_vae_memory_state(0)


# ---- layers of at most 3 output channels (conv3d_narrow_kernels.hip) ----------
# The VAE's RGB output conv and its kin (3x3x3, unit strides, one pixel of
# padding, 16..128 input channels) run the narrow kernel, whose temporal
# memory holds partial sums of the next forward's first two output frames.
# The chains below compare slices against the oracle run on the whole clip:
# head frames, frames that need several workgroups per pixel (more than 6
# output frames with the memory's two), memory buffers rewritten in place,
# single-frame slices, ragged strips and rows read element by element.

@pytest.mark.parametrize("cin,cout", [(128, 3), (64, 1), (16, 2)])
@pytest.mark.parametrize("hw", [(6, 10), (9, 136), (5, 250)])
@pytest.mark.parametrize("reuse", [False, True])
def test_conv3d_narrow_memory_chains_slices(cin, cout, hw, reuse):
    cfgs = _cfg(cin, cout)
    x, wts, bias = _case(cin, cout, 14, hw[0], hw[1], cfgs, 5 + cin + cout)
    conv = _device(cfgs[0], wts, bias)
    outs = []
    # 6 frames with head frames: 6 output frames + 2 memory frames = 2 groups;
    # then 5 (2 groups, the in-place memory read from a copy), 1, 2
    for i, (a, b) in enumerate([(0, 6), (6, 11), (11, 12), (12, 14)]):
        outs.append(_run(conv, x[:, a:b], use_memory=i > 0, keep_memory=True,
                         reuse_memory_buffer=reuse))
    got = np.concatenate(outs, axis=1)
    _, ref, _ = oracle.decomposed_conv3d(cfgs[1], x, wts, bias)
    assert got.shape == ref.shape
    assert_close(got, ref)
    _, tight, _ = oracle.decomposed_conv3d(cfgs[1], bf16_round(x), bf16_round(wts), bias)
    assert float(np.max(np.abs(got - tight))) <= 1e-4 * max(1.0, float(np.max(np.abs(tight))))


@pytest.mark.parametrize("head", [0, 1, 2, 4])
def test_conv3d_narrow_head_frames(head):
    cfgs = _cfg(32, 3, head=head)
    x, wts, bias = _case(32, 3, 4, 7, 129, cfgs, 40 + head)
    _check(_run(_device(cfgs[0], wts, bias), x), x, wts, bias, cfgs[1])


@pytest.mark.parametrize("in_dtype,out_dtype", [("bf16", "bf16"), ("f16", "f32"), ("f32", "f16"),
                                                ("f32", "f32")])
@pytest.mark.parametrize("cstep_pad", [0, 4])
def test_conv3d_narrow_blob_types(in_dtype, out_dtype, cstep_pad):
    import torch
    dt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
    cfgs = _cfg(128, 3)
    x, wts, bias = _case(128, 3, 3, 10, 256, cfgs, 17)
    if in_dtype != "f32":
        x = torch.from_numpy(x).to(dt[in_dtype]).float().numpy()    # the stored values
    conv = _device(cfgs[0], wts, bias)
    a = _run(conv, x[:, :1], cstep_pad=cstep_pad, dtype=dt[in_dtype], out_dtype=dt[out_dtype],
             keep_memory=True)
    b = _run(conv, x[:, 1:], cstep_pad=cstep_pad, dtype=dt[in_dtype], out_dtype=dt[out_dtype],
             use_memory=True, keep_memory=True)
    _, ref, _ = oracle.decomposed_conv3d(cfgs[1], x, wts, bias)
    assert_close(np.concatenate([a, b], axis=1), ref)


def test_conv3d_narrow_720p_rows_against_torch():
    """The RGB output conv (128 -> 3) on 2 frames of 90 x 1280 pixels (ten
    128-column strips, bands of rows over the CUs) continuing a memory,
    against torch's fp32 conv3d on the CPU over the same bf16-rounded
    operands."""
    import torch
    cfgs = _cfg(128, 3)
    x, wts, bias = _case(128, 3, 4, 90, 1280, cfgs, 23)
    conv = _device(cfgs[0], wts, bias)
    a = _run(conv, x[:, :2], keep_memory=True)
    b = _run(conv, x[:, 2:], use_memory=True, keep_memory=True)
    got = np.concatenate([a, b], axis=1)
    xp = np.concatenate([np.repeat(bf16_round(x)[:, :1], 2, axis=1), bf16_round(x)], axis=1)
    ref = torch.nn.functional.conv3d(
        torch.from_numpy(xp)[None], torch.from_numpy(bf16_round(wts)).permute(1, 2, 0, 3, 4),
        torch.from_numpy(bias), padding=(0, 1, 1))[0].numpy()
    assert got.shape == ref.shape
    assert float(np.max(np.abs(got - ref))) <= 1e-4 * max(1.0, float(np.max(np.abs(ref))))


def test_conv3d_narrow_rejects_extra_padding():
    cfgs = _cfg(128, 3)
    n = ctypes.c_size_t()
    assert capi.lib().s2_conv3d_workspace_bytes_padded(ctypes.byref(cfgs[0]), 2, 8, 8, 1, 0, 0,
                                                       ctypes.byref(n)) != 0


# ---- at most 8 input channels, 3x3x3, unit strides (conv3d_rgbin_kernel) ------
# The encoder's RGB-input conv and its kin run with the output channels as the
# MFMA rows; 32..128 outputs in multiples of 32, ragged strips and rows, slice
# chains through the memory (copied in front of the staged input), every
# output type, rows that leave in 16-byte runs (widths a multiple of 8) and
# rows that do not.

@pytest.mark.parametrize("cin,cout,frames,h,w", [
    (3, 128, 4, 9, 200),     # two strips, the second ragged
    (8, 64, 3, 7, 130),      # two waves idle, a strip of 2 pixels
    (3, 32, 2, 5, 10),       # one wave of output channels
    (5, 96, 3, 33, 128),     # one full strip, rows over several bands
    (8, 64, 2, 6, 136),      # 16-byte output runs with two waves idle
])
def test_conv3d_rgb_input(cin, cout, frames, h, w):
    cfgs = _cfg(cin, cout)
    x, wts, bias = _case(cin, cout, frames, h, w, cfgs, 70 + cin + cout)
    _check(_run(_device(cfgs[0], wts, bias), x), x, wts, bias, cfgs[1])


@pytest.mark.parametrize("out_dtype,w", [("bf16", 150), ("bf16", 152), ("f16", 150),
                                         ("f16", 152), ("f32", 152)])
def test_conv3d_rgb_input_chain_and_types(out_dtype, w):
    # widths a multiple of 8 take the 16-byte store path for 16-bit outputs
    import torch
    dt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
    cfgs = _cfg(3, 128, head=1)
    x, wts, bias = _case(3, 128, 6, 12, w, cfgs, 90)
    # outputs of magnitude below 4, where one bf16 rounding stays under the
    # 2e-2 bar (1.4 M outputs of unit variance reach 5 and beyond)
    x = (0.5 * x).astype(np.float32)
    conv = _device(cfgs[0], wts, bias)
    parts = []
    for i, (a, b) in enumerate([(0, 2), (2, 5), (5, 6)]):
        parts.append(_run(conv, x[:, a:b], out_dtype=dt[out_dtype], use_memory=i > 0,
                          keep_memory=True))
    _, ref, _ = oracle.decomposed_conv3d(cfgs[1], x, wts, bias)
    assert_close(np.concatenate(parts, axis=1), ref)
