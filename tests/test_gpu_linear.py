"""SharedLinear on the GPU against the CPU oracle (src/seedvr2/shared_linear.cpp:83-96):
y = act(x W^T + b) for the video and text streams in one grouped launch.

The device computes in bf16 with fp32 accumulation: W is held in bf16, fp32
activations are rounded to bf16 as they are staged.  Two comparisons per
case: against the fp32 oracle on the unrounded inputs with the path's bar
(max-abs <= 2e-2, cosine >= 0.9999), and against the oracle on the
bf16-rounded inputs with a tight bound that isolates the kernel's own
arithmetic (accumulation order only)."""
import os

import numpy as np
import pytest

import oracle
from common import Layer, assert_close, bf16_round
from seedvr2_ncnn_amd import capi

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
THREADS = min(16, os.cpu_count() or 1)


def _gpu_linear(xv, xt, w, b, act, x_bf16, y_bf16):
    import torch
    assert capi.device_count() >= 1
    xdt = torch.bfloat16 if x_bf16 else torch.float32
    ydt = torch.bfloat16 if y_bf16 else torch.float32
    tv = torch.from_numpy(xv).cuda().to(xdt)
    tt = torch.from_numpy(xt).cuda().to(xdt) if xt is not None else None
    wb = capi.cast_f32_to_bf16(torch.from_numpy(w).cuda())
    tb = torch.from_numpy(b).cuda() if b is not None else None
    yv, yt = capi.shared_linear(tv, tt, wb, tb, act, out_dtype=ydt)
    torch.cuda.synchronize()
    return yv.float().cpu().numpy(), (yt.float().cpu().numpy() if yt is not None else None)


def _tight(got, xr, wr, b, act, rows=None):
    ref = oracle.linear(xr, wr, b, act, rows=rows, threads=THREADS)
    scale = max(1.0, float(np.max(np.abs(ref))))
    err = float(np.max(np.abs(got - ref)))
    return err / scale


# the last three put video and text rows in one 256-row tile: the video tail
# ends off (257, 300) or on (250 -> 256) an 8-row boundary, and n = 260 takes
# the direct-store epilogue
SHAPES = [(1, 0, 8, 16), (37, 5, 24, 40), (130, 64, 72, 136), (64, 64, 128, 2560),
          (257, 3, 2560, 96), (300, 40, 128, 260), (250, 70, 192, 512)]


@pytest.mark.parametrize("mv,mt,k,n", SHAPES)
@pytest.mark.parametrize("act", [0, 1])
def test_small_shapes(mv, mt, k, n, act):
    g = np.random.default_rng(mv * 7 + k + act)
    xv = g.standard_normal((mv, k)).astype(np.float32)
    xt = g.standard_normal((mt, k)).astype(np.float32) if mt else None
    w = (0.02 * g.standard_normal((n, k))).astype(np.float32)
    b = (0.02 * g.standard_normal(n)).astype(np.float32) if act == 0 or k % 16 else None
    for x_bf16, y_bf16 in ((False, False), (True, True), (True, False)):
        yv, yt = _gpu_linear(xv, xt, w, b, act, x_bf16, y_bf16)
        assert_close(yv, oracle.linear(xv, w, b, act, threads=THREADS), "video")
        # kernel arithmetic: same bf16 operands, fp32 accumulation
        tol = 1e-2 if y_bf16 else 2e-4
        assert _tight(yv, bf16_round(xv), bf16_round(w), b, act) < tol
        if mt:
            assert_close(yt, oracle.linear(xt, w, b, act, threads=THREADS), "text")


def test_tiny_fixture():
    f = np.load(os.path.join(GOLDEN, "linear_tiny.npz"))
    yv, yt = _gpu_linear(f["x_video"], f["x_text"], f["weight"], f["bias"], 1, False, False)
    assert_close(yv, f["y_video"], "video")
    assert_close(yt, f["y_text"], "text")


# Block GEMMs at the 720p video shape, 21,600 video + 64 text tokens: the
# SeedVR2-3B block (hidden 2560) and the SeedVR2-7B block (hidden 3072).
VIDEO_GEMMS = [("qkv", 2560, 7680, 0), ("out", 2560, 2560, 0), ("mlp_up_gelu", 2560, 10240, 1),
               ("mlp_down", 10240, 2560, 0),
               ("qkv_3072", 3072, 9216, 0), ("out_3072", 3072, 3072, 0),
               ("mlp_up_gelu_3072", 3072, 12288, 1), ("mlp_down_3072", 12288, 3072, 0)]


@pytest.mark.parametrize("name,k,n,act", VIDEO_GEMMS)
def test_video_shape_gemms(name, k, n, act):
    import torch
    g = np.random.default_rng(sum(map(ord, name)))
    mv, mt = 21600, 64
    xv = g.standard_normal((mv, k), dtype=np.float32)
    xt = g.standard_normal((mt, k), dtype=np.float32)
    w = (0.02 * g.standard_normal((n, k), dtype=np.float32))
    b = (0.02 * g.standard_normal(n)).astype(np.float32)
    xv, xt = bf16_round(xv), bf16_round(xt)
    # fp32 output carries the parity bar; the bf16 output must be the
    # round-to-nearest-even of that same fp32 result (one rounding).
    yv, yt = _gpu_linear(xv, xt, w, b, act, True, False)
    yv16, yt16 = _gpu_linear(xv, xt, w, b, act, True, True)
    np.testing.assert_array_equal(yv16, bf16_round(yv))
    np.testing.assert_array_equal(yt16, bf16_round(yt))
    rows = np.concatenate([np.arange(0, 3), np.arange(127, 131), g.integers(0, mv, 40),
                           np.arange(mv - 5, mv)]).astype(np.int32)
    assert_close(yv[rows], oracle.linear(xv, w, b, act, rows=rows, threads=THREADS), "video rows")
    assert_close(yt, oracle.linear(xt, w, b, act, threads=THREADS), "text")
    # whole output against torch (hipBLASLt) on the same bf16 operands
    ref = (torch.from_numpy(xv).cuda() @ torch.from_numpy(bf16_round(w)).cuda().T
           + torch.from_numpy(b).cuda())
    if act:
        ref = torch.nn.functional.gelu(ref)
    d = (torch.from_numpy(yv).cuda() - ref).abs().max().item()
    assert d < 2e-3, d


def test_layer_host_fp32_and_device_bf16():
    import torch
    g = np.random.default_rng(5)
    k, n, mv, mt = 256, 384, 300, 64
    w = (0.02 * g.standard_normal((n, k))).astype(np.float32)
    b = (0.02 * g.standard_normal(n)).astype(np.float32)
    xv = g.standard_normal((mv, k)).astype(np.float32)
    xt = g.standard_normal((mt, k)).astype(np.float32)
    layer = Layer("SharedLinear", f"0={n} 1={k} 2=1", [w, b])
    assert layer.create_code == 0 and layer.create_pipeline() == 0
    code, (yv, yt) = layer.forward([xv, xt], [((mv, n), np.float32), ((mt, n), np.float32)])
    assert code == 0
    assert_close(yv, oracle.linear(xv, w, b), "host video")
    assert_close(yt, oracle.linear(xt, w, b), "host text")
    dv = torch.from_numpy(xv).cuda().to(torch.bfloat16)
    dt = torch.from_numpy(xt).cuda().to(torch.bfloat16)
    code, (yv, yt) = layer.forward([dv, dt], [((mv, n), torch.bfloat16), ((mt, n), torch.bfloat16)],
                                   device_out=True)
    assert code == 0
    assert_close(yv.float().cpu().numpy(), oracle.linear(xv, w, b), "device video")
    assert_close(yt.float().cpu().numpy(), oracle.linear(xt, w, b), "device text")


def test_layer_gelu_activation_param():
    g = np.random.default_rng(6)
    k, n = 64, 96
    w = (0.1 * g.standard_normal((n, k))).astype(np.float32)
    layer = Layer("SharedLinear", f"0={n} 1={k} 2=0 3=1", [w])
    xv = g.standard_normal((10, k)).astype(np.float32)
    xt = g.standard_normal((2, k)).astype(np.float32)
    code, (yv, yt) = layer.forward([xv, xt], [((10, n), np.float32), ((2, n), np.float32)])
    assert code == 0
    assert_close(yv, oracle.linear(xv, w, None, 1), "video")


def test_text_projection_5120_to_3072():
    """The 64 conditioning tokens of the 7B stack enter at the frontend text
    width 5120 and are projected to the hidden width 3072 once; a small-M,
    long-K GEMM (one 256-row tile)."""
    g = np.random.default_rng(5120)
    k, n, m = 5120, 3072, 64
    x = bf16_round(g.standard_normal((m, k), dtype=np.float32))
    w = (0.02 * g.standard_normal((n, k), dtype=np.float32))
    b = (0.02 * g.standard_normal(n)).astype(np.float32)
    y, _ = _gpu_linear(x, None, w, b, 0, True, False)
    assert_close(y, oracle.linear(x, w, b, threads=THREADS), "text projection")
    assert _tight(y, x, bf16_round(w), b, 0) < 1e-4


@pytest.mark.parametrize("mv,mt,k,n", [(300, 0, 2560, 2560), (1000, 64, 640, 768), (21600, 64, 2560, 2560)])
def test_split_tail_is_deterministic(mv, mt, k, n):
    """Tiles of a partly filled last wave are split along k between
    workgroups and summed by whichever part finishes last; the sum runs in a
    fixed order, so repeated calls give identical bits."""
    g = np.random.default_rng(mv + k)
    xv = bf16_round(g.standard_normal((mv, k), dtype=np.float32))
    xt = bf16_round(g.standard_normal((mt, k), dtype=np.float32)) if mt else None
    w = (0.02 * g.standard_normal((n, k), dtype=np.float32))
    b = (0.02 * g.standard_normal(n)).astype(np.float32)
    outs = [_gpu_linear(xv, xt, w, b, 1, True, False) for _ in range(3)]
    for yv, yt in outs[1:]:
        np.testing.assert_array_equal(yv, outs[0][0])
        if mt:
            np.testing.assert_array_equal(yt, outs[0][1])
    rows = np.concatenate([np.arange(0, 3), g.integers(0, mv, 20), np.arange(mv - 3, mv)]).astype(np.int32)
    assert_close(outs[0][0][rows], oracle.linear(xv, w, b, 1, rows=rows, threads=THREADS), "video rows")
    assert _tight(outs[0][0][rows], xv, bf16_round(w), b, 1, rows=rows) < 2e-4


@pytest.mark.parametrize("mv,mt,k,n", [(300, 40, 128, 260), (1000, 64, 640, 768)])
@pytest.mark.parametrize("act", [0, 1])
def test_fp16_activations(mv, mt, k, n, act):
    """fp16 activations (rounded to bf16, the MFMA operand type, while staged)
    with fp16 and fp32 outputs."""
    import torch
    g = np.random.default_rng(mv + k + 7 * act)
    xv = g.standard_normal((mv, k)).astype(np.float16).astype(np.float32)
    xt = g.standard_normal((mt, k)).astype(np.float16).astype(np.float32)
    w = (0.02 * g.standard_normal((n, k))).astype(np.float32)
    b = (0.02 * g.standard_normal(n)).astype(np.float32)
    tv = torch.from_numpy(xv).cuda().to(torch.float16)
    tt = torch.from_numpy(xt).cuda().to(torch.float16)
    wb = capi.cast_f32_to_bf16(torch.from_numpy(w).cuda())
    tb = torch.from_numpy(b).cuda()
    for odt in (torch.float16, torch.float32):
        yv, yt = capi.shared_linear(tv, tt, wb, tb, act, out_dtype=odt)
        torch.cuda.synchronize()
        assert yv.dtype == odt and yt.dtype == odt
        assert_close(yv.float().cpu().numpy(), oracle.linear(xv, w, b, act, threads=THREADS), "video")
        assert_close(yt.float().cpu().numpy(), oracle.linear(xt, w, b, act, threads=THREADS), "text")
        # kernel arithmetic: the same bf16 operands, fp32 accumulation
        tol = 1e-2 if odt == torch.float16 else 2e-4
        assert _tight(yv.float().cpu().numpy(), bf16_round(xv), bf16_round(w), b, act) < tol


# one full wave of 256 tiles (no split tail), a split tail (860 tiles), and an
# n that is not a multiple of 8 (the direct-store epilogue)
@pytest.mark.parametrize("mv,mt,k,n", [(4000, 64, 256, 4096), (21600, 64, 2560, 2560),
                                       (300, 40, 128, 260)])
@pytest.mark.parametrize("act", [0, 1])
def test_bf16_activations_16bit_outputs(mv, mt, k, n, act):
    """bf16 activations with fp16 and bf16 outputs: each 16-bit output is the
    round-to-nearest-even of the fp32 output of the same call (one rounding
    of the fp32 accumulators), on every epilogue the 256x256-tile kernel
    has."""
    import torch
    g = np.random.default_rng(mv + n + act)
    xv = bf16_round(g.standard_normal((mv, k), dtype=np.float32))
    xt = bf16_round(g.standard_normal((mt, k), dtype=np.float32))
    w = (0.02 * g.standard_normal((n, k), dtype=np.float32))
    b = (0.02 * g.standard_normal(n)).astype(np.float32)
    tv = torch.from_numpy(xv).cuda().to(torch.bfloat16)
    tt = torch.from_numpy(xt).cuda().to(torch.bfloat16)
    wb = capi.cast_f32_to_bf16(torch.from_numpy(w).cuda())
    tb = torch.from_numpy(b).cuda()
    outs = {}
    for odt in (torch.float32, torch.float16, torch.bfloat16):
        yv, yt = capi.shared_linear(tv, tt, wb, tb, act, out_dtype=odt)
        torch.cuda.synchronize()
        assert yv.dtype == odt and yt.dtype == odt
        outs[odt] = (yv.float().cpu().numpy(), yt.float().cpu().numpy())
    yv, yt = outs[torch.float32]
    for got, ref in zip(outs[torch.float16], (yv, yt)):
        np.testing.assert_array_equal(got, ref.astype(np.float16).astype(np.float32))
    for got, ref in zip(outs[torch.bfloat16], (yv, yt)):
        np.testing.assert_array_equal(got, bf16_round(ref))
    rows = np.concatenate([np.arange(0, 3), g.integers(0, mv, 24), np.arange(mv - 3, mv)]).astype(np.int32)
    assert_close(yv[rows], oracle.linear(xv, w, b, act, rows=rows, threads=THREADS), "video rows")
    assert_close(yt, oracle.linear(xt, w, b, act, threads=THREADS), "text")


def test_fp32_activations_medium_shape():
    """fp32 activations take the 128x128-tile path (rounded to bf16 while
    staged): a 4,100-row, K = 2560 -> N = 2560 projection with GELU."""
    g = np.random.default_rng(4100)
    mv, mt, k, n = 4036, 64, 2560, 2560
    xv = g.standard_normal((mv, k), dtype=np.float32)
    xt = g.standard_normal((mt, k), dtype=np.float32)
    w = (0.02 * g.standard_normal((n, k), dtype=np.float32))
    b = (0.02 * g.standard_normal(n)).astype(np.float32)
    yv, yt = _gpu_linear(xv, xt, w, b, 1, False, False)
    rows = np.concatenate([np.arange(0, 4), g.integers(0, mv, 40), np.arange(mv - 4, mv)]).astype(np.int32)
    assert_close(yv[rows], oracle.linear(xv, w, b, 1, rows=rows, threads=THREADS), "video rows")
    assert_close(yt, oracle.linear(xt, w, b, 1, threads=THREADS), "text")
    assert _tight(yv[rows], bf16_round(xv), bf16_round(w), b, 1, rows=rows) < 2e-4



def test_concurrent_streams_keep_their_own_split_scratch():
    """Two SharedLinear calls whose kernels overlap on two streams, both with
    a split-k tail (the 720p out projection: 860 tiles, the last 82 split in
    three): each stream has its own partial-tile scratch, so both results
    equal the same calls made one at a time (bit for bit) and meet the bar
    against the oracle."""
    import torch
    g = np.random.default_rng(2024)
    mv, mt, k, n = 21600, 64, 2560, 2560
    xs = [bf16_round(g.standard_normal((mv + mt, k), dtype=np.float32)) for _ in range(2)]
    ws = [(0.02 * g.standard_normal((n, k), dtype=np.float32)) for _ in range(2)]
    bs = [(0.02 * g.standard_normal(n)).astype(np.float32) for _ in range(2)]
    dx = [torch.from_numpy(x).cuda().to(torch.bfloat16) for x in xs]
    dw = [capi.cast_f32_to_bf16(torch.from_numpy(w).cuda()) for w in ws]
    db = [torch.from_numpy(b).cuda() for b in bs]
    torch.cuda.synchronize()

    def call(i, stream=None):
        return capi.shared_linear(dx[i][:mv], dx[i][mv:], dw[i], db[i], capi.ACT_NONE,
                                  out_dtype=torch.float32, stream=stream)

    alone = [call(i) for i in range(2)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    outs = [[], []]
    for _ in range(4):   # interleaved: the tails of calls on the two streams overlap
        for i in range(2):
            with torch.cuda.stream(streams[i]):
                outs[i].append(call(i, stream=streams[i]))
    torch.cuda.synchronize()
    rows = np.concatenate([np.arange(0, 2), g.integers(0, mv, 24), np.arange(mv - 2, mv)]).astype(np.int32)
    for i in range(2):
        ref_v, ref_t = (t.cpu().numpy() for t in alone[i])
        for yv, yt in outs[i]:
            np.testing.assert_array_equal(yv.cpu().numpy(), ref_v)
            np.testing.assert_array_equal(yt.cpu().numpy(), ref_t)
        assert_close(ref_v[rows], oracle.linear(xs[i][:mv], ws[i], bs[i], rows=rows,
                                                threads=THREADS), f"stream {i} video rows")
        assert_close(ref_t, oracle.linear(xs[i][mv:], ws[i], bs[i], threads=THREADS),
                     f"stream {i} text")
