"""AdaptiveWindowAttention on the GPU against the CPU oracle.

Inputs are seeded N(0,1) activations (rounded to bf16 where the device path
reads bf16, with the oracle consuming the same rounded values) and norm
weights 1+N(0,0.02) ("peaky", a real softmax) or N(0,0.02) ("literal").
Bar: max-abs <= 2e-2 and cosine >= 0.9999 against the fp32 oracle; window
tables bit-exact.  The reference CPU forward restated by the oracle is
src/seedvr2/adaptive_window_attention.cpp:764-978."""
import os

import numpy as np
import pytest

import oracle
from common import (COSINE_TOL, MAX_ABS_TOL, Layer, assert_close, awa_param_string,
                    bf16_round, make_awa_inputs, oracle_awa)
from seedvr2_ncnn_amd import capi

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def torch_mod():
    import torch
    assert capi.device_count() >= 1, "no gfx950 device visible to libseedvr2_hip"
    return torch


def _run_capi(case, heads, d, target, shifted, pairs, shapes, text_lengths, bf16_in, out_dtype,
              official=False, split=False, eps=1e-5, in_dtype=None):
    torch = torch_mod()
    inner = heads * d
    dt = in_dtype or (torch.bfloat16 if bf16_in else torch.float32)
    v = torch.from_numpy(case["video"]).to("cuda").to(dt)
    t = torch.from_numpy(case["text"]).to("cuda").to(dt)
    if split:
        vq, vk, vv = (v[:, i * inner:(i + 1) * inner].contiguous() for i in range(3))
        tq, tk, tv = (t[:, i * inner:(i + 1) * inner].contiguous() for i in range(3))
    else:
        vq, vk, vv = (v[:, i * inner:(i + 1) * inner] for i in range(3))
        tq, tk, tv = (t[:, i * inner:(i + 1) * inner] for i in range(3))
    norms = torch.from_numpy(case["norms"]).cuda()
    freqs = torch.from_numpy(case["freqs"]).cuda()
    cfg = capi.awa_config(heads, d, target, shifted, eps, pairs, official_bf16=official)
    with capi.AwaPlan(cfg, shapes, text_lengths) as plan:
        ov, ot = capi.awa_forward(plan, norms, freqs, vq, vk, vv, tq, tk, tv, out_dtype=out_dtype)
        torch.cuda.synchronize()
    return ov.float().cpu().numpy(), ot.float().cpu().numpy()


# ---- window tables -------------------------------------------------------------------

TABLE_CASES = [
    ([(1, 32, 32)], (1, 8, 8)), ([(1, 64, 64)], (4, 3, 3)), ([(6, 45, 80)], (4, 3, 3)),
    ([(3, 17, 29), (1, 8, 8), (7, 45, 80)], (4, 3, 3)), ([(2, 5, 3)], (2, 5, 2)),
    ([(21, 90, 160)], (4, 3, 3)),
]


@pytest.mark.parametrize("shifted", [0, 1])
def test_device_window_tables_bit_exact(shifted):
    torch = torch_mod()
    for shapes, target in TABLE_CASES:
        p = oracle.plan(shapes, target, shifted)
        cfg = capi.awa_config(8, 64, target, shifted, 1e-5, 10)
        with capi.AwaPlan(cfg, shapes, [7] * len(shapes)) as plan:
            idx, inv, pos = plan.tables()
            torch.cuda.synchronize()
            wins, counts = plan.windows()
        np.testing.assert_array_equal(np.asarray(wins, np.int32).reshape(-1, 9), p.windows)
        np.testing.assert_array_equal(counts, p.sample_window_count)
        np.testing.assert_array_equal(idx.cpu().numpy(), p.video_indices)
        np.testing.assert_array_equal(inv.cpu().numpy(), p.inverse_video_indices)
        np.testing.assert_array_equal(pos.cpu().numpy(), p.local_positions)


# ---- committed fixture ---------------------------------------------------------------------

@pytest.mark.parametrize("shifted", [0, 1])
def test_tiny_fixture(shifted):
    f = np.load(os.path.join(GOLDEN, "awa_tiny.npz"))
    heads, d, pairs, *target = [int(x) for x in f["config"]]
    shapes = [tuple(int(x) for x in s) for s in f["video_shapes"]]
    tl = [int(x) for x in f["text_lengths"]]
    case = dict(video=f["video"], text=f["text"], norms=f["norms"], freqs=f["freqs"])
    import torch
    ov, ot = _run_capi(case, heads, d, target, shifted, pairs, shapes, tl, False, torch.float32)
    assert_close(ov, f[f"out_video_{shifted}"], "video")
    assert_close(ot, f[f"out_text_{shifted}"], "text")


# ---- single-layer configuration on the ncnn surface, fp32 host blobs ---------------

def test_layer_grid_32x32_dim512_8x64_fp32_host_blobs():
    """1x32x32 grid, D=512, 8 heads x 64, target (1,8,8): 16 windows of 8x8,
    unshifted, fp32 host blobs through the ncnn-surface layer."""
    torch_mod()
    shapes, tl = [(1, 32, 32)], [64]
    heads, d, pairs, target = 8, 64, 10, (1, 8, 8)
    case = make_awa_inputs(101, shapes, tl, heads, d, pairs, peaky=False)
    layer = Layer("AdaptiveWindowAttention", awa_param_string(heads, d, target, 0, 1e-5, pairs),
                  [case["norms"][i] for i in range(4)] + [case["freqs"]])
    assert layer.create_code == 0 and layer.create_pipeline() == 0
    inner = heads * d
    blobs = [case["video"], case["text"], np.asarray(shapes[0], np.float32), np.asarray(tl, np.float32)]
    outs = [((1024, inner), np.float32), ((64, inner), np.float32)]
    code, (ov, ot) = layer.forward(blobs, outs)
    assert code == 0
    rv, rt = oracle_awa(case, heads, d, target, 0, 1e-5, pairs, shapes, tl)
    assert_close(ov, rv, "video")
    assert_close(ot, rt, "text")


@pytest.mark.parametrize("shifted", [0, 1])
def test_layer_split_form_int32_shapes_peaky(shifted):
    torch_mod()
    shapes, tl = [(2, 12, 20), (1, 9, 7)], [5, 70]
    heads, d, pairs, target = 2, 128, 21, (4, 3, 3)
    case = make_awa_inputs(202 + shifted, shapes, tl, heads, d, pairs)
    inner = heads * d
    layer = Layer("AdaptiveWindowAttention",
                  awa_param_string(heads, d, target, shifted, 1e-5, pairs, int32_shapes=True),
                  [case["norms"][i] for i in range(4)] + [case["freqs"]])
    assert layer.create_code == 0
    v, t = case["video"], case["text"]
    blobs = [v[:, :inner], v[:, inner:2 * inner], v[:, 2 * inner:],
             t[:, :inner], t[:, inner:2 * inner], t[:, 2 * inner:],
             np.asarray(shapes, np.int32), np.asarray(tl, np.int32).reshape(-1, 1)]
    lv = sum(a * b * c for a, b, c in shapes)
    code, (ov, ot) = layer.forward(blobs, [((lv, inner), np.float32), ((sum(tl), inner), np.float32)])
    assert code == 0
    rv, rt = oracle_awa(case, heads, d, target, shifted, 1e-5, pairs, shapes, tl)
    assert_close(ov, rv, "video")
    assert_close(ot, rt, "text")


def test_layer_device_blobs_bf16_zero_copy():
    """Device bf16 blobs (HipDeviceAllocator) run zero-copy and return bf16
    device blobs; shapes come from the runtime state (no shape blobs)."""
    torch = torch_mod()
    shapes, tl = [(2, 16, 16)], [64]
    heads, d, pairs, target = 4, 128, 21, (4, 3, 3)
    case = make_awa_inputs(303, shapes, tl, heads, d, pairs, bf16=True)
    inner = heads * d
    layer = Layer("AdaptiveWindowAttention", awa_param_string(heads, d, target, 1, 1e-5, pairs),
                  [case["norms"][i] for i in range(4)] + [case["freqs"]])
    layer.set_state(shapes, tl)
    v = torch.from_numpy(case["video"]).cuda().to(torch.bfloat16)
    t = torch.from_numpy(case["text"]).cuda().to(torch.bfloat16)
    code, (ov, ot) = layer.forward([v, t, None, None],
                                   [((512, inner), torch.bfloat16), ((64, inner), torch.bfloat16)],
                                   device_out=True)
    assert code == 0
    rv, rt = oracle_awa(case, heads, d, target, 1, 1e-5, pairs, shapes, tl)
    assert_close(ov.float().cpu().numpy(), rv, "video")
    assert_close(ot.float().cpu().numpy(), rt, "text")


def test_layer_device_blobs_fp16_zero_copy():
    """Device blobs of elemsize 2 under ncnn's use_fp16_storage are fp16: they
    run zero-copy and return fp16 device blobs."""
    torch = torch_mod()
    shapes, tl = [(2, 16, 16)], [64]
    heads, d, pairs, target = 4, 128, 21, (4, 3, 3)
    case = make_awa_inputs(313, shapes, tl, heads, d, pairs, fp16=True)
    inner = heads * d
    layer = Layer("AdaptiveWindowAttention", awa_param_string(heads, d, target, 1, 1e-5, pairs),
                  [case["norms"][i] for i in range(4)] + [case["freqs"]])
    layer.set_storage(fp16=True, bf16=False)
    layer.set_state(shapes, tl)
    v = torch.from_numpy(case["video"]).cuda().to(torch.float16)
    t = torch.from_numpy(case["text"]).cuda().to(torch.float16)
    code, (ov, ot) = layer.forward([v, t, None, None],
                                   [((512, inner), torch.float16), ((64, inner), torch.float16)],
                                   device_out=True)
    assert code == 0
    rv, rt = oracle_awa(case, heads, d, target, 1, 1e-5, pairs, shapes, tl)
    assert_close(ov.float().cpu().numpy(), rv, "video")
    assert_close(ot.float().cpu().numpy(), rt, "text")


# ---- SeedVR2-3B shapes through the C-ABI, bf16 -------------------------------------------

@pytest.mark.parametrize("shifted", [0, 1])
def test_image_grid_64x64_dim2560(shifted):
    """One 1024x1024 image: 1x64x64 tokens, hidden 2560, 20 heads x 128."""
    import torch
    shapes, tl = [(1, 64, 64)], [64]
    case = make_awa_inputs(404 + shifted, shapes, tl, 20, 128, 21, bf16=True)
    rv, rt = oracle_awa(case, 20, 128, (4, 3, 3), shifted, 1e-5, 21, shapes, tl)
    outs = {}
    for out_dtype in (torch.float32, torch.bfloat16):
        ov, ot = _run_capi(case, 20, 128, (4, 3, 3), shifted, 21, shapes, tl, True, out_dtype)
        assert_close(ov, rv, f"video {out_dtype}")
        assert_close(ot, rt, f"text {out_dtype}")
        outs[out_dtype] = (ov, ot)
    # the bf16 output is the round-to-nearest-even of the fp32 one (one rounding)
    for got, ref in zip(outs[torch.bfloat16], outs[torch.float32]):
        np.testing.assert_array_equal(got, bf16_round(ref))


@pytest.mark.parametrize("shifted", [0, 1])
def test_image_grid_64x64_dim2560_fp16(shifted):
    """The same image in fp16 storage (the reference Vulkan path's usual 16-bit
    blobs): fp16 inputs, fp16 and fp32 outputs."""
    import torch
    shapes, tl = [(1, 64, 64)], [64]
    case = make_awa_inputs(414 + shifted, shapes, tl, 20, 128, 21, fp16=True)
    rv, rt = oracle_awa(case, 20, 128, (4, 3, 3), shifted, 1e-5, 21, shapes, tl)
    outs = {}
    for out_dtype in (torch.float16, torch.float32):
        ov, ot = _run_capi(case, 20, 128, (4, 3, 3), shifted, 21, shapes, tl, False, out_dtype,
                           in_dtype=torch.float16)
        assert_close(ov, rv, f"video {out_dtype}")
        assert_close(ot, rt, f"text {out_dtype}")
        outs[out_dtype] = (ov, ot)
    # the fp16 output is the round-to-nearest-even of the fp32 one (one rounding)
    for got, ref in zip(outs[torch.float16], outs[torch.float32]):
        np.testing.assert_array_equal(got, ref.astype(np.float16).astype(np.float32))


@pytest.mark.parametrize("shifted", [0, 1])
def test_video_grid_6x45x80_dim2560(shifted):
    """21 frames at 1280x720: 6x45x80 = 21,600 tokens, ragged shifted windows."""
    import torch
    shapes, tl = [(6, 45, 80)], [64]
    case = make_awa_inputs(505 + shifted, shapes, tl, 20, 128, 21, bf16=True)
    ov, ot = _run_capi(case, 20, 128, (4, 3, 3), shifted, 21, shapes, tl, True, torch.bfloat16)
    rv, rt = oracle_awa(case, 20, 128, (4, 3, 3), shifted, 1e-5, 21, shapes, tl, fast=True)
    assert_close(ov, rv, "video")
    assert_close(ot, rt, "text")


@pytest.mark.parametrize("shifted", [0, 1])
def test_batch_of_video_image_and_ragged_samples_dim2560(shifted):
    """Three samples in one call (720p video, one 1024x1024 image, a ragged
    3x17x29 grid) with different text lengths: windows never mix samples and
    every sample pools its own text over its own windows (:963-974)."""
    import torch
    shapes, tl = [(6, 45, 80), (1, 64, 64), (3, 17, 29)], [64, 32, 77]
    case = make_awa_inputs(909 + shifted, shapes, tl, 20, 128, 21, bf16=True)
    ov, ot = _run_capi(case, 20, 128, (4, 3, 3), shifted, 21, shapes, tl, True, torch.float32)
    rv, rt = oracle_awa(case, 20, 128, (4, 3, 3), shifted, 1e-5, 21, shapes, tl, fast=True)
    assert_close(ov, rv, "video")
    assert_close(ot, rt, "text")


@pytest.mark.parametrize("shifted", [0, 1])
def test_video_grid_6x45x80_dim3072_24_heads(shifted):
    """SeedVR2-7B attention shape: the 720p 21-frame grid, hidden 3072,
    24 heads x 128 (one layer of the 32-block stack)."""
    import torch
    shapes, tl = [(6, 45, 80)], [64]
    case = make_awa_inputs(707 + shifted, shapes, tl, 24, 128, 21, bf16=True)
    ov, ot = _run_capi(case, 24, 128, (4, 3, 3), shifted, 21, shapes, tl, True, torch.bfloat16)
    rv, rt = oracle_awa(case, 24, 128, (4, 3, 3), shifted, 1e-5, 21, shapes, tl, fast=True)
    assert_close(ov, rv, "video")
    assert_close(ot, rt, "text")


# ---- variants ------------------------------------------------------------------------------

@pytest.mark.parametrize("official", [False, True])
def test_official_bf16_attention(official):
    import torch
    shapes, tl = [(3, 10, 14)], [9]
    heads, d, pairs = 3, 128, 21
    case = make_awa_inputs(606, shapes, tl, heads, d, pairs, bf16=True)
    ov, ot = _run_capi(case, heads, d, (4, 3, 3), 1, pairs, shapes, tl, True, torch.float32,
                       official=official)
    rv, rt = oracle_awa(case, heads, d, (4, 3, 3), 1, 1e-5, pairs, shapes, tl, official_bf16=official)
    assert_close(ov, rv, "video")
    assert_close(ot, rt, "text")
    if official:
        # the context is rounded to bf16 before the scatter, as the reference does
        assert np.array_equal(ov.view(np.uint32) & 0xFFFF, np.zeros_like(ov.view(np.uint32)))


def test_official_bf16_non_finite_values():
    """round_bf16 (adaptive_window_attention.cpp:499-508) skips the rounding
    increment for Inf and NaN and then clears the low 16 bits, so a NaN whose
    payload lies only in those bits becomes an infinity (the GLSL copy at
    :50-57 keeps it a NaN); the device follows the CPU forward.  fp32 inputs
    (the only storage that holds such a NaN) with +-Inf, quiet and negative
    NaNs and low-payload NaNs in v: the non-finite pattern of both outputs
    (NaN, +Inf, -Inf per element) equals the oracle's, the finite elements
    meet the path's bar."""
    import torch
    shapes, tl = [(2, 10, 14)], [9]
    heads, d, pairs = 2, 128, 21
    inner = heads * d
    case = make_awa_inputs(808, shapes, tl, heads, d, pairs)
    video, text = case["video"].copy(), case["text"].copy()
    vbits, tbits = video.view(np.uint32), text.view(np.uint32)
    v0 = 2 * inner   # first v column of the fused rows
    specials = [  # (token, head, channel, bits)
        (5, 0, 3, 0x7F800001),      # low-payload NaN -> +Inf
        (37, 1, 10, 0x7F800000),    # +Inf
        (80, 0, 20, 0xFF800000),    # -Inf
        (100, 1, 40, 0x7FC00000),   # quiet NaN
        (120, 0, 50, 0xFFC12345),   # negative NaN with a high payload
        (150, 1, 70, 0xFF800003),   # negative low-payload NaN -> -Inf
    ]
    for tok, h, c, bits in specials:
        vbits[tok, v0 + h * d + c] = bits
    tbits[2, v0 + 1 * d + 60] = 0x7F800002   # a text key's low-payload NaN -> +Inf everywhere
    case["video"], case["text"] = video, text
    ov, ot = _run_capi(case, heads, d, (4, 3, 3), 0, pairs, shapes, tl, False, torch.float32,
                       official=True)
    rv, rt = oracle_awa(case, heads, d, (4, 3, 3), 0, 1e-5, pairs, shapes, tl, official_bf16=True)
    for got, ref, what in ((ov, rv, "video"), (ot, rt, "text")):
        assert np.isposinf(ref).any() and np.isneginf(ref).any() and np.isnan(ref).any(), what
        np.testing.assert_array_equal(np.isnan(got), np.isnan(ref), what + " NaN pattern")
        np.testing.assert_array_equal(np.isposinf(got), np.isposinf(ref), what + " +Inf pattern")
        np.testing.assert_array_equal(np.isneginf(got), np.isneginf(ref), what + " -Inf pattern")
        fin = np.isfinite(ref)
        assert_close(got[fin], ref[fin], what + " finite elements")


def test_literal_weights_and_fp32_inputs_split():
    import torch
    shapes, tl = [(4, 20, 33)], [64]
    heads, d, pairs = 4, 128, 21
    case = make_awa_inputs(707, shapes, tl, heads, d, pairs, peaky=False)
    ov, ot = _run_capi(case, heads, d, (4, 3, 3), 0, pairs, shapes, tl, False, torch.float32, split=True)
    rv, rt = oracle_awa(case, heads, d, (4, 3, 3), 0, 1e-5, pairs, shapes, tl)
    assert_close(ov, rv, "video")
    assert_close(ot, rt, "text")


@pytest.mark.parametrize("d,pairs", [(64, 10), (64, 0), (128, 0)])
def test_head_dims_and_rope_widths(d, pairs):
    import torch
    shapes, tl = [(1, 13, 9), (2, 3, 5)], [1, 130]
    heads = 3
    case = make_awa_inputs(808 + d + pairs, shapes, tl, heads, d, pairs)
    if pairs == 0:
        case["freqs"] = np.zeros(1, np.float32)   # the C-ABI ignores it
        ref_case = dict(case, freqs=np.zeros(1, np.float32))
    else:
        ref_case = case
    ov, ot = _run_capi(case, heads, d, (2, 2, 2), 1, pairs, shapes, tl, True, torch.float32)
    rv, rt = oracle_awa(ref_case, heads, d, (2, 2, 2), 1, 1e-5, pairs, shapes, tl)
    assert_close(ov, rv, "video")
    assert_close(ot, rt, "text")


def test_repeated_forward_is_deterministic():
    import torch
    shapes, tl = [(2, 30, 40)], [64]
    case = make_awa_inputs(909, shapes, tl, 4, 128, 21, bf16=True)
    a = _run_capi(case, 4, 128, (4, 3, 3), 1, 21, shapes, tl, True, torch.float32)
    b = _run_capi(case, 4, 128, (4, 3, 3), 1, 21, shapes, tl, True, torch.float32)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_layer_rebuilds_plan_and_rope_table_when_shapes_change():
    """One layer instance fed three shape sets in turn (A, B, A): each change
    of shapes rebuilds the plan, whose cached RoPE table the layer fills from
    its frequency weights before the forward; every result is at the oracle
    bar."""
    torch_mod()
    heads, d, pairs, target = 2, 128, 21, (4, 3, 3)
    layer = None
    for shapes, tl, seed in (([(2, 12, 20)], [33], 301), ([(1, 9, 7)], [70], 302),
                             ([(2, 12, 20)], [33], 303)):
        case = make_awa_inputs(seed, shapes, tl, heads, d, pairs)
        if layer is None:
            weights = dict(norms=case["norms"], freqs=case["freqs"])
            layer = Layer("AdaptiveWindowAttention", awa_param_string(heads, d, target, 1, 1e-5, pairs),
                          [weights["norms"][i] for i in range(4)] + [weights["freqs"]])
            assert layer.create_code == 0
        case.update(weights)   # the layer keeps its first weights
        lv = sum(a * b * c for a, b, c in shapes)
        inner = heads * d
        blobs = [case["video"], case["text"], np.asarray(shapes[0], np.float32),
                 np.asarray(tl, np.float32)]
        code, (ov, ot) = layer.forward(blobs, [((lv, inner), np.float32), ((sum(tl), inner), np.float32)])
        assert code == 0
        rv, rt = oracle_awa(case, heads, d, target, 1, 1e-5, pairs, shapes, tl)
        assert_close(ov, rv, f"video {shapes}")
        assert_close(ot, rt, f"text {shapes}")


# ---- softmax reference: fixed score bound and running maximum ---------------------------
# The attention kernel takes the softmax relative to a fixed reference when the
# norm weights bound every exponent to |s * log2(e) / sqrt(d)| <= 60, and
# relative to a running row maximum otherwise.  The official bf16 mode rounds
# q and k to bf16 in the oracle as on the device, so even very sharp softmaxes
# compare at the usual bar.
NORM_CASES = {
    "unit": (1.0, 1.0, 1.0, 1.0),          # bound ~18 (d = 128): fixed reference
    "near_limit": (1.7, 1.7, 1.7, 1.7),    # bound ~54: fixed reference
    "large": (2.4, 2.4, 2.4, 2.4),         # bound ~100: running maximum
    "text_q_only": (1.0, 1.0, 40.0, 1.0),  # only the text q weights are large
    "text_k_only": (1.0, 1.0, 1.0, 30.0),
}


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("name", list(NORM_CASES))
def test_softmax_reference_paths(name, d):
    import torch
    shapes, tl = [(2, 16, 24), (1, 9, 13)], [64, 7]
    heads, pairs = 4, (21 if d == 128 else 10)
    case = make_awa_inputs(1200 + d + len(name), shapes, tl, heads, d, pairs, bf16=True)
    g = np.random.default_rng(1300 + d)
    scales = np.asarray(NORM_CASES[name], np.float32)[:, None]
    case["norms"] = (scales * (1.0 + 0.02 * g.standard_normal((4, d)))).astype(np.float32)
    for shifted in (0, 1):
        ov, ot = _run_capi(case, heads, d, (4, 3, 3), shifted, pairs, shapes, tl, True,
                           torch.float32, official=True)
        rv, rt = oracle_awa(case, heads, d, (4, 3, 3), shifted, 1e-5, pairs, shapes, tl,
                            official_bf16=True)
        assert np.isfinite(ov).all() and np.isfinite(ot).all()
        assert_close(ov, rv, f"{name} video (shifted={shifted})")
        assert_close(ot, rt, f"{name} text (shifted={shifted})")
