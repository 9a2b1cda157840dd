"""The fused QKV projection + attention layer (s2_awa_qkv_forward) on the GPU.

Each case runs two checks:
 1. Bit-identity with the separate path it replaces: s2_shared_linear_forward
    writing a bf16 QKV blob, then s2_awa_forward on it.  The fused epilogue
    rounds the projection to bf16 exactly as that blob holds it and applies
    the prologue's RMSNorm and RoPE in the same fp32 operation order, and
    both GEMMs accumulate every output element in the same k order.  The
    shapes are chosen so that neither launch splits k.
 2. Parity with the fp32 oracle: oracle.linear (X W^T + b, the SharedLinear
    forward of shared_linear.cpp:83-96) feeding the oracle's attention
    forward (adaptive_window_attention.cpp:764-978), on the same bf16
    activations and weights, at the bar max-abs <= 2e-2, cosine >= 0.9999.
Cases: regular and shifted windows; odd window sizes, which leave gap rows
in the fused row space; two samples with different text lengths; head_dim
64 and 128; official_bf16_attention; and the 720p shape at full size
(bit-identity only: the oracle's textbook GEMM is too slow there; the
separate path is itself checked against the oracle at that shape)."""
import numpy as np
import pytest

import oracle
from common import assert_close, bf16_round, oracle_awa, rope_freqs
from seedvr2_ncnn_amd import capi

pytestmark = pytest.mark.gpu


def torch_mod():
    import torch
    assert capi.device_count() >= 1, "no gfx950 device visible to libseedvr2_hip"
    return torch


def _inputs(seed, lv, lt, hidden, heads, d, pairs):
    g = np.random.default_rng(seed)
    inner = heads * d
    return dict(
        xv=bf16_round(g.standard_normal((lv, hidden), dtype=np.float32)),
        xt=bf16_round(g.standard_normal((lt, hidden), dtype=np.float32)),
        w=bf16_round(0.02 * g.standard_normal((3 * inner, hidden)).astype(np.float32)),
        b=(0.02 * g.standard_normal(3 * inner)).astype(np.float32),
        norms=(1.0 + 0.02 * g.standard_normal((4, d))).astype(np.float32),
        freqs=rope_freqs(pairs))


def _run(case, shapes, tl, heads, d, pairs, target, shifted, official=False):
    """(fused video, fused text, separate video, separate text) as fp32 numpy."""
    torch = torch_mod()
    inner = heads * d
    bf = torch.bfloat16
    xv = torch.from_numpy(case["xv"]).cuda().to(bf)
    xt = torch.from_numpy(case["xt"]).cuda().to(bf)
    w = torch.from_numpy(case["w"]).cuda().to(bf)
    b = torch.from_numpy(case["b"]).cuda()
    norms = torch.from_numpy(case["norms"]).cuda()
    freqs = torch.from_numpy(case["freqs"]).cuda()
    cfg = capi.awa_config(heads, d, target, shifted, 1e-5, pairs, official_bf16=official)
    with capi.AwaPlan(cfg, shapes, tl) as plan:
        ws = torch.empty(plan.info.workspace_bytes, dtype=torch.uint8, device="cuda")
        # poison the workspace: the fused path must write every row the
        # attention reads (text rows, V^T padding keys) itself
        ws.view(torch.int16).fill_(-1)
        fv, ft = capi.awa_qkv_forward(plan, xv, xt, w, b, norms, freqs, out_dtype=torch.float32,
                                      workspace=ws)
        qv, qt = capi.shared_linear(xv, xt, w, b, capi.ACT_NONE, out_dtype=bf)
        sv, st = capi.awa_forward(plan, norms, freqs, qv[:, :inner], qv[:, inner:2 * inner],
                                  qv[:, 2 * inner:], qt[:, :inner], qt[:, inner:2 * inner],
                                  qt[:, 2 * inner:], out_dtype=torch.float32)
        torch.cuda.synchronize()
    return fv.cpu().numpy(), ft.cpu().numpy(), sv.cpu().numpy(), st.cpu().numpy()


def _oracle(case, shapes, tl, heads, d, pairs, target, shifted, official=False):
    qv = oracle.linear(case["xv"], case["w"], case["b"], 0, threads=8)
    qt = oracle.linear(case["xt"], case["w"], case["b"], 0, threads=8)
    oc = dict(video=qv, text=qt, norms=case["norms"], freqs=case["freqs"])
    return oracle_awa(oc, heads, d, target, shifted, 1e-5, pairs, shapes, tl, official_bf16=official)


CASES = [
    # (shapes, text lengths, heads, head_dim, pairs, target, hidden)
    ([(2, 16, 24), (1, 9, 13)], [64, 7], 4, 128, 21, (4, 3, 3), 512),   # odd window, 2 samples
    ([(1, 32, 32)], [64], 8, 64, 10, (1, 8, 8), 256),                   # cfg1-shaped, d = 64
    ([(1, 64, 64)], [64], 20, 128, 21, (4, 3, 3), 512),                 # cfg2-shaped heads
    ([(3, 17, 29)], [5], 4, 64, 10, (4, 3, 3), 192),                     # ragged, odd sizes
]


@pytest.mark.parametrize("shifted", [0, 1])
@pytest.mark.parametrize("ci", range(len(CASES)))
def test_fused_qkv_matches_separate_path_and_oracle(ci, shifted):
    shapes, tl, heads, d, pairs, target, hidden = CASES[ci]
    lv = sum(t * h * w for t, h, w in shapes)
    case = _inputs(100 + ci, lv, sum(tl), hidden, heads, d, pairs)
    fv, ft, sv, st = _run(case, shapes, tl, heads, d, pairs, target, shifted)
    assert np.all(np.isfinite(fv)) and np.all(np.isfinite(ft))
    np.testing.assert_array_equal(fv, sv)
    np.testing.assert_array_equal(ft, st)
    rv, rt = _oracle(case, shapes, tl, heads, d, pairs, target, shifted)
    assert_close(fv, rv, f"fused video case {ci} shifted={shifted}")
    assert_close(ft, rt, f"fused text case {ci} shifted={shifted}")


def test_fused_qkv_official_bf16():
    shapes, tl, heads, d, pairs, target, hidden = CASES[0]
    lv = sum(t * h * w for t, h, w in shapes)
    case = _inputs(7, lv, sum(tl), hidden, heads, d, pairs)
    fv, ft, sv, st = _run(case, shapes, tl, heads, d, pairs, target, 1, official=True)
    np.testing.assert_array_equal(fv, sv)
    np.testing.assert_array_equal(ft, st)
    rv, rt = _oracle(case, shapes, tl, heads, d, pairs, target, 1, official=True)
    assert_close(fv, rv, "fused official_bf16 video")
    assert_close(ft, rt, "fused official_bf16 text")


@pytest.mark.parametrize("shifted", [0, 1])
def test_fused_qkv_720p_bit_identical(shifted):
    """SeedVR2-3B block shape: 6x45x80 + 64 text tokens, hidden 2560, 20x128."""
    shapes, tl = [(6, 45, 80)], [64]
    case = _inputs(31 + shifted, 21600, 64, 2560, 20, 128, 21)
    fv, ft, sv, st = _run(case, shapes, tl, 20, 128, 21, (4, 3, 3), shifted)
    assert np.all(np.isfinite(fv)) and np.all(np.isfinite(ft))
    np.testing.assert_array_equal(fv, sv)
    np.testing.assert_array_equal(ft, st)


def test_fused_qkv_rejects_unsupported_shapes():
    torch = torch_mod()
    bf = torch.bfloat16
    # heads * head_dim = 128 is not a multiple of 256
    cfg = capi.awa_config(2, 64, (4, 3, 3), 0, 1e-5, 10)
    with capi.AwaPlan(cfg, [(1, 8, 8)], [4]) as plan:
        xv = torch.zeros(64, 256, dtype=bf, device="cuda")
        xt = torch.zeros(4, 256, dtype=bf, device="cuda")
        w = torch.zeros(384, 256, dtype=bf, device="cuda")
        norms = torch.ones(4, 64, device="cuda")
        freqs = torch.ones(10, device="cuda")
        with pytest.raises(capi.S2Error) as e:
            capi.awa_qkv_forward(plan, xv, xt, w, None, norms, freqs)
        assert e.value.code == capi.S2_ERR_INVALID


def test_plan_rope_cache():
    """s2_awa_plan_cache_rope: forwards given the cached frequencies read the
    plan's table and match the uncached forward bit for bit (both the fused
    and the separate path); a different frequency tensor is not served from
    the cache; after the cached tensor is rewritten in place, caching again
    picks up the new values; a NULL pointer clears the cache."""
    torch = torch_mod()
    heads, d, pairs, hidden = 2, 128, 21, 256
    shapes, tl = [(3, 16, 20)], [24]
    lv = 3 * 16 * 20
    case = _inputs(91, lv, 24, hidden, heads, d, pairs)
    bf = torch.bfloat16
    xv = torch.from_numpy(case["xv"]).cuda().to(bf)
    xt = torch.from_numpy(case["xt"]).cuda().to(bf)
    w = torch.from_numpy(case["w"]).cuda().to(bf)
    b = torch.from_numpy(case["b"]).cuda()
    norms = torch.from_numpy(case["norms"]).cuda()
    f1 = torch.from_numpy(case["freqs"]).cuda()
    f2 = (f1 * 0.5).contiguous()
    inner = heads * d
    cfg = capi.awa_config(heads, d, (4, 3, 3), 1, 1e-5, pairs)
    qv, qt = capi.shared_linear(xv, xt, w, b, capi.ACT_NONE, out_dtype=bf)

    def both(plan, freqs):
        fv, ft = capi.awa_qkv_forward(plan, xv, xt, w, b, norms, freqs, out_dtype=torch.float32)
        sv, st = capi.awa_forward(plan, norms, freqs, qv[:, :inner], qv[:, inner:2 * inner],
                                  qv[:, 2 * inner:], qt[:, :inner], qt[:, inner:2 * inner],
                                  qt[:, 2 * inner:], out_dtype=torch.float32)
        torch.cuda.synchronize()
        return [t.cpu().numpy() for t in (fv, ft, sv, st)]

    def same(a, b):
        for x, y in zip(a, b):
            np.testing.assert_array_equal(x, y)

    with capi.AwaPlan(cfg, shapes, tl) as ref_plan, capi.AwaPlan(cfg, shapes, tl) as plan:
        ref1, ref2 = both(ref_plan, f1), both(ref_plan, f2)
        assert not np.array_equal(ref1[0], ref2[0])
        plan.cache_rope(f1)
        same(both(plan, f1), ref1)           # served from the cache
        same(both(plan, f2), ref2)           # another tensor: computed per call
        f1.copy_(f2)                          # rewritten in place ...
        plan.cache_rope(f1)                   # ... and cached again
        same(both(plan, f1), ref2)
        plan.cache_rope(None)                 # cleared: computed per call again
        f1.mul_(2.0)
        same(both(plan, f1), ref1)
    # the cached table feeds an oracle-checked result as well
    rv, rt = oracle_awa(dict(video=oracle.linear(case["xv"], case["w"], case["b"], 0, threads=8),
                             text=oracle.linear(case["xt"], case["w"], case["b"], 0, threads=8),
                             norms=case["norms"], freqs=case["freqs"]),
                        heads, d, (4, 3, 3), 1, 1e-5, pairs, shapes, tl)
    assert_close(ref1[0], rv, "cached rope video")
    assert_close(ref1[1], rt, "cached rope text")


@pytest.mark.parametrize("shifted", [0, 1])
def test_fused_qkv_720p_against_the_oracle(shifted):
    """The headline kernel at the shape it is timed on: s2_awa_qkv_forward at
    6x45x80 + 64 text tokens, hidden 2560, 20x128 heads, against the oracle's
    attention forward (adaptive_window_attention.cpp:886-945) on every video
    and text row, at max-abs <= 2e-2 and cosine >= 0.9999.

    The projection feeding the oracle is X W^T + b in fp32.  For all 21,664
    rows it is torch's CPU matmul (a library GEMM; the oracle's textbook
    loop would take minutes here), tied to oracle.linear (the SharedLinear
    forward of shared_linear.cpp:83-96) on every row of two windows -- the
    first and a ragged edge window -- and every text row, where both must
    agree to 1e-5 of the output scale."""
    import torch
    shapes, tl = [(6, 45, 80)], [64]
    heads, d, pairs, hidden, target = 20, 128, 21, 2560, (4, 3, 3)
    inner = heads * d
    case = _inputs(71 + shifted, 21600, 64, hidden, heads, d, pairs)
    bf = torch.bfloat16
    cfg = capi.awa_config(heads, d, target, shifted, 1e-5, pairs)
    with capi.AwaPlan(cfg, shapes, tl) as plan:
        windows = plan.windows()[0]
        fv, ft = capi.awa_qkv_forward(plan, torch.from_numpy(case["xv"]).cuda().to(bf),
                                      torch.from_numpy(case["xt"]).cuda().to(bf),
                                      torch.from_numpy(case["w"]).cuda().to(bf),
                                      torch.from_numpy(case["b"]).cuda(),
                                      torch.from_numpy(case["norms"]).cuda(),
                                      torch.from_numpy(case["freqs"]).cuda(),
                                      out_dtype=torch.float32)
        torch.cuda.synchronize()
    fv, ft = fv.cpu().numpy(), ft.cpu().numpy()
    assert np.all(np.isfinite(fv)) and np.all(np.isfinite(ft))

    w = torch.from_numpy(case["w"])
    b = torch.from_numpy(case["b"])
    qv = torch.addmm(b, torch.from_numpy(case["xv"]), w.t()).numpy()
    qt = torch.addmm(b, torch.from_numpy(case["xt"]), w.t()).numpy()

    # pin the library GEMM to the oracle's on the rows of two windows: the
    # first, and the last one, a ragged edge window in both modes
    def window_rows(win):
        _, t0, t1, h0, h1, w0, w1, _, count = win
        assert count == (t1 - t0) * (h1 - h0) * (w1 - w0)
        return [(t * 45 + h) * 80 + x for t in range(t0, t1) for h in range(h0, h1)
                for x in range(w0, w1)]
    first, edge = windows[0], windows[-1]
    assert edge[6] == 80 and edge[8] < 810       # ends at the grid's edge, not full size
    rows = np.asarray(window_rows(first) + window_rows(edge), np.int32)
    ov = oracle.linear(case["xv"], case["w"], case["b"], 0, rows=rows, threads=16, fast=True)
    ot = oracle.linear(case["xt"], case["w"], case["b"], 0, threads=16, fast=True)
    scale = max(float(np.abs(ov).max()), float(np.abs(ot).max()))
    assert float(np.abs(qv[rows] - ov).max()) <= 1e-5 * scale
    assert float(np.abs(qt - ot).max()) <= 1e-5 * scale

    oc = dict(video=qv, text=qt, norms=case["norms"], freqs=case["freqs"])
    rv, rt = oracle_awa(oc, heads, d, target, shifted, 1e-5, pairs, shapes, tl, fast=True)
    assert_close(fv, rv, f"fused 720p video shifted={shifted}")
    assert_close(ft, rt, f"fused 720p text shifted={shifted}")
    # the two windows' rows on their own (a mistake confined to a window
    # would be diluted in the whole-array cosine)
    assert_close(fv[rows], rv[rows], f"fused 720p two windows shifted={shifted}")
