"""The v3 DiT graph shapes on the GPU (seedvr2_pipeline.cpp:434-438: "v3
manifests split QKV into separate q/k/v projections, so the largest DiT
activation is the SwiGLU gate/up projection [tokens, 3456]"):

- SharedLinear with N = 3456 (a half-filled last 256-column tile) and
  K = 3456 (the MLP down projection, 54 k-steps), against the oracle;
- the fused SwiGLU epilogue (S2_ACT_SWIGLU, silu(x Wg^T + bg) * (x Wu^T + bu)
  over an interleaved gate/up weight built by s2_swiglu_pack_weight) against
  the oracle's two projections composed in float64, fp32 and bf16 outputs,
  including a k split over several workgroups;
- separate q, k, v projections (to 2560 each) feeding the attention's
  8-input split form (adaptive_window_attention.cpp:783-797), against the
  fused-QKV path on the same weights (bit-identical: the same GEMM tiles, the
  same attention inputs) and the oracle.
Bar: max-abs <= 2e-2 and cosine >= 0.9999 against fp32 references."""
import numpy as np
import pytest

import oracle
from common import assert_close, bf16_round, oracle_awa
from seedvr2_ncnn_amd import capi

pytestmark = pytest.mark.gpu


def _t(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t.to(dtype) if dtype is not None else t


def _silu(x):
    return x / (1.0 + np.exp(-x))


@pytest.mark.parametrize("mv,mt,k,n", [(300, 64, 2560, 3456), (257, 7, 3456, 2560),
                                       (1024, 64, 3456, 3456)])
def test_3456_shapes(mv, mt, k, n):
    import torch
    g = np.random.default_rng(mv + k + n)
    xv = bf16_round(g.standard_normal((mv, k)).astype(np.float32))
    xt = bf16_round(g.standard_normal((mt, k)).astype(np.float32))
    w = bf16_round((0.02 * g.standard_normal((n, k))).astype(np.float32))
    b = (0.02 * g.standard_normal(n)).astype(np.float32)
    yv, yt = capi.shared_linear(_t(xv, torch.bfloat16), _t(xt, torch.bfloat16),
                                _t(w, torch.bfloat16), _t(b), capi.ACT_NONE, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert_close(yv.cpu().numpy(), oracle.linear(xv, w, b, threads=8), f"video {k}->{n}")
    assert_close(yt.cpu().numpy(), oracle.linear(xt, w, b, threads=8), f"text {k}->{n}")


@pytest.mark.parametrize("mv,mt,k,n", [(300, 64, 2560, 3456), (77, 5, 512, 128),
                                       (2048, 64, 2560, 3456), (64, 0, 1024, 256)])
@pytest.mark.parametrize("out_bf16", [False, True])
def test_swiglu_epilogue(mv, mt, k, n, out_bf16):
    import torch
    g = np.random.default_rng(mv * 3 + k + n + out_bf16)
    xv = bf16_round(g.standard_normal((mv, k)).astype(np.float32))
    xt = bf16_round(g.standard_normal((max(mt, 1), k)).astype(np.float32))[:mt]
    wg = bf16_round((0.03 * g.standard_normal((n, k))).astype(np.float32))
    wu = bf16_round((0.03 * g.standard_normal((n, k))).astype(np.float32))
    bg = (0.05 * g.standard_normal(n)).astype(np.float32)
    bu = (0.05 * g.standard_normal(n)).astype(np.float32)
    packed, pb = capi.swiglu_pack_weight(_t(wg, torch.bfloat16), _t(wu, torch.bfloat16), _t(bg), _t(bu))
    ydt = torch.bfloat16 if out_bf16 else torch.float32
    yv, yt = capi.shared_linear(_t(xv, torch.bfloat16), _t(xt, torch.bfloat16) if mt else None,
                                packed, pb, capi.ACT_SWIGLU, out_dtype=ydt)
    torch.cuda.synchronize()
    assert yv.shape == (mv, n)
    for x, y in ((xv, yv), (xt, yt)):
        if x.shape[0] == 0:
            continue
        gate = oracle.linear(x, wg, bg, threads=8).astype(np.float64)
        up = oracle.linear(x, wu, bu, threads=8).astype(np.float64)
        ref = _silu(gate) * up
        got = y.float().cpu().numpy()
        if out_bf16:
            # one bf16 rounding of a result within the fp32 bar (|y| reaches
            # ~8 here, where a bf16 step is 0.0625)
            assert np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 2e-3), f"swiglu {k}->{n}"
            assert_close(got, ref, f"swiglu {k}->{n}", max_abs=np.inf)
        else:
            assert_close(got, ref, f"swiglu {k}->{n}")


def test_swiglu_pack_layout():
    import torch
    n, k = 256, 64
    gate = torch.arange(n * k, dtype=torch.float32, device="cuda").reshape(n, k).to(torch.bfloat16)
    up = -gate
    gb = torch.arange(n, dtype=torch.float32, device="cuda")
    packed, pb = capi.swiglu_pack_weight(gate, up, gb, -gb)
    torch.cuda.synchronize()
    p = packed.float().cpu().numpy()
    g, u = gate.float().cpu().numpy(), up.float().cpu().numpy()
    for j in range(n // 128):
        np.testing.assert_array_equal(p[256 * j:256 * j + 128], g[128 * j:128 * j + 128])
        np.testing.assert_array_equal(p[256 * j + 128:256 * j + 256], u[128 * j:128 * j + 128])
    np.testing.assert_array_equal(pb.cpu().numpy()[128:256], -np.arange(128, dtype=np.float32))


def test_swiglu_rejects_unsupported_shapes():
    import torch
    x = torch.zeros(8, 512, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(2 * 192, 512, dtype=torch.bfloat16, device="cuda")   # n = 192
    with pytest.raises(capi.S2Error) as e:
        capi.shared_linear(x, None, w, None, capi.ACT_SWIGLU)
    assert e.value.code == capi.S2_ERR_INVALID
    with pytest.raises(capi.S2Error):
        capi.shared_linear(x.float(), None, torch.zeros(256, 512, dtype=torch.bfloat16,
                                                        device="cuda"), None, capi.ACT_SWIGLU)


@pytest.mark.parametrize("shifted", [0, 1])
def test_split_qkv_projections_feed_the_split_attention_form(shifted):
    """q, k, v as three projections to 2560 (the v3 graph) at a 1x32x48 grid
    with 20 heads x 128.  The input width is 512 so that neither the three
    2560-wide GEMMs nor the 7680-wide fused one split k (fewer than 16
    k-steps), which keeps every output element's accumulation order the same."""
    import torch
    heads, d, pairs = 20, 128, 21
    inner = heads * d
    hidden = 512
    shapes, tl = [(1, 32, 48)], [64]
    lv = 32 * 48
    g = np.random.default_rng(40 + shifted)
    xv = bf16_round(g.standard_normal((lv, hidden)).astype(np.float32))
    xt = bf16_round(g.standard_normal((64, hidden)).astype(np.float32))
    ws = [bf16_round((0.04 * g.standard_normal((inner, hidden))).astype(np.float32)) for _ in range(3)]
    bs = [(0.02 * g.standard_normal(inner)).astype(np.float32) for _ in range(3)]
    norms = (1.0 + 0.02 * g.standard_normal((4, d))).astype(np.float32)
    freqs = (10000.0 ** (-np.arange(pairs) / pairs)).astype(np.float32)
    bf = torch.bfloat16
    tv, tt = _t(xv, bf), _t(xt, bf)
    qkv = [capi.shared_linear(tv, tt, _t(w, bf), _t(b), capi.ACT_NONE) for w, b in zip(ws, bs)]
    cfg = capi.awa_config(heads, d, (4, 3, 3), shifted, 1e-5, pairs)
    with capi.AwaPlan(cfg, shapes, tl) as plan:
        sv, st = capi.awa_forward(plan, _t(norms), _t(freqs), qkv[0][0], qkv[1][0], qkv[2][0],
                                  qkv[0][1], qkv[1][1], qkv[2][1], out_dtype=torch.float32)
        # the same weights as one fused QKV projection
        w_all = _t(np.concatenate(ws), bf)
        b_all = _t(np.concatenate(bs))
        fv, ft = capi.awa_qkv_forward(plan, tv, tt, w_all, b_all, _t(norms), _t(freqs),
                                      out_dtype=torch.float32)
        torch.cuda.synchronize()
    np.testing.assert_array_equal(sv.cpu().numpy(), fv.cpu().numpy())
    np.testing.assert_array_equal(st.cpu().numpy(), ft.cpu().numpy())
    qv = np.concatenate([oracle.linear(xv, w, b, threads=8) for w, b in zip(ws, bs)], axis=1)
    qt = np.concatenate([oracle.linear(xt, w, b, threads=8) for w, b in zip(ws, bs)], axis=1)
    rv, rt = oracle_awa(dict(video=qv, text=qt, norms=norms, freqs=freqs), heads, d, (4, 3, 3),
                        shifted, 1e-5, pairs, shapes, tl)
    assert_close(sv.cpu().numpy(), rv, "split-qkv video")
    assert_close(st.cpu().numpy(), rt, "split-qkv text")


def test_shared_linear_layer_swiglu_param():
    """SharedLinear with this build's param 3 = 2: the gate projection's
    [N][K] weight, then the up projection's, then the two biases, from the
    .bin; host fp32 blobs (rounded to bf16 on the device) and device bf16
    blobs."""
    import torch
    from common import Layer
    g = np.random.default_rng(9)
    k, n, mv, mt = 512, 256, 200, 17
    wg = (0.03 * g.standard_normal((n, k))).astype(np.float32)
    wu = (0.03 * g.standard_normal((n, k))).astype(np.float32)
    bg = (0.05 * g.standard_normal(n)).astype(np.float32)
    bu = (0.05 * g.standard_normal(n)).astype(np.float32)
    xv = g.standard_normal((mv, k)).astype(np.float32)
    xt = g.standard_normal((mt, k)).astype(np.float32)
    layer = Layer("SharedLinear", f"0={n} 1={k} 2=1 3=2", [wg, wu, bg, bu])
    assert layer.create_code == 0 and layer.create_pipeline() == 0

    def ref(x):
        xr, gr, ur = bf16_round(x), bf16_round(wg), bf16_round(wu)
        return _silu(oracle.linear(xr, gr, bg, threads=8).astype(np.float64)) * \
            oracle.linear(xr, ur, bu, threads=8).astype(np.float64)
    code, (yv, yt) = layer.forward([xv, xt], [((mv, n), np.float32), ((mt, n), np.float32)])
    assert code == 0
    assert_close(yv, ref(xv), "host video")
    assert_close(yt, ref(xt), "host text")
    dv = torch.from_numpy(xv).cuda().to(torch.bfloat16)
    dt = torch.from_numpy(xt).cuda().to(torch.bfloat16)
    code, (yv, yt) = layer.forward([dv, dt], [((mv, n), torch.bfloat16), ((mt, n), torch.bfloat16)],
                                   device_out=True)
    assert code == 0
    for got, x in ((yv, xv), (yt, xt)):
        r = ref(x)
        got = got.float().cpu().numpy()
        assert np.all(np.abs(got - r) <= 2.0 ** -8 * np.abs(r) + 2e-3)
        assert_close(got, r, "device swiglu", max_abs=np.inf)
    # N not a multiple of 128 is refused at load_param
    assert Layer("SharedLinear", f"0=192 1={k} 2=1 3=2", None).create_code == -1
