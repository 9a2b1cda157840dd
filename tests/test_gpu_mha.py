"""VAEChunkedMHA on the GPU (src/seedvr2/vae_chunked_mha.cpp:223-281: ncnn
MultiHeadAttention over one blob) against the CPU oracle.

The device runs the projections and both attention products in bf16 with
fp32 accumulation (scores stay fp32 until the softmax, probabilities are
rounded to bf16).  The bar is the path's: max-abs <= 2e-2 and cosine >=
0.9999 against the fp32-input oracle.  Sequences of VAE size are checked on
a spread of query rows (the oracle computes only those rows)."""
import numpy as np
import pytest

import oracle
from common import assert_close, bf16_round
from seedvr2_ncnn_amd import capi

pytestmark = pytest.mark.gpu


def _weights(g, qdim, embed):
    w = lambda *s: (g.standard_normal(s) / np.sqrt(s[-1])).astype(np.float32)
    b = lambda n: (0.1 * g.standard_normal(n)).astype(np.float32)
    return [w(embed, qdim), b(embed), w(embed, qdim), b(embed), w(embed, qdim), b(embed),
            w(qdim, embed), b(qdim)]


def _device(heads, ws, scale=None):
    import torch
    return capi.Mha(heads, *[torch.from_numpy(a).cuda() for a in ws], scale=scale)


def _run(mha, x, dtype=None, out_dtype=None):
    import torch
    t = torch.from_numpy(x).cuda()
    if dtype is not None:
        t = t.to(dtype)
    y = mha.forward(t, out_dtype=out_dtype)
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


@pytest.mark.parametrize("seq,qdim,heads", [(1, 64, 1), (37, 64, 2), (200, 128, 4), (1000, 512, 1),
                                            (333, 256, 2)])
def test_mha_matches_oracle(seq, qdim, heads):
    g = np.random.default_rng(seq + qdim)
    x = g.standard_normal((seq, qdim)).astype(np.float32)
    ws = _weights(g, qdim, qdim)
    got = _run(_device(heads, ws), x)
    ref = oracle.mha(x, heads, *ws, threads=16)
    assert_close(got, ref)


def test_mha_explicit_scale_and_16bit_blobs():
    import torch
    g = np.random.default_rng(2)
    x = g.standard_normal((300, 128)).astype(np.float32)
    ws = _weights(g, 128, 128)
    mha = _device(2, ws, scale=0.3)
    for dt, odt in ((torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32)):
        xs = torch.from_numpy(x).to(dt).float().numpy()    # the stored values
        got = _run(mha, xs, dtype=dt, out_dtype=odt)
        assert_close(got, oracle.mha(xs, 2, *ws, scale=0.3, threads=16))


def test_mha_16bit_outputs_round_the_fp32_output():
    """bf16 and fp16 outputs are the round-to-nearest-even of the fp32
    output of the same call (one rounding of the fp32 result)."""
    import torch
    g = np.random.default_rng(12)
    x = bf16_round(g.standard_normal((333, 256)).astype(np.float32))
    ws = _weights(g, 256, 256)
    mha = _device(2, ws)
    outs = {odt: _run(mha, x, dtype=torch.bfloat16, out_dtype=odt)
            for odt in (torch.float32, torch.bfloat16, torch.float16)}
    ref = outs[torch.float32]
    np.testing.assert_array_equal(outs[torch.bfloat16], bf16_round(ref))
    np.testing.assert_array_equal(outs[torch.float16], ref.astype(np.float16).astype(np.float32))
    assert_close(ref, oracle.mha(x, 2, *ws, threads=16))


def test_mha_vae_frame_rows():
    """One 720p latent frame (90 x 160 = 14,400 tokens, 512 channels, one
    head): 64 query rows spread over the sequence against the oracle."""
    g = np.random.default_rng(9)
    seq, qdim = 14400, 512
    x = g.standard_normal((seq, qdim)).astype(np.float32)
    ws = _weights(g, qdim, qdim)
    got = _run(_device(1, ws), x)
    rows = np.linspace(0, seq - 1, 64).astype(np.int32)
    ref = oracle.mha(x, 1, *ws, rows=rows, threads=16, fast=True)
    assert_close(got[rows], ref)


# ---- the ncnn-surface layer (vae_chunked_mha.h:12-50) --------------------------

FP16_TAG = np.frombuffer(np.uint32(0x01306B47).tobytes(), np.float32)


def _fp16_blob(a):
    """ncnn's tagged fp16 weight: the tag, then the halves padded to 4 bytes."""
    h = np.asarray(a, np.float16).ravel()
    if h.size % 2:
        h = np.concatenate([h, np.zeros(1, np.float16)])
    return np.concatenate([FP16_TAG, h.view(np.float32)])


def _layer(embed, heads, qdim, ws, scale=None, fp16_out_weight=False):
    from common import Layer
    wq, bq, wk, bk, wv, bv, wo, bo = ws
    params = f"0={embed} 1={heads} 2={embed * qdim} 3={qdim} 4={qdim} 20=64"
    if scale is not None:
        params += f" 6={scale}"
    tag0 = np.zeros(1, np.float32)   # raw fp32 tag of a type-0 blob
    out_w = _fp16_blob(wo) if fp16_out_weight else np.concatenate([tag0, wo.ravel()])
    blobs = [tag0, wq, bq, tag0, wk, bk, tag0, wv, bv, out_w, bo]
    layer = Layer("SeedVR2ChunkedMHA", params, weights=blobs)
    assert layer.create_code == 0
    assert layer.create_pipeline() == 0
    return layer


@pytest.mark.parametrize("device", [False, True])
def test_layer_forward(device):
    import torch
    g = np.random.default_rng(12)
    x = g.standard_normal((500, 128)).astype(np.float32)
    ws = _weights(g, 128, 128)
    layer = _layer(128, 2, 128, ws)
    dt = torch.bfloat16 if device else None
    xs = torch.from_numpy(x).to(torch.bfloat16).float().numpy() if device else x
    code, got = layer.forward_rows(xs, 128, device=device, dtype=dt)
    assert code == 0
    assert_close(got, oracle.mha(xs, 2, *ws, threads=16))


def test_layer_fp16_weights_and_scale():
    g = np.random.default_rng(13)
    x = g.standard_normal((64, 64)).astype(np.float32)
    ws = _weights(g, 64, 64)
    ws[6] = ws[6].astype(np.float16).astype(np.float32)   # what the fp16 blob stores
    layer = _layer(64, 1, 64, ws, scale=0.2, fp16_out_weight=True)
    code, got = layer.forward_rows(x, 64)
    assert code == 0
    assert_close(got, oracle.mha(x, 1, *ws, scale=0.2, threads=16))


def test_layer_rejects_wrong_width():
    g = np.random.default_rng(14)
    ws = _weights(g, 64, 64)
    layer = _layer(64, 1, 64, ws)
    assert layer.forward_rows(np.zeros((8, 32), np.float32), 32)[0] == -1
