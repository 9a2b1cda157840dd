"""CPU pinning of the oracle's VAEChunkedMHA (src/seedvr2/vae_chunked_mha.cpp:223-235,
ncnn MultiHeadAttention over one blob) against torch's float64
multi_head_attention_forward."""
import numpy as np
import pytest
import torch

import oracle


def _weights(g, qdim, embed):
    w = lambda *s: (g.standard_normal(s) / np.sqrt(s[-1])).astype(np.float32)
    b = lambda n: (0.1 * g.standard_normal(n)).astype(np.float32)
    return w(embed, qdim), b(embed), w(embed, qdim), b(embed), w(embed, qdim), b(embed), \
        w(qdim, embed), b(qdim)


def _torch(x, heads, wq, bq, wk, bk, wv, bv, wo, bo):
    t = lambda a: torch.from_numpy(a).double()
    xt = t(x)[:, None, :]   # (seq, batch, qdim)
    out, _ = torch.nn.functional.multi_head_attention_forward(
        xt, xt, xt, wq.shape[1], heads, None, torch.cat([t(bq), t(bk), t(bv)]), None, None, False,
        0.0, t(wo), t(bo), training=False, need_weights=False, use_separate_proj_weight=True,
        q_proj_weight=t(wq), k_proj_weight=t(wk), v_proj_weight=t(wv))
    return out[:, 0, :].numpy()


@pytest.mark.parametrize("seq,qdim,heads", [(1, 8, 1), (37, 16, 1), (50, 32, 4), (128, 64, 2)])
def test_matches_torch_mha(seq, qdim, heads):
    g = np.random.default_rng(seq + qdim + heads)
    x = g.standard_normal((seq, qdim)).astype(np.float32)
    ws = _weights(g, qdim, qdim)
    got = oracle.mha(x, heads, *ws)
    ref = _torch(x, heads, *ws)
    assert np.max(np.abs(got - ref)) < 1e-5


def test_explicit_scale_and_row_subset():
    g = np.random.default_rng(3)
    x = g.standard_normal((40, 24)).astype(np.float32)
    ws = _weights(g, 24, 24)
    full = oracle.mha(x, 3, *ws, scale=0.5)
    rows = [39, 0, 17]
    assert np.array_equal(oracle.mha(x, 3, *ws, scale=0.5, rows=rows), full[rows])
    # scale 0.5 against a float64 numpy restatement
    q = x.astype(np.float64) @ ws[0].T.astype(np.float64) + ws[1]
    k = x.astype(np.float64) @ ws[2].T.astype(np.float64) + ws[3]
    v = x.astype(np.float64) @ ws[4].T.astype(np.float64) + ws[5]
    o = np.zeros_like(q)
    for h in range(3):
        sl = slice(8 * h, 8 * h + 8)
        s = 0.5 * q[:, sl] @ k[:, sl].T
        p = np.exp(s - s.max(1, keepdims=True))
        o[:, sl] = (p / p.sum(1, keepdims=True)) @ v[:, sl]
    ref = o @ ws[6].T.astype(np.float64) + ws[7]
    assert np.max(np.abs(full - ref)) < 1e-5


def test_constant_keys_average_the_values():
    # zero q/k weights and biases: uniform attention, the mean of v
    g = np.random.default_rng(4)
    x = g.standard_normal((20, 8)).astype(np.float32)
    wq, bq, wk, bk, wv, bv, wo, bo = _weights(g, 8, 8)
    z = np.zeros_like(wq)
    zb = np.zeros_like(bq)
    eye = np.eye(8, dtype=np.float32)
    got = oracle.mha(x, 2, z, zb, z, zb, eye, zb, eye, np.zeros(8, np.float32))
    assert np.max(np.abs(got - x.mean(0, keepdims=True))) < 1e-6
