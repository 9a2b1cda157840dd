"""Pins the CPU oracle (oracle/oracle.c) against checks that do not restate
its code: library routines (torch), closed forms and special cases.  The
reference ships no golden vectors or tests for this path, so these checks,
the window-plan checks in test_plan.py and the committed fixtures are what
anchors the oracle."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from common import bf16_round, make_awa_inputs, oracle_awa, rope_freqs
import plan_model


# ---- round_bf16 (adaptive_window_attention.cpp:499-508) --------------------

def test_round_bf16_matches_torch_rne_on_finite_values():
    g = np.random.default_rng(1)
    x = np.concatenate([g.standard_normal(2000).astype(np.float32) * 10.0 ** g.integers(-30, 30, 2000),
                        np.array([0.0, -0.0, 1.0, 65504.0, 3.4e38, -3.4e38, 1e-40], np.float32)])
    got = oracle.round_bf16(x)
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_round_bf16_ties_go_to_even():
    # 1 + 2^-8 lies halfway between two bf16 values; the even neighbour is 1.
    x = np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -(1.0 + 2.0 ** -8)], np.float32)
    got = oracle.round_bf16(x)
    np.testing.assert_array_equal(got, np.array([1.0, 1.0 + 2.0 ** -6, -1.0], np.float32))


def test_round_bf16_inf_and_nan_edge_cases():
    bits = np.array([0x7F800000, 0xFF800000, 0x7FC00000, 0x7F800001, 0x7F80FFFF], np.uint32)
    got = oracle.round_bf16(bits.view(np.float32)).view(np.uint32)
    # +-Inf stay, a quiet NaN stays NaN; a NaN whose payload is only in the
    # low 16 bits becomes +Inf, as the reference CPU rounding does.
    np.testing.assert_array_equal(got, np.array([0x7F800000, 0xFF800000, 0x7FC00000, 0x7F800000,
                                                 0x7F800000], np.uint32))


# ---- rms_norm (:510-519) -----------------------------------------------------

@pytest.mark.parametrize("d", [16, 64, 128])
def test_rms_norm_matches_torch(d):
    g = np.random.default_rng(d)
    x = g.standard_normal(d).astype(np.float32) * 3
    w = (1 + 0.1 * g.standard_normal(d)).astype(np.float32)
    got = oracle.rms_norm(x, w, 1e-5)
    want = F.rms_norm(torch.from_numpy(x).double(), (d,), torch.from_numpy(w).double(), eps=1e-5)
    np.testing.assert_allclose(got, want.numpy(), rtol=2e-6, atol=1e-6)


def test_rms_norm_unit_weight_gives_unit_rms():
    x = np.random.default_rng(3).standard_normal(128).astype(np.float32) * 7
    y = oracle.rms_norm(x, np.ones(128, np.float32), 0.0)
    assert abs(float(np.sqrt(np.mean(y.astype(np.float64) ** 2))) - 1.0) < 1e-6


# ---- apply_mm_rope (:521-543) -------------------------------------------------

def _rope_complex(x, freqs, pairs, pos):
    """Rotation of interleaved pairs written as complex multiplication."""
    y = x.astype(np.float64).copy()
    for a in range(3):
        seg = y[a * 2 * pairs:(a + 1) * 2 * pairs]
        z = seg[0::2] + 1j * seg[1::2]
        z = z * np.exp(1j * pos[a] * freqs.astype(np.float64))
        seg[0::2], seg[1::2] = z.real, z.imag
    return y


def test_rope_matches_complex_rotation():
    g = np.random.default_rng(5)
    d, pairs = 128, 21
    x = g.standard_normal(d).astype(np.float32)
    freqs = rope_freqs(pairs)
    pos = [70, 11, 26]
    got = oracle.apply_mm_rope(x, freqs, pairs, pos)
    np.testing.assert_allclose(got, _rope_complex(x, freqs, pairs, pos), atol=2e-5)
    np.testing.assert_array_equal(got[6 * pairs:], x[6 * pairs:])   # dims >= 6P untouched


def test_rope_identity_cases():
    x = np.random.default_rng(6).standard_normal(64).astype(np.float32)
    np.testing.assert_array_equal(oracle.apply_mm_rope(x, np.zeros(10, np.float32), 10, [5, 6, 7]), x)
    np.testing.assert_array_equal(oracle.apply_mm_rope(x, rope_freqs(10), 10, [0, 0, 0]), x)
    # rotary width beyond head_dim: untouched (:526-527)
    np.testing.assert_array_equal(oracle.apply_mm_rope(x, rope_freqs(11), 11, [1, 2, 3]), x)


def test_rope_preserves_pair_norms():
    x = np.random.default_rng(7).standard_normal(128).astype(np.float32)
    y = oracle.apply_mm_rope(x, rope_freqs(21), 21, [9, 3, 4])
    n0 = x[:126:2] ** 2 + x[1:126:2] ** 2
    n1 = y[:126:2] ** 2 + y[1:126:2] ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-5)


# ---- SDPA (ncnn SDPA, :847-861, 943) ---------------------------------------

def test_sdpa_matches_torch():
    g = np.random.default_rng(8)
    q, k, v = (g.standard_normal((3, 37, 32)).astype(np.float32) for _ in range(3))
    got = oracle.sdpa(q, k, v)
    want = F.scaled_dot_product_attention(*(torch.from_numpy(a).double() for a in (q, k, v)))
    np.testing.assert_allclose(got, want.numpy(), atol=2e-6)


def test_sdpa_constant_keys_average_values():
    g = np.random.default_rng(9)
    q = g.standard_normal((2, 11, 16)).astype(np.float32)
    k = np.broadcast_to(g.standard_normal((2, 1, 16)), (2, 11, 16)).astype(np.float32)
    v = g.standard_normal((2, 11, 16)).astype(np.float32)
    got = oracle.sdpa(q, k, v)
    np.testing.assert_allclose(got, np.broadcast_to(v.mean(1, keepdims=True), v.shape), atol=1e-6)


def test_sdpa_one_hot_logits_select_a_value_row():
    d = 16
    k = np.zeros((1, 5, d), np.float32)
    k[0, 3, 0] = 100.0
    q = np.zeros((1, 5, d), np.float32)
    q[0, :, 0] = 100.0        # logit 100*100/4 on key 3, 0 elsewhere
    v = np.random.default_rng(10).standard_normal((1, 5, d)).astype(np.float32)
    got = oracle.sdpa(q, k, v)
    np.testing.assert_allclose(got[0], np.broadcast_to(v[0, 3], (5, d)), atol=1e-6)


# ---- SharedLinear / Gemm (shared_linear.cpp:83-96) ----------------------------

@pytest.mark.parametrize("act", [0, 1])
def test_linear_matches_torch(act):
    g = np.random.default_rng(11 + act)
    x = g.standard_normal((19, 40)).astype(np.float32)
    w = (0.2 * g.standard_normal((24, 40))).astype(np.float32)
    b = g.standard_normal(24).astype(np.float32)
    got = oracle.linear(x, w, b, act)
    y = torch.from_numpy(x).double() @ torch.from_numpy(w).double().T + torch.from_numpy(b).double()
    if act:
        y = F.gelu(y)
    np.testing.assert_allclose(got, y.numpy(), atol=2e-5)


def test_linear_row_subset_and_no_bias():
    g = np.random.default_rng(13)
    x = g.standard_normal((30, 16)).astype(np.float32)
    w = g.standard_normal((8, 16)).astype(np.float32)
    full = oracle.linear(x, w)
    sub = oracle.linear(x, w, rows=[29, 0, 7])
    np.testing.assert_array_equal(sub, full[[29, 0, 7]])


# ---- the whole layer (:764-978) ----------------------------------------------

def _torch_layer(case, heads, d, target, shifted, eps, pairs, shapes, text_lengths):
    """The layer semantics in float64 torch, built on plan_model's windows,
    torch rms_norm, complex-form rope and torch SDPA."""
    inner = heads * d
    v = torch.from_numpy(case["video"]).double()
    t = torch.from_numpy(case["text"]).double()
    n = torch.from_numpy(case["norms"]).double()
    freqs = case["freqs"].astype(np.float64)
    wins, counts, idx, inv, pos = plan_model.plan(shapes, target, shifted)
    lv, lt = v.shape[0], t.shape[0]
    out_v = torch.zeros(lv, inner, dtype=torch.float64)
    out_t = torch.zeros(lt, inner, dtype=torch.float64)
    toff = np.concatenate([[0], np.cumsum(text_lengths)])

    def rope(x, p):   # x [S, heads, d], p [S, 3]
        x = x.clone()
        for a in range(3):
            ang = torch.from_numpy(p[:, a:a + 1].astype(np.float64) * freqs[None, :])  # [S, P]
            sl = x[..., a * 2 * pairs:(a + 1) * 2 * pairs]
            z = torch.complex(sl[..., 0::2], sl[..., 1::2]) * torch.polar(torch.ones_like(ang), ang)[:, None, :]
            sl[..., 0::2], sl[..., 1::2] = z.real, z.imag
        return x

    for (b, t0, t1, h0, h1, w0, w1, part, cnt) in wins:
        L = text_lengths[b]
        src = idx[part:part + cnt]
        vv = v[src].view(cnt, 3, heads, d)
        tt = t[toff[b]:toff[b] + L].view(L, 3, heads, d)
        q = torch.cat([F.rms_norm(vv[:, 0], (d,), n[0], eps), F.rms_norm(tt[:, 0], (d,), n[2], eps)])
        k = torch.cat([F.rms_norm(vv[:, 1], (d,), n[1], eps), F.rms_norm(tt[:, 1], (d,), n[3], eps)])
        val = torch.cat([vv[:, 2], tt[:, 2]])
        p = np.concatenate([pos[part:part + cnt] + np.array([L, 0, 0]),
                            np.repeat(np.arange(L)[:, None], 3, 1)])
        q, k = rope(q, p), rope(k, p)
        ctx = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), val.transpose(0, 1))
        ctx = ctx.transpose(0, 1).reshape(-1, inner)
        out_v[src] = ctx[:cnt]
        out_t[toff[b]:toff[b] + L] += ctx[cnt:] / counts[b]
    return out_v.numpy(), out_t.numpy()


@pytest.mark.parametrize("shifted", [0, 1])
def test_awa_forward_matches_independent_torch_model(shifted):
    shapes = [(2, 4, 6), (3, 5, 4)]
    text_lengths = [3, 5]
    heads, d, pairs, target = 2, 16, 2, (2, 2, 3)
    case = make_awa_inputs(21 + shifted, shapes, text_lengths, heads, d, pairs, peaky=True)
    got_v, got_t = oracle_awa(case, heads, d, target, shifted, 1e-5, pairs, shapes, text_lengths)
    want_v, want_t = _torch_layer(case, heads, d, target, shifted, 1e-5, pairs, shapes, text_lengths)
    np.testing.assert_allclose(got_v, want_v, atol=2e-5)
    np.testing.assert_allclose(got_t, want_t, atol=2e-5)


def test_awa_single_window_text_pool_is_that_window():
    # target (1,1,1) makes one window per sample: the pooled text output is
    # that window's text rows (scale 1/1).
    shapes, text_lengths = [(2, 3, 4)], [4]
    heads, d, pairs = 2, 16, 2
    case = make_awa_inputs(31, shapes, text_lengths, heads, d, pairs)
    ov, ot = oracle_awa(case, heads, d, (1, 1, 1), 0, 1e-5, pairs, shapes, text_lengths)
    wv, wt = _torch_layer(case, heads, d, (1, 1, 1), 0, 1e-5, pairs, shapes, text_lengths)
    np.testing.assert_allclose(ot, wt, atol=2e-5)


def test_awa_official_bf16_rounds_outputs():
    shapes, text_lengths = [(1, 4, 4)], [2]
    heads, d, pairs = 1, 16, 2
    case = make_awa_inputs(41, shapes, text_lengths, heads, d, pairs)
    ov, _ = oracle_awa(case, heads, d, (1, 2, 2), 0, 1e-5, pairs, shapes, text_lengths,
                       official_bf16=True)
    np.testing.assert_array_equal(ov, bf16_round(ov))


def test_awa_error_codes():
    shapes, text_lengths = [(1, 4, 4)], [2]
    case = make_awa_inputs(51, shapes, text_lengths, 1, 16, 2)
    with pytest.raises(ValueError, match="-1"):
        oracle_awa(case, 1, 16, (1, 2, 2), 0, 1e-5, 3, shapes, text_lengths)   # 6P > d
    with pytest.raises(ValueError, match="-1"):
        oracle_awa(case, 1, 16, (1, 2, 2), 0, 1e-5, 2, shapes, [0])            # empty text
