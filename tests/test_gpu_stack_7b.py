"""The SeedVR2-7B-shaped block stack on the GPU at the 720p grid (6x45x80
video + 64 text tokens, hidden 3072, 24 heads x 128, MLP 3072 -> 12288 GELU
-> 3072, even blocks regular and odd blocks shifted windows, the text tokens
projected 5120 -> 3072 once; src/seedvr2/seedvr2_dit.cpp:722-833 runs the
exported graph of this shape).

- The whole 32-block stack with each block's norm and AdaSingle modulation on
  an fp32 residual stream: finite, bit-identical when run again, and each
  block's output RMS within a factor of two of its input's (the residual
  stream carries the signal; a broken stage shows up as an explosion or a
  collapse).
- Two blocks at the same shape, stage by stage against the oracle (each stage
  on the values the device stage read): the row-wise stages on 512 video rows
  and all text rows, the attention on a subset of its windows (video rows of
  those windows).  GEMM outputs: within one bf16 rounding of the fp32
  reference (they are bf16 and reach magnitudes where one rounding exceeds
  2e-2) and cosine >= 0.9999; attention: max-abs <= 2e-2 and cosine >=
  0.9999; modulated norms: one bf16 rounding; residual sums: bit-exact."""
import numpy as np
import pytest

import oracle
from common import assert_close, oracle_awa
from seedvr2_ncnn_amd import capi

pytestmark = pytest.mark.gpu

SHAPE = (6, 45, 80)
LV = 6 * 45 * 80
LT = 64
D, H, HD, F, PAIRS = 3072, 24, 128, 12288, 21
TARGET = (4, 3, 3)


def _close_bf16(got, ref, what):
    """A bf16 stage output against the fp32 reference applied to the same
    bf16 inputs: one rounding of the result (|y| reaches ~8 at K = 12288,
    where a bf16 step is 0.03) plus accumulation-order noise, and the
    path's cosine bar."""
    tol = 2.0 ** -8 * np.abs(ref) + 1e-4 * float(np.max(np.abs(ref)))
    assert np.all(np.abs(got - ref) <= tol), f"{what}: beyond one bf16 rounding"
    assert_close(got, ref, what, max_abs=np.inf)


def _weights(torch, gen, blocks):
    dev = "cuda"
    bf = torch.bfloat16

    def randn(*shape, std=1.0):
        return (torch.randn(*shape, generator=gen, device=dev) * std).to(bf)

    def bias(n):
        return torch.randn(n, generator=gen, device=dev) * 0.02
    out = []
    for _ in range(blocks):
        out.append(dict(qkv=randn(3 * D, D, std=0.02), bqkv=bias(3 * D), o=randn(D, D, std=0.02),
                        bo=bias(D), up=randn(F, D, std=0.02), bup=bias(F),
                        dn=randn(D, F, std=0.02), bdn=bias(D),
                        norms=(1.0 + 0.02 * torch.randn(4, HD, generator=gen, device=dev)).contiguous(),
                        mods=[torch.randn(1, D, generator=gen, device=dev) * 0.1 +
                              (1.0 if k in (1, 4) else 0.0) for k in range(6)]))
    return out


def _block(torch, blk, plan, freqs, r_v, r_t, keep=None):
    """One block through the C-ABI on the residual (r_v, r_t), in place."""
    bf = torch.bfloat16
    md = blk["mods"]
    vr, tr = [LV], [LT]
    h_v, h_t = capi.ada_in(r_v, r_t, vr, tr, md[0], md[1], out_dtype=bf)
    q_v, q_t = capi.shared_linear(h_v, h_t, blk["qkv"], blk["bqkv"], capi.ACT_NONE)
    a_v, a_t = capi.awa_forward(plan, blk["norms"], freqs, q_v[:, :D], q_v[:, D:2 * D],
                                q_v[:, 2 * D:], q_t[:, :D], q_t[:, D:2 * D], q_t[:, 2 * D:])
    o_v, o_t = capi.shared_linear(a_v, a_t, blk["o"], blk["bo"], capi.ACT_NONE)
    if keep is not None:
        keep.update(r_v=r_v.clone(), r_t=r_t.clone())
    _, _, m_v, m_t = capi.ada_out_in(r_v, r_t, o_v, o_t, vr, tr, md[2], md[3], md[4])
    if keep is not None:
        keep.update(r1_v=r_v.clone(), r1_t=r_t.clone())
    u_v, u_t = capi.shared_linear(m_v, m_t, blk["up"], blk["bup"], capi.ACT_GELU)
    y_v, y_t = capi.shared_linear(u_v, u_t, blk["dn"], blk["bdn"], capi.ACT_NONE)
    capi.ada_out(r_v, r_t, y_v, y_t, vr, tr, md[5])
    if keep is not None:
        keep.update(h_v=h_v, h_t=h_t, q_v=q_v, q_t=q_t, a_v=a_v, a_t=a_t, o_v=o_v, o_t=o_t,
                    m_v=m_v, m_t=m_t, u_v=u_v, u_t=u_t, y_v=y_v, y_t=y_t)


def test_32_block_stack_properties():
    import torch
    gen = torch.Generator(device="cuda").manual_seed(77)
    blocks = _weights(torch, gen, 32)
    w_text = (torch.randn(D, 5120, generator=gen, device="cuda") * 0.02).to(torch.bfloat16)
    b_text = torch.randn(D, generator=gen, device="cuda") * 0.02
    x_v0 = torch.randn(LV, D, generator=gen, device="cuda")
    text_in = torch.randn(LT, 5120, generator=gen, device="cuda").to(torch.bfloat16)
    freqs = (10000.0 ** (-torch.arange(PAIRS, device="cuda", dtype=torch.float64) / PAIRS)).float()
    plans = {s: capi.AwaPlan(capi.awa_config(H, HD, TARGET, s, 1e-5, PAIRS), [SHAPE], [LT])
             for s in (0, 1)}
    try:
        def run():
            r_v = x_v0.clone()
            r_t, _ = capi.shared_linear(text_in, None, w_text, b_text, capi.ACT_NONE,
                                        out_dtype=torch.float32)
            rms = [float(r_v.square().mean().sqrt())]
            for i, blk in enumerate(blocks):
                _block(torch, blk, plans[i % 2], freqs, r_v, r_t)
                rms.append(float(r_v.square().mean().sqrt()))
            torch.cuda.synchronize()
            return r_v, r_t, rms
        v1, t1, rms = run()
        assert bool(torch.isfinite(v1).all()) and bool(torch.isfinite(t1).all())
        for i in range(32):
            assert 0.5 < rms[i + 1] / rms[i] < 2.0, f"block {i}: rms {rms[i]:.4f} -> {rms[i + 1]:.4f}"
        v2, t2, _ = run()
        assert torch.equal(v1, v2) and torch.equal(t1, t2)
    finally:
        for p in plans.values():
            p.close()


def test_two_blocks_stage_by_stage_on_row_and_window_subsets():
    import torch
    gen = torch.Generator(device="cuda").manual_seed(78)
    blocks = _weights(torch, gen, 2)
    freqs = (10000.0 ** (-torch.arange(PAIRS, device="cuda", dtype=torch.float64) / PAIRS)).float()
    r_v = torch.randn(LV, D, generator=gen, device="cuda")
    r_t = torch.randn(LT, D, generator=gen, device="cuda")
    rows = np.sort(np.random.default_rng(5).choice(LV, 512, replace=False)).astype(np.int32)
    f = lambda t: t.float().cpu().numpy()
    for b, blk in enumerate(blocks):
        cfg = capi.awa_config(H, HD, TARGET, b % 2, 1e-5, PAIRS)
        keep = {}
        with capi.AwaPlan(cfg, [SHAPE], [LT]) as plan:
            _block(torch, blk, plan, freqs, r_v, r_t, keep)
            torch.cuda.synchronize()
            wins, _ = plan.windows()
        md = [f(m) for m in blk["mods"]]
        w = {k: f(blk[k]) for k in ("qkv", "o", "up", "dn")}
        bb = {k: f(blk[k]) for k in ("bqkv", "bo", "bup", "bdn")}
        x_v, x_t = f(keep["r_v"]), f(keep["r_t"])
        # norm + modulation (row-wise): one bf16 rounding
        for x, h, n in ((x_v[rows], f(keep["h_v"])[rows], len(rows)), (x_t, f(keep["h_t"]), LT)):
            ref = oracle.ada_in(x, [n], md[0], md[1])
            assert np.all(np.abs(h - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-6), f"block {b} ada_in"
        # QKV on the row subset
        for h, q, name in ((f(keep["h_v"])[rows], f(keep["q_v"])[rows], "video"),
                           (f(keep["h_t"]), f(keep["q_t"]), "text")):
            _close_bf16(q, oracle.linear(h, w["qkv"], bb["bqkv"], threads=16), f"block {b} qkv {name}")
        # attention on two windows (the first and a middle one): their video rows
        q_v, q_t = f(keep["q_v"]), f(keep["q_t"])
        subset = [0, len(wins) // 2]
        case = dict(video=q_v, text=q_t, norms=f(blk["norms"]), freqs=f(freqs))
        ref_v, _ = oracle_awa(case, H, HD, TARGET, b % 2, 1e-5, PAIRS, [SHAPE], [LT],
                              window_subset=subset, threads=16)
        pl = oracle.plan([SHAPE], TARGET, b % 2)
        for wi in subset:
            w0, n = pl.windows[wi][7], pl.windows[wi][8]
            src = pl.video_indices[w0:w0 + n]
            # the kernel also rounds the normalised q, k, v and the
            # probabilities to bf16: the path's bar (the outputs stay small)
            assert_close(f(keep["a_v"])[src], ref_v[src], f"block {b} attention window {wi}")
        # out, gate + residual (bit-exact), MLP norm, up (GELU), down on the rows
        a_v, o_v = f(keep["a_v"])[rows], f(keep["o_v"])[rows]
        _close_bf16(o_v, oracle.linear(a_v, w["o"], bb["bo"], threads=16), f"block {b} out")
        r1 = oracle.ada_out(x_v[rows], o_v, [len(rows)], md[2])
        np.testing.assert_array_equal(f(keep["r1_v"])[rows], r1)
        ref_m = oracle.ada_in(r1, [len(rows)], md[3], md[4])
        m_v = f(keep["m_v"])[rows]
        assert np.all(np.abs(m_v - ref_m) <= 2.0 ** -8 * np.abs(ref_m) + 1e-6), f"block {b} mlp norm"
        u_v = f(keep["u_v"])[rows]
        _close_bf16(u_v, oracle.linear(m_v, w["up"], bb["bup"], 1, threads=16), f"block {b} up")
        y_v = f(keep["y_v"])[rows]
        _close_bf16(y_v, oracle.linear(u_v, w["dn"], bb["bdn"], threads=16), f"block {b} down")
        np.testing.assert_array_equal(f(r_v)[rows], oracle.ada_out(r1, y_v, [len(rows)], md[5]))
