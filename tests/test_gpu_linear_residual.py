"""s2_shared_linear_residual on the GPU: the block's out / MLP-down projection
with the gated residual sum in its epilogue.  It must equal, bit for bit,
s2_shared_linear_forward with bf16 y followed by s2_dit_ada_out on that y
(the two calls a block makes when the projection output is a blob,
seedvr2_dit.cpp:722-833; shared_linear.cpp:83-96), for fp32 and bf16
residual streams, in place and out of place, with and without per-stream
gate vectors, on 3B-sized rows (hidden 2560, k 2560 and the MLP's 10240 with
the split-k tail), several samples per stream and no text.  One small case is
also held to the oracle (the fp32 product of the bf16 operands, rounded to
bf16, then oracle.ada_out) at the path's bar."""
import numpy as np
import pytest

import oracle
from common import assert_close

pytestmark = pytest.mark.gpu


def _case(seed, vrows, trows, n, k, res_dtype):
    import torch
    g = torch.Generator().manual_seed(seed)
    dev = "cuda"
    mv, mt = sum(vrows), sum(trows or [0])
    x_v = (torch.randn(mv, k, generator=g)).to(torch.bfloat16).to(dev)
    x_t = (torch.randn(mt, k, generator=g)).to(torch.bfloat16).to(dev) if mt else None
    w = (0.02 * torch.randn(n, k, generator=g)).to(torch.bfloat16).to(dev)
    b = (0.02 * torch.randn(n, generator=g)).to(dev)
    r_v = torch.randn(mv, n, generator=g).to(res_dtype).to(dev)
    r_t = torch.randn(mt, n, generator=g).to(res_dtype).to(dev) if mt else None
    gate = (0.5 + 0.1 * torch.randn(len(vrows), n, generator=g)).to(dev)
    gv = (0.1 * torch.randn(n, generator=g)).to(dev)
    gt = (0.1 * torch.randn(n, generator=g)).to(dev)
    return x_v, x_t, w, b, r_v, r_t, gate, gv, gt


def _two_calls(x_v, x_t, w, b, vrows, trows, r_v, r_t, gate, gv, gt):
    import torch
    from seedvr2_ncnn_amd import capi
    y_v, y_t = capi.shared_linear(x_v, x_t, w, b, out_dtype=torch.bfloat16)
    o_v = r_v.clone()
    o_t = r_t.clone() if r_t is not None else None
    capi.ada_out(o_v, o_t, y_v, y_t, vrows, trows, gate, gv, gt)
    return o_v, o_t


CASES = [
    # (video rows per sample, text rows per sample, n, k)
    ([3000, 1234], [77, 58], 2560, 2560),
    ([2048, 700], [120, 9], 2560, 10240),
    ([5000], None, 2560, 2560),
    ([513, 1, 96], [0, 31, 200], 1024, 512),
]


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("res_dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("in_place", [True, False])
@pytest.mark.parametrize("stream_gates", [True, False])
def test_fused_equals_linear_then_ada_out(case, res_dtype, in_place, stream_gates):
    import torch
    from seedvr2_ncnn_amd import capi
    vrows, trows, n, k = CASES[case]
    x_v, x_t, w, b, r_v, r_t, gate, gv, gt = _case(7 + case, vrows, trows, n, k,
                                                   getattr(torch, res_dtype))
    if not stream_gates:
        gv = gt = None
    want_v, want_t = _two_calls(x_v, x_t, w, b, vrows, trows, r_v, r_t, gate, gv, gt)
    if in_place:
        o_v, o_t = r_v.clone(), (r_t.clone() if r_t is not None else None)
        capi.shared_linear_residual(x_v, x_t, w, b, vrows, trows, o_v, o_t, gate, gv, gt)
    else:
        o_v = torch.full_like(r_v, float("nan"))
        o_t = torch.full_like(r_t, float("nan")) if r_t is not None else None
        capi.shared_linear_residual(x_v, x_t, w, b, vrows, trows, r_v, r_t, gate, gv, gt,
                                    out_video=o_v, out_text=o_t)
    torch.cuda.synchronize()
    assert torch.equal(o_v, want_v)
    if r_t is not None:
        assert torch.equal(o_t, want_t)


def test_fused_residual_against_the_oracle():
    import torch
    from seedvr2_ncnn_amd import capi
    vrows, trows, n, k = [300, 77], [13, 20], 512, 1024
    x_v, x_t, w, b, r_v, r_t, gate, gv, gt = _case(3, vrows, trows, n, k, torch.float32)
    want_v = r_v.cpu().numpy().copy()
    want_t = r_t.cpu().numpy().copy()
    o_v, o_t = capi.shared_linear_residual(x_v, x_t, w, b, vrows, trows, r_v, r_t, gate, gv, gt)
    torch.cuda.synchronize()
    wf = w.float().cpu().numpy()
    bf = b.cpu().numpy()
    for x, rows, res, gs, got, name in ((x_v, vrows, want_v, gv, o_v, "video"),
                                        (x_t, trows, want_t, gt, o_t, "text")):
        y = oracle.linear(x.float().cpu().numpy(), wf, bf, threads=8)
        want = oracle.ada_out(res, y, rows, gate.cpu().numpy(), gs.cpu().numpy())
        assert_close(got.cpu().numpy(), want, f"fused residual {name} vs oracle")


def test_argument_errors():
    import torch
    from seedvr2_ncnn_amd import capi
    x_v, x_t, w, b, r_v, r_t, gate, gv, gt = _case(5, [64], [8], 256, 256, torch.float32)
    with pytest.raises(capi.S2Error):   # row counts do not sum to m_video
        capi.shared_linear_residual(x_v, x_t, w, b, [63], [8], r_v, r_t, gate)
    w_odd = torch.zeros(256, 96, dtype=torch.bfloat16, device="cuda")
    x_odd = torch.zeros(64, 96, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(capi.S2Error):   # k % 64 != 0
        capi.shared_linear_residual(x_odd, None, w_odd, b, [64], None, r_v, None, gate)
