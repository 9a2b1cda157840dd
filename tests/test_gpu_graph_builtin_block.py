"""The two-block DiT graph written with ncnn built-ins in place of this
build's DiTAdaIn / DiTAdaOut / DiTAdaOutIn layers
(tests/golden/dit_blocks_2_builtin.param: RMSNorm written out as UnaryOp /
Reduction / BinaryOp in block 0 and as an RMSNorm layer in block 1, the
modulation as BinaryOp mul / add with MemoryData vectors, the gated residual
as BinaryOp mul / add, Splits wherever a blob has two readers), run by the
graph loader (seedvr2::DiTBlockGraph over ncnn::Net) on device blobs:

 1. as written (no folding; every built-in runs its own kernel), on one
    sample, against the fp32 oracle chain (oracle ada_in / linear with
    erf-GELU / the attention forward of adaptive_window_attention.cpp:
    764-978 / ada_out) at max-abs <= 2e-2 and cosine >= 0.9999;
 2. with its norm / modulation / residual chains folded onto the fused
    passes (dit_block_fold.h) and the QKV projection folded into the
    attention, bit for bit against the custom-layer graph
    (tests/golden/dit_blocks_2.param) on the same weights, on one and on two
    samples, and against the oracle chain;
 3. the unfolded and the folded graph agree at the bar.
The graph is fed in0..in9 as the reference's BlockGraph is
(src/seedvr2/seedvr2_dit.cpp:722-833)."""
import ctypes
import os
import sys

import numpy as np
import pytest

import oracle
from common import HBlob, assert_close, harness, oracle_awa

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import dit_graph  # noqa: E402

pytestmark = pytest.mark.gpu

D = dit_graph.HIDDEN


def _lib():
    L = harness()
    P, vp, ci = ctypes.POINTER, ctypes.c_void_p, ctypes.c_int
    L.h_graph_create.argtypes = [ctypes.c_char_p, vp, ctypes.c_long, ci, ci, P(vp)]
    L.h_graph_folded_modulation.argtypes = [vp]
    L.h_graph_fused_qkv.argtypes = [vp]
    L.h_graph_destroy.argtypes = [vp]
    L.h_graph_run.argtypes = [vp, P(ci), P(ci), ci, P(HBlob), P(HBlob), ci, P(ctypes.c_char_p)]
    return L


class Graph:
    def __init__(self, builtin, fuse):
        text = dit_graph.builtin_param_text() if builtin else dit_graph.param_text()
        w = dit_graph.block_weights()
        model = dit_graph.builtin_model_bytes(w) if builtin else dit_graph.model_bytes(w)
        self._buf = ctypes.create_string_buffer(model, len(model))
        self.h = ctypes.c_void_p()
        assert _lib().h_graph_create(text.encode(), self._buf, len(model), 0, fuse,
                                     ctypes.byref(self.h)) == 0
        self.folded = _lib().h_graph_folded_modulation(self.h)
        self.fused_qkv = _lib().h_graph_fused_qkv(self.h)

    def run(self, inputs, shapes, text, checkpoints=()):
        import torch
        blobs = (HBlob * 10)()
        keep = []
        for i, a in enumerate(inputs):
            a = np.ascontiguousarray(a)
            keep.append(a)
            blobs[i] = HBlob(a.ndim, a.shape[-1], a.shape[0] if a.ndim == 2 else 1, a.itemsize, 0,
                             a.ctypes.data)
        lv = sum(a * b * c for a, b, c in shapes)
        lt = sum(text)
        outs_t = [torch.empty(lv, D, device="cuda"), torch.empty(lt, D, device="cuda")]
        for name in checkpoints:
            outs_t.append(torch.empty(lv if name.endswith("_v") else lt, D, device="cuda"))
        outs = (HBlob * len(outs_t))()
        for i, t in enumerate(outs_t):
            outs[i] = HBlob(2, t.shape[1], t.shape[0], 4, 1, t.data_ptr())
        names = (ctypes.c_char_p * max(1, len(checkpoints)))(*[n.encode() for n in checkpoints])
        sh = np.asarray(shapes, np.int32).ravel()
        tl = np.asarray(text, np.int32)
        ret = _lib().h_graph_run(self.h, sh.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
                                 tl.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), len(shapes), blobs,
                                 outs, len(checkpoints), names)
        assert ret == 0, ret
        torch.cuda.synchronize()
        return [t.cpu().numpy() for t in outs_t]

    def close(self):
        if self.h:
            _lib().h_graph_destroy(self.h)
            self.h = None


def _inputs(seed, shapes, text):
    g = np.random.default_rng(seed)
    lv = sum(a * b * c for a, b, c in shapes)
    lt = sum(text)
    x_v = g.standard_normal((lv, D)).astype(np.float32)
    x_t = g.standard_normal((lt, D)).astype(np.float32)
    # video_shape Mat(3, batch), text_length Mat(1, batch) (seedvr2_dit.cpp:143-161)
    shape_blob = np.asarray(shapes, np.float32)
    tl_blob = np.asarray(text, np.float32).reshape(-1, 1)
    mods = [(0.1 * g.standard_normal((len(shapes), D)) + (1.0 if k in (1, 4) else 0.0)).astype(np.float32)
            for k in range(6)]   # a_shift a_scale a_gate m_shift m_scale m_gate
    return [x_v, x_t, shape_blob, tl_blob] + mods


def _oracle_chain(inputs, shapes, text):
    x_v, x_t = inputs[0], inputs[1]
    mods = inputs[4:]
    vr = [a * b * c for a, b, c in shapes]
    r_v, r_t = x_v.copy(), x_t.copy()
    for b, w in enumerate(dit_graph.block_weights()):
        s = w["stream"] or {}
        g = s.get
        h_v = oracle.ada_in(r_v, vr, mods[0], mods[1], g("vshift"), g("vscale"))
        h_t = oracle.ada_in(r_t, text, mods[0], mods[1], g("tshift"), g("tscale"))
        q_v = oracle.linear(h_v, w["qkv"], w["b_qkv"], threads=8)
        q_t = oracle.linear(h_t, w["qkv"], w["b_qkv"], threads=8)
        case = dict(video=q_v, text=q_t, norms=w["norms"], freqs=w["freqs"])
        a_v, a_t = oracle_awa(case, dit_graph.HEADS, dit_graph.HEAD_DIM, dit_graph.TARGET, b % 2, 1e-5,
                              dit_graph.PAIRS, shapes, text)
        o_v = oracle.linear(a_v, w["o"], w["b_o"], threads=8)
        o_t = oracle.linear(a_t, w["o"], w["b_o"], threads=8)
        r_v = oracle.ada_out(r_v, o_v, vr, mods[2], g("vgate"))
        r_t = oracle.ada_out(r_t, o_t, text, mods[2], g("tgate"))
        m_v = oracle.ada_in(r_v, vr, mods[3], mods[4], g("m_vshift"), g("m_vscale"))
        m_t = oracle.ada_in(r_t, text, mods[3], mods[4], g("m_tshift"), g("m_tscale"))
        u_v = oracle.linear(m_v, w["up"], w["b_up"], 1, threads=8)
        u_t = oracle.linear(m_t, w["up"], w["b_up"], 1, threads=8)
        y_v = oracle.linear(u_v, w["dn"], w["b_dn"], threads=8)
        y_t = oracle.linear(u_t, w["dn"], w["b_dn"], threads=8)
        r_v = oracle.ada_out(r_v, y_v, vr, mods[5], g("m_vgate"))
        r_t = oracle.ada_out(r_t, y_t, text, mods[5], g("m_tgate"))
    return r_v, r_t


ONE = ([(2, 6, 10)], [8])
TWO = ([(2, 6, 10), (1, 4, 6)], [8, 5])


def test_unfolded_builtin_graph_matches_the_oracle():
    """Every built-in runs as its own layer (BinaryOp broadcast of the
    [1][hidden] modulation rows: one sample)."""
    shapes, text = ONE
    inputs = _inputs(41, shapes, text)
    g = Graph(builtin=True, fuse=1)
    try:
        assert g.folded == 0 and g.fused_qkv == 0
        out = g.run(inputs, shapes, text)
    finally:
        g.close()
    rv, rt = _oracle_chain(inputs, shapes, text)
    assert_close(out[0], rv, "unfolded built-in graph out0 vs oracle")
    assert_close(out[1], rt, "unfolded built-in graph out1 vs oracle")


@pytest.mark.parametrize("case", [ONE, TWO], ids=["one_sample", "two_samples"])
def test_folded_builtin_graph_equals_the_custom_layer_graph(case):
    shapes, text = case
    inputs = _inputs(42, shapes, text)
    folded, custom = Graph(builtin=True, fuse=7), Graph(builtin=False, fuse=3)
    try:
        assert folded.folded == 10 and folded.fused_qkv == 2 and custom.fused_qkv == 2
        cps = ["b0_out_v", "b0_out_t"]
        got = folded.run(inputs, shapes, text, checkpoints=cps)
        ref = custom.run(inputs, shapes, text, checkpoints=cps)
        for a, b in zip(got, ref):
            np.testing.assert_array_equal(a, b)
        again = folded.run(inputs, shapes, text)   # pooled blocks
        np.testing.assert_array_equal(again[0], ref[0])
        np.testing.assert_array_equal(again[1], ref[1])
    finally:
        folded.close()
        custom.close()
    rv, rt = _oracle_chain(inputs, shapes, text)
    assert_close(got[0], rv, "folded built-in graph out0 vs oracle")
    assert_close(got[1], rt, "folded built-in graph out1 vs oracle")


def test_unfolded_and_folded_builtin_graphs_agree():
    shapes, text = ONE
    inputs = _inputs(43, shapes, text)
    plain, folded = Graph(builtin=True, fuse=1), Graph(builtin=True, fuse=5)
    try:
        a = plain.run(inputs, shapes, text)
        b = folded.run(inputs, shapes, text)
    finally:
        plain.close()
        folded.close()
    assert_close(a[0], b[0], "unfolded vs folded out0")
    assert_close(a[1], b[1], "unfolded vs folded out1")
