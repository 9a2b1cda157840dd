"""The DiT block graph run by the graph loader (seedvr2::DiTBlockGraph over
ncnn::Net) on device-resident blobs, on the GPU.

The graph is tests/golden/dit_blocks_2.param (two blocks, regular then
shifted windows, block 1 with its own per-stream modulation vectors) with
seeded weights (tests/golden/dit_graph.py).  It is fed in0..in9 as the
reference's BlockGraph is (src/seedvr2/seedvr2_dit.cpp:722-833) and checked
 1. bit for bit against the same block chain called stage by stage through
    the C-ABI (s2_dit_ada_in, s2_shared_linear_forward, s2_awa_forward,
    s2_dit_ada_out_in, s2_dit_ada_out; each stage is itself held to the
    oracle by test_gpu_dit_block.py and the layer tests), including a block
    boundary blob extracted as a checkpoint;
 2. against the fp32 oracle chain end to end (oracle.ada_in, oracle.linear
    with erf-GELU, the attention forward of adaptive_window_attention.cpp:
    764-978, oracle.ada_out) at max-abs <= 2e-2 and cosine >= 0.9999;
 3. with the GELU layers left as layers (no folding into SharedLinear), bit
    for bit against the chain with s2_gelu, and a second run of the same
    graph, which reuses pooled device blocks, against the first;
 4. with each QKV SharedLinear folded into its attention layer
    (s2_awa_qkv_forward), bit for bit against the unfused graph."""
import ctypes
import os
import sys

import numpy as np
import pytest

import oracle
from common import HBlob, assert_close, harness, oracle_awa
from seedvr2_ncnn_amd import capi

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import dit_graph  # noqa: E402

pytestmark = pytest.mark.gpu

SHAPES = [(2, 6, 10), (1, 4, 6)]
TEXT = [8, 5]
D = dit_graph.HIDDEN


def _lib():
    L = harness()
    P, vp, ci = ctypes.POINTER, ctypes.c_void_p, ctypes.c_int
    L.h_graph_create.argtypes = [ctypes.c_char_p, vp, ctypes.c_long, ci, ci, P(vp)]
    L.h_graph_fused_gelu.argtypes = [vp]
    L.h_graph_fused_qkv.argtypes = [vp]
    L.h_graph_destroy.argtypes = [vp]
    L.h_graph_run.argtypes = [vp, P(ci), P(ci), ci, P(HBlob), P(HBlob), ci,
                              P(ctypes.c_char_p)]
    return L


class Graph:
    def __init__(self, fuse=1):
        """fuse: bit 0 folds SharedLinear -> GELU, bit 1 the QKV SharedLinear
        into the attention layer."""
        with open(dit_graph.PARAM_PATH) as f:
            text = f.read()
        self.weights = dit_graph.block_weights()
        model = dit_graph.model_bytes(self.weights)
        self._buf = ctypes.create_string_buffer(model, len(model))
        self.h = ctypes.c_void_p()
        assert _lib().h_graph_create(text.encode(), self._buf, len(model), 0, int(fuse),
                                     ctypes.byref(self.h)) == 0
        self.fused = _lib().h_graph_fused_gelu(self.h)
        self.fused_qkv = _lib().h_graph_fused_qkv(self.h)

    def run(self, inputs, checkpoints=()):
        """inputs: 10 torch tensors (device) or numpy arrays (host) for in0..in9.
        Returns device torch tensors: out0, out1, then the checkpoints."""
        import torch
        blobs = (HBlob * 10)()
        keep = []
        for i, t in enumerate(inputs):
            if isinstance(t, np.ndarray):
                a = np.ascontiguousarray(t)
                keep.append(a)
                blobs[i] = HBlob(a.ndim, a.shape[-1], a.shape[0] if a.ndim == 2 else 1,
                                 a.itemsize, 0, a.ctypes.data)
            else:
                blobs[i] = HBlob(t.dim(), t.shape[-1], t.shape[0] if t.dim() == 2 else 1,
                                 t.element_size(), 1, t.data_ptr())
        lv = sum(a * b * c for a, b, c in SHAPES)
        lt = sum(TEXT)
        outs_t = [torch.empty(lv, D, device="cuda"), torch.empty(lt, D, device="cuda")]
        for name in checkpoints:
            outs_t.append(torch.empty(lv if name.endswith("_v") else lt, D, device="cuda"))
        outs = (HBlob * len(outs_t))()
        for i, t in enumerate(outs_t):
            outs[i] = HBlob(2, t.shape[1], t.shape[0], 4, 1, t.data_ptr())
        names = (ctypes.c_char_p * max(1, len(checkpoints)))(*[n.encode() for n in checkpoints])
        shapes = np.asarray(SHAPES, np.int32).ravel()
        tl = np.asarray(TEXT, np.int32)
        ret = _lib().h_graph_run(self.h, shapes.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
                                 tl.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), len(SHAPES),
                                 blobs, outs, len(checkpoints), names)
        assert ret == 0, ret
        for i in range(len(outs_t)):   # all fp32 residual blobs
            assert outs[i].elemsize == 4 and outs[i].h == outs_t[i].shape[0]
        return outs_t

    def close(self):
        if self.h:
            _lib().h_graph_destroy(self.h)
            self.h = None


def _inputs(seed):
    g = np.random.default_rng(seed)
    lv = sum(a * b * c for a, b, c in SHAPES)
    lt = sum(TEXT)
    x_v = g.standard_normal((lv, D)).astype(np.float32)
    x_t = g.standard_normal((lt, D)).astype(np.float32)
    # the reference's shape blobs: video_shape Mat(3, batch), text_length
    # Mat(1, batch) (src/seedvr2/seedvr2_dit.cpp:143-161), which the
    # attention layers decode on the host
    shape_blob = np.asarray(SHAPES, np.float32)
    tl_blob = np.asarray(TEXT, np.float32).reshape(-1, 1)
    mods = [(0.1 * g.standard_normal((len(SHAPES), D)) + (1.0 if k in (1, 4) else 0.0)).astype(np.float32)
            for k in range(6)]   # a_shift a_scale a_gate m_shift m_scale m_gate
    return x_v, x_t, shape_blob, tl_blob, mods


def _chain(x_v, x_t, mods, weights, gelu_layer=False, stop_after=None):
    """The graph's blocks called stage by stage through the C-ABI."""
    import torch
    bf = torch.bfloat16
    vr = [a * b * c for a, b, c in SHAPES]
    f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    md = [f32(m) for m in mods]
    r_v, r_t = f32(x_v), f32(x_t)
    for b, w in enumerate(weights):
        s = w["stream"]
        sv = (lambda k: f32(s[k])) if s is not None else (lambda k: None)
        h_v, h_t = capi.ada_in(r_v, r_t, vr, TEXT, md[0], md[1], video_shift=sv("vshift"),
                               video_scale=sv("vscale"), text_shift=sv("tshift"),
                               text_scale=sv("tscale"), out_dtype=bf)
        wq = f32(w["qkv"]).to(bf)
        q_v, q_t = capi.shared_linear(h_v, h_t, wq, f32(w["b_qkv"]), capi.ACT_NONE)
        cfg = capi.awa_config(dit_graph.HEADS, dit_graph.HEAD_DIM, dit_graph.TARGET, b % 2, 1e-5,
                              dit_graph.PAIRS)
        with capi.AwaPlan(cfg, SHAPES, TEXT) as plan:
            a_v, a_t = capi.awa_forward(plan, f32(w["norms"]), f32(w["freqs"]), q_v[:, :D],
                                        q_v[:, D:2 * D], q_v[:, 2 * D:], q_t[:, :D],
                                        q_t[:, D:2 * D], q_t[:, 2 * D:])
            torch.cuda.synchronize()
        o_v, o_t = capi.shared_linear(a_v, a_t, f32(w["o"]).to(bf), f32(w["b_o"]), capi.ACT_NONE)
        r1_v, r1_t = torch.empty_like(r_v), torch.empty_like(r_t)
        _, _, m_v, m_t = capi.ada_out_in(r_v, r_t, o_v, o_t, vr, TEXT, md[2], md[3], md[4],
                                         video_gate=sv("vgate"), text_gate=sv("tgate"),
                                         video_shift=sv("m_vshift"), video_scale=sv("m_vscale"),
                                         text_shift=sv("m_tshift"), text_scale=sv("m_tscale"),
                                         out_video=r1_v, out_text=r1_t)
        wu = f32(w["up"]).to(bf)
        if gelu_layer:
            u_v, u_t = capi.shared_linear(m_v, m_t, wu, f32(w["b_up"]), capi.ACT_NONE)
            u_v, u_t = capi.gelu(u_v), capi.gelu(u_t)
        else:
            u_v, u_t = capi.shared_linear(m_v, m_t, wu, f32(w["b_up"]), capi.ACT_GELU)
        y_v, y_t = capi.shared_linear(u_v, u_t, f32(w["dn"]).to(bf), f32(w["b_dn"]), capi.ACT_NONE)
        r_v, r_t = capi.ada_out(r1_v, r1_t, y_v, y_t, vr, TEXT, md[5], video_gate=sv("m_vgate"),
                                text_gate=sv("m_tgate"), out_video=torch.empty_like(r1_v),
                                out_text=torch.empty_like(r1_t))
        if stop_after == b:
            break
    torch.cuda.synchronize()
    return r_v, r_t


def _oracle_chain(x_v, x_t, mods, weights):
    vr = [a * b * c for a, b, c in SHAPES]
    r_v, r_t = x_v.copy(), x_t.copy()
    for b, w in enumerate(weights):
        s = w["stream"] or {}
        g = s.get
        h_v = oracle.ada_in(r_v, vr, mods[0], mods[1], g("vshift"), g("vscale"))
        h_t = oracle.ada_in(r_t, TEXT, mods[0], mods[1], g("tshift"), g("tscale"))
        q_v = oracle.linear(h_v, w["qkv"], w["b_qkv"], threads=8)
        q_t = oracle.linear(h_t, w["qkv"], w["b_qkv"], threads=8)
        case = dict(video=q_v, text=q_t, norms=w["norms"], freqs=w["freqs"])
        a_v, a_t = oracle_awa(case, dit_graph.HEADS, dit_graph.HEAD_DIM, dit_graph.TARGET, b % 2,
                              1e-5, dit_graph.PAIRS, SHAPES, TEXT)
        o_v = oracle.linear(a_v, w["o"], w["b_o"], threads=8)
        o_t = oracle.linear(a_t, w["o"], w["b_o"], threads=8)
        r_v = oracle.ada_out(r_v, o_v, vr, mods[2], g("vgate"))
        r_t = oracle.ada_out(r_t, o_t, TEXT, mods[2], g("tgate"))
        m_v = oracle.ada_in(r_v, vr, mods[3], mods[4], g("m_vshift"), g("m_vscale"))
        m_t = oracle.ada_in(r_t, TEXT, mods[3], mods[4], g("m_tshift"), g("m_tscale"))
        u_v = oracle.linear(m_v, w["up"], w["b_up"], 1, threads=8)
        u_t = oracle.linear(m_t, w["up"], w["b_up"], 1, threads=8)
        y_v = oracle.linear(u_v, w["dn"], w["b_dn"], threads=8)
        y_t = oracle.linear(u_t, w["dn"], w["b_dn"], threads=8)
        r_v = oracle.ada_out(r_v, y_v, vr, mods[5], g("m_vgate"))
        r_t = oracle.ada_out(r_t, y_t, TEXT, mods[5], g("m_tgate"))
    return r_v, r_t


def test_graph_matches_the_stage_chain_and_the_oracle():
    import torch
    x_v, x_t, shape_blob, tl_blob, mods = _inputs(1)
    g = Graph(fuse=True)
    try:
        assert g.fused == 2
        # in0/in1 and the modulation vectors as host Mats (uploaded once by
        # the graph), the shape blobs as host Mats
        outs = g.run([x_v, x_t, shape_blob, tl_blob] + mods, checkpoints=["b0_out_v", "b0_out_t"])
        ref_v, ref_t = _chain(x_v, x_t, mods, g.weights)
        np.testing.assert_array_equal(outs[0].cpu().numpy(), ref_v.cpu().numpy())
        np.testing.assert_array_equal(outs[1].cpu().numpy(), ref_t.cpu().numpy())
        b0_v, b0_t = _chain(x_v, x_t, mods, g.weights, stop_after=0)
        np.testing.assert_array_equal(outs[2].cpu().numpy(), b0_v.cpu().numpy())
        np.testing.assert_array_equal(outs[3].cpu().numpy(), b0_t.cpu().numpy())
        # a second run with device inputs reuses the pooled blocks
        dev = [torch.from_numpy(a).cuda() if i not in (2, 3) else a
               for i, a in enumerate([x_v, x_t, shape_blob, tl_blob] + mods)]
        outs2 = g.run(dev)
        np.testing.assert_array_equal(outs2[0].cpu().numpy(), ref_v.cpu().numpy())
        np.testing.assert_array_equal(outs2[1].cpu().numpy(), ref_t.cpu().numpy())
    finally:
        g.close()
    o_v, o_t = _oracle_chain(x_v, x_t, mods, dit_graph.block_weights())
    assert_close(outs[0].cpu().numpy(), o_v, "graph out0 vs oracle")
    assert_close(outs[1].cpu().numpy(), o_t, "graph out1 vs oracle")


def test_graph_with_gelu_layers_matches_the_chain_with_s2_gelu():
    x_v, x_t, shape_blob, tl_blob, mods = _inputs(2)
    g = Graph(fuse=False)
    try:
        assert g.fused == 0
        outs = g.run([x_v, x_t, shape_blob, tl_blob] + mods)
        ref_v, ref_t = _chain(x_v, x_t, mods, g.weights, gelu_layer=True)
        np.testing.assert_array_equal(outs[0].cpu().numpy(), ref_v.cpu().numpy())
        np.testing.assert_array_equal(outs[1].cpu().numpy(), ref_t.cpu().numpy())
    finally:
        g.close()


def test_s2_gelu_against_the_erf_closed_form():
    import torch
    x = torch.linspace(-8, 8, 4099, device="cuda")
    ref = torch.nn.functional.gelu(x.double()).float()
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        y = capi.gelu(x.to(dt)).float()
        torch.cuda.synchronize()
        want = torch.nn.functional.gelu(x.to(dt).double()).to(dt).float()
        tol = 2e-6 if dt == torch.float32 else 1e-2
        assert float((y - want).abs().max()) <= tol * max(1.0, float(want.abs().max())), dt
    assert float((capi.gelu(x) - ref).abs().max()) < 2e-6


def test_graph_with_qkv_folded_into_the_attention_matches_the_unfused_graph():
    """ncnn::Net::fuse_qkv_attention: each block's QKV projection runs inside
    its attention layer (s2_awa_qkv_forward, which rounds the projection to
    bf16 exactly as the QKV blob holds it; k = 256 is not split, so every
    element accumulates in the same order).  Outputs equal the unfused
    graph's bit for bit, on a first run and on a second one over pooled
    device blocks; the folded QKV blob can no longer be extracted."""
    import torch
    x_v, x_t, shape_blob, tl_blob, mods = _inputs(3)
    inputs = [x_v, x_t, shape_blob, tl_blob] + mods
    plain, fused = Graph(fuse=1), Graph(fuse=3)
    try:
        assert plain.fused_qkv == 0 and fused.fused_qkv == 2 and fused.fused == 2
        ref = plain.run(inputs)
        for _ in range(2):
            got = fused.run(inputs)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(got[0].cpu().numpy(), ref[0].cpu().numpy())
            np.testing.assert_array_equal(got[1].cpu().numpy(), ref[1].cpu().numpy())
        with pytest.raises(AssertionError):
            fused.run(inputs, checkpoints=["b0_qkv_v"])
    finally:
        plain.close()
        fused.close()


def test_graph_orders_itself_behind_inputs_from_another_stream():
    """Device inputs produced on another stream, by an allocator of that
    stream, and handed over without a host synchronisation: the graph's
    stream waits for that stream (ncnn::Extractor::input, s2_stream_wait)
    and every layer runs on the graph's stream.  The producer stream first
    spins, then writes the real inputs over garbage, so a graph that did not
    wait would read the garbage."""
    import torch
    x_v, x_t, shape_blob, tl_blob, mods = _inputs(4)
    host = [x_v, x_t, shape_blob, tl_blob] + mods
    g = Graph(fuse=3)
    try:
        ref = g.run(host)
        torch.cuda.synchronize()
        ref = [r.clone() for r in ref]
        side = torch.cuda.Stream()
        dev = [torch.full(a.shape, float("nan"), device="cuda") if i not in (2, 3) else a
               for i, a in enumerate(host)]
        src = [torch.from_numpy(a).cuda() if i not in (2, 3) else None for i, a in enumerate(host)]
        torch.cuda.synchronize()
        with torch.cuda.stream(side):
            torch.cuda._sleep(20_000_000)   # a bounded spin (cycles) on the producer stream
            for i, t in enumerate(dev):
                if i not in (2, 3):
                    t.copy_(src[i])
        blobs = (HBlob * 10)()
        keep = []
        for i, t in enumerate(dev):
            if isinstance(t, np.ndarray):
                keep.append(t)
                blobs[i] = HBlob(t.ndim, t.shape[-1], t.shape[0] if t.ndim == 2 else 1, 4, 0,
                                 t.ctypes.data)
            else:
                blobs[i] = HBlob(t.dim(), t.shape[-1], t.shape[0], 4, 1, t.data_ptr())
        lv, lt = sum(a * b * c for a, b, c in SHAPES), sum(TEXT)
        outs_t = [torch.empty(lv, D, device="cuda"), torch.empty(lt, D, device="cuda")]
        outs = (HBlob * 2)()
        for i, t in enumerate(outs_t):
            outs[i] = HBlob(2, t.shape[1], t.shape[0], 4, 1, t.data_ptr())
        shapes = np.asarray(SHAPES, np.int32).ravel()
        tl = np.asarray(TEXT, np.int32)
        L = _lib()
        L.h_graph_run_from_stream.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int),
                                              ctypes.POINTER(ctypes.c_int), ctypes.c_int,
                                              ctypes.POINTER(HBlob), ctypes.POINTER(HBlob),
                                              ctypes.c_void_p]
        ret = L.h_graph_run_from_stream(g.h, shapes.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
                                        tl.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), len(SHAPES),
                                        blobs, outs, ctypes.c_void_p(side.cuda_stream))
        assert ret == 0, ret
        torch.cuda.synchronize()
        np.testing.assert_array_equal(outs_t[0].cpu().numpy(), ref[0].cpu().numpy())
        np.testing.assert_array_equal(outs_t[1].cpu().numpy(), ref[1].cpu().numpy())
    finally:
        g.close()


def test_repeated_runs_keep_a_fixed_set_of_device_blocks():
    """Host inputs are uploaded into blocks the extractor owns and pools
    again once consumed (the shape blobs in2 / in3 are read on the host and
    never uploaded), and each run's outputs go back to the pool at the next
    run: the graph's allocator holds the same number of blocks after every
    run from the second on."""
    import torch
    x_v, x_t, shape_blob, tl_blob, mods = _inputs(5)
    host = [x_v, x_t, shape_blob, tl_blob] + mods
    L = _lib()
    L.h_graph_owned_blocks.argtypes = [ctypes.c_void_p]
    L.h_graph_owned_blocks.restype = ctypes.c_long
    g = Graph(fuse=3)
    try:
        counts = []
        for _ in range(4):
            g.run(host)
            torch.cuda.synchronize()
            counts.append(L.h_graph_owned_blocks(g.h))
        assert counts[1] == counts[2] == counts[3], counts
    finally:
        g.close()
