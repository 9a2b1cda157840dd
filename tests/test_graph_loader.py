"""The ncnn-compatible graph loader (ncnn::Net over the SeedVR2 layers,
seedvr2::DiTBlockGraph) on the CPU: parsing, weight loading, the
SharedLinear -> GELU folding and the error codes.  The loader replaces the
reference's Net::load_param / load_model of blocks/seedvr2_blocks.ncnn
(src/seedvr2/seedvr2_dit.cpp:603-633).  Running the graph is
tests/test_gpu_graph.py."""
import ctypes
import os
import sys

import pytest

from common import harness

sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
import dit_graph  # noqa: E402


def _lib():
    L = harness()
    P, vp, ci = ctypes.POINTER, ctypes.c_void_p, ctypes.c_int
    L.h_graph_create.argtypes = [ctypes.c_char_p, vp, ctypes.c_long, ci, ci, P(vp)]
    L.h_graph_fused_gelu.argtypes = [vp]
    L.h_graph_layer_count.argtypes = [vp]
    L.h_graph_fused_qkv.argtypes = [vp]
    L.h_graph_destroy.argtypes = [vp]
    return L


def _create(text, model, fuse=1, fp32_blobs=0, qkv=False):
    L = _lib()
    g = ctypes.c_void_p()
    buf = ctypes.create_string_buffer(model, max(1, len(model)))
    ret = L.h_graph_create(text.encode(), buf, len(model), fp32_blobs, fuse, ctypes.byref(g))
    info = None
    if ret == 0:
        info = (L.h_graph_layer_count(g), L.h_graph_fused_gelu(g))
        if qkv:
            info += (L.h_graph_fused_qkv(g),)
        L.h_graph_destroy(g)
    return ret, info


@pytest.fixture(scope="module")
def graph():
    with open(dit_graph.PARAM_PATH) as f:
        text = f.read()
    return text, dit_graph.model_bytes(dit_graph.block_weights())


def test_committed_param_is_the_generators(graph):
    assert graph[0] == dit_graph.param_text()


def test_header_counts_match_the_layer_lines(graph):
    lines = graph[0].strip().split("\n")
    assert lines[0] == "7767517"
    nl, nb = map(int, lines[1].split())
    body = lines[2:]
    assert len(body) == nl
    tops = set()
    for line in body:
        f = line.split()
        b, t = int(f[2]), int(f[3])
        tops.update(f[4 + b:4 + b + t])
    assert len(tops) == nb and {"out0", "out1"} <= tops


def test_loads_and_folds_gelu(graph):
    text, model = graph
    assert _create(text, model) == (0, (42, 2))
    assert _create(text, model, fuse=0) == (0, (42, 0))


def test_folds_the_qkv_projection_into_the_attention(graph):
    # both blocks' QKV SharedLinear -> AdaptiveWindowAttention pairs, on bf16
    # blobs only; the GELU folding is independent of it
    text, model = graph
    assert _create(text, model, fuse=3, qkv=True) == (0, (42, 2, 2))
    assert _create(text, model, fuse=2, qkv=True) == (0, (42, 0, 2))
    assert _create(text, model, fuse=3, fp32_blobs=1, qkv=True) == (0, (42, 2, 0))


@pytest.mark.parametrize("edit, code", [
    (lambda t: t.replace("7767517", "7767518", 1), -1),                          # magic
    (lambda t: t.replace("DiTAdaOut ", "NoSuchOp  ", 1), -1),                    # unknown type
    (lambda t: t.replace(" b0_h_v b0_h_t b0_qkv_v", " b0_h_v b0_h_x b0_qkv_v", 1), -1),  # no producer
    (lambda t: t.replace("0=256 1=256 2=1", "0=256 1=0 2=1", 1), -1),           # bad SharedLinear param
    (lambda t: t.replace("42 74", "43 74", 1), -1),                              # layer count
])
def test_malformed_param_is_rejected(graph, edit, code):
    text, model = graph
    assert _create(edit(text), model)[0] == code


def test_weight_file_must_match_the_graph(graph):
    text, model = graph
    assert _create(text, model[:-4])[0] == -100     # a layer runs out of weights
    assert _create(text, model + b"\0\0\0\0")[0] == -1   # bytes left over


def _linear_gelu_graph(act):
    """Two inputs -> SharedLinear (param 3 = act) -> GELU on both tops."""
    return ("7767517\n5 6\n"
            "Input in0 0 1 in0\n"
            "Input in1 0 1 in1\n"
            f"SharedLinear lin 2 2 in0 in1 a b 0=256 1=256 2=1 3={act}\n"
            "GELU g0 1 1 a ga 0=0\n"
            "GELU g1 1 1 b gb 0=0\n")


@pytest.mark.parametrize("act, folded", [(0, 1), (1, 0), (2, 0)])
def test_gelu_folds_only_into_a_projection_without_an_activation(act, folded):
    """A GELU after a projection that already has a GELU (param 3 = 1) or
    SwiGLU (3 = 2) epilogue stays a layer: folding it would drop one GELU,
    or run the interleaved gate/up weight as a plain GELU GEMM."""
    import numpy as np
    rows = 512 if act == 2 else 256
    model = np.zeros(rows * 256 + rows, np.float32).tobytes()
    ret, info = _create(_linear_gelu_graph(act), model)
    assert ret == 0 and info == (5, folded)


@pytest.mark.parametrize("edit", [
    lambda t: t.replace("Input                    in9              0 1 in9",
                        "Input                    in9              0 2 in9", 1),       # short top list
    lambda t: t.replace("Split                    split_in2        1 2 in2 in2_s0 in2_s1",
                        "Split                    split_in2        3 2", 1),           # short bottom list
])
def test_short_blob_lists_leave_an_empty_net(graph, edit):
    """A line whose bottom or top list ends early is refused and leaves no
    half-built net behind: load_model on the same net then fails too."""
    text, model = graph
    edited = edit(text)
    assert edited != text
    L = harness()
    P = ctypes.POINTER
    L.h_net_load.argtypes = [ctypes.c_char_p, ctypes.c_void_p, ctypes.c_long, P(ctypes.c_int),
                             P(ctypes.c_int)]
    pr, mr = ctypes.c_int(), ctypes.c_int()
    buf = ctypes.create_string_buffer(model, len(model))
    layers = L.h_net_load(edited.encode(), buf, len(model), ctypes.byref(pr), ctypes.byref(mr))
    assert pr.value == -1 and mr.value == -1 and layers == 0


# ---- the same blocks written with ncnn built-ins ------------------------------------


@pytest.fixture(scope="module")
def builtin_graph():
    with open(dit_graph.BUILTIN_PARAM_PATH) as f:
        text = f.read()
    return text, dit_graph.builtin_model_bytes(dit_graph.block_weights())


def _create_counts(text, model, fuse):
    L = _lib()
    L.h_graph_folded_modulation.argtypes = [ctypes.c_void_p]
    g = ctypes.c_void_p()
    buf = ctypes.create_string_buffer(model, max(1, len(model)))
    ret = L.h_graph_create(text.encode(), buf, len(model), 0, fuse, ctypes.byref(g))
    if ret != 0:
        return ret, None
    counts = (L.h_graph_fused_gelu(g), L.h_graph_folded_modulation(g), L.h_graph_fused_qkv(g))
    L.h_graph_destroy(g)
    return 0, counts


def test_committed_builtin_param_is_the_generators(builtin_graph):
    assert builtin_graph[0] == dit_graph.builtin_param_text()


def test_builtin_graph_uses_only_ncnn_layer_types(builtin_graph):
    types = {line.split()[0] for line in builtin_graph[0].strip().split("\n")[2:]}
    assert types == {"Input", "Split", "UnaryOp", "Reduction", "BinaryOp", "RMSNorm", "MemoryData",
                     "SharedLinear", "AdaptiveWindowAttention", "GELU"}


def test_builtin_graph_folds_its_norm_modulation_and_residual_chains(builtin_graph):
    """Per block and stream: the attention's ada_in, its gated residual merged
    with the MLP's ada_in (ada_out_in), and the MLP's gated residual, which
    for block 0 merges with block 1's attention ada_in: 2 x (2 + 2) + 2
    passes.  Without the fold the graph loads as written."""
    text, model = builtin_graph
    assert _create_counts(text, model, 7) == (0, (2, 10, 2))
    assert _create_counts(text, model, 1) == (0, (2, 0, 0))
    assert _create_counts(text, model, 5) == (0, (2, 10, 0))


def test_chain_with_an_extra_consumer_is_not_folded(builtin_graph):
    """A norm whose intermediate blob has a second reader stays as written:
    here block 0's video mean of squares also feeds an extra layer, so that
    stream's attention ada_in is not folded (9 passes instead of 10)."""
    text, model = builtin_graph
    lines = text.strip().split("\n")
    nl, nb = map(int, lines[1].split())
    body = lines[2:] + ["UnaryOp extra 1 1 b0_an_v_ms extra_out 0=0"]
    edited = "7767517\n" + f"{nl + 1} {nb + 1}\n" + "\n".join(body) + "\n"
    ret, counts = _create_counts(edited, model, 5)
    assert ret == 0 and counts[1] == 9


# ---- the v3 graph form: split q / k / v and the SwiGLU MLP --------------------------


def test_committed_v3_param_is_the_generators():
    with open(dit_graph.V3_PARAM_PATH) as f:
        assert f.read() == dit_graph.v3_param_text()


def test_v3_graph_folds_split_qkv_and_swiglu():
    text = dit_graph.v3_param_text()
    model = dit_graph.v3_model_bytes(dit_graph.v3_block_weights())
    L = _lib()
    L.h_graph_fused_swiglu.argtypes = [ctypes.c_void_p]
    for fuse, fp32, want in ((3, 0, (2, 2)), (2, 0, (0, 2)), (1, 0, (2, 0)), (0, 0, (0, 0)), (3, 1, (0, 0))):
        g = ctypes.c_void_p()
        buf = ctypes.create_string_buffer(model, len(model))
        assert L.h_graph_create(text.encode(), buf, len(model), fp32, fuse, ctypes.byref(g)) == 0
        got = (L.h_graph_fused_swiglu(g), L.h_graph_fused_qkv(g))
        L.h_graph_destroy(g)
        assert got == want, (fuse, fp32, got)
