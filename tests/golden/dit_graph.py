"""Writes a small fused DiT block graph in ncnn's text .param / raw .bin
format, with seeded random weights, for the graph-loader tests.

The exported blocks/seedvr2_blocks.ncnn graph (loaded by the reference at
src/seedvr2/seedvr2_dit.cpp:603-633, run at :722-833) is not in the
reference repository.  This graph follows its interface (inputs in0 video,
in1 text, in2 video_shape, in3 text_length, in4..in9 the six per-sample
modulation vectors; outputs out0 / out1) and the published NaDiT block
restated for this build: per block
    DiTAdaIn -> SharedLinear (QKV) -> AdaptiveWindowAttention (4-input form)
    -> SharedLinear (out) -> DiTAdaOutIn -> SharedLinear (MLP up) -> GELU x 2
    -> SharedLinear (MLP down) -> DiTAdaOut
with Split layers wherever a blob has more than one consumer, as ncnn graphs
have.  Even blocks use regular windows, odd blocks shifted ones; block 1
carries the block's own per-stream modulation vectors (param 2 = 1).

Usage: python tests/golden/dit_graph.py  rewrites dit_blocks_2.param,
dit_blocks_2_builtin.param and dit_blocks_2_v3.param here.
"""
from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PARAM_PATH = os.path.join(HERE, "dit_blocks_2.param")

# Shapes of the committed graph.
HEADS, HEAD_DIM, PAIRS = 2, 128, 21
HIDDEN = HEADS * HEAD_DIM
MLP = 4 * HIDDEN
TARGET = (4, 3, 3)
BLOCKS = 2
SEED = 2024


def _bf16(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    bits = a.view(np.uint32).astype(np.uint64)
    bits = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
    return bits.astype(np.uint32).view(np.float32).reshape(a.shape)


def block_weights(blocks=BLOCKS, seed=SEED):
    """Per block: the GEMM weights (rounded to bf16, as the layer keeps them
    on the device) and fp32 biases, the attention norm weights and RoPE
    frequencies, and, for odd blocks, the block's own modulation vectors."""
    g = np.random.default_rng(seed)
    out = []
    for b in range(blocks):
        w = {}
        for name, n, k in (("qkv", 3 * HIDDEN, HIDDEN), ("o", HIDDEN, HIDDEN), ("up", MLP, HIDDEN),
                           ("dn", HIDDEN, MLP)):
            w[name] = _bf16(0.02 * g.standard_normal((n, k)))
            w["b_" + name] = (0.02 * g.standard_normal(n)).astype(np.float32)
        w["norms"] = (1.0 + 0.02 * g.standard_normal((4, HEAD_DIM))).astype(np.float32)
        w["freqs"] = (10000.0 ** (-np.arange(PAIRS, dtype=np.float64) / PAIRS)).astype(np.float32)
        w["stream"] = None
        if b % 2 == 1:
            # video_shift, video_scale, text_shift, text_scale, video_gate, text_gate
            w["stream"] = {k: (0.05 * g.standard_normal(HIDDEN)).astype(np.float32)
                           for k in ("vshift", "vscale", "tshift", "tscale", "vgate", "tgate",
                                     "m_vshift", "m_vscale", "m_tshift", "m_tscale",
                                     "m_vgate", "m_tgate")}
        out.append(w)
    return out


def param_text(blocks=BLOCKS):
    """The .param text of a `blocks`-block graph."""
    layers = []

    def add(type_, name, bottoms, tops, params=""):
        line = f"{type_:<24} {name:<16} {len(bottoms)} {len(tops)} " + " ".join(bottoms + tops)
        layers.append(line + (" " + params if params else ""))

    for i in range(10):
        add("Input", f"in{i}", [], [f"in{i}"])
    # every shared input feeds one consumer per block
    def split(blob, n):
        if n == 1:
            return [blob]
        tops = [f"{blob}_s{i}" for i in range(n)]
        add("Split", f"split_{blob}", [blob], tops)
        return tops
    vshape = split("in2", blocks)
    tlen = split("in3", blocks)
    mods = [split(f"in{4 + i}", blocks) for i in range(6)]   # a_shift a_scale a_gate m_shift m_scale m_gate
    rv, rt = "in0", "in1"
    for b in range(blocks):
        p = f"b{b}_"
        sv = 1 if b % 2 == 1 else 0
        rv0, rv1 = split(rv, 2)
        rt0, rt1 = split(rt, 2)
        add("DiTAdaIn", p + "ada_in", [rv0, rt0, mods[0][b], mods[1][b]], [p + "h_v", p + "h_t"],
            f"0={HIDDEN} 1=1.000000e-05 2={sv}")
        add("SharedLinear", p + "qkv", [p + "h_v", p + "h_t"], [p + "qkv_v", p + "qkv_t"],
            f"0={3 * HIDDEN} 1={HIDDEN} 2=1")
        add("AdaptiveWindowAttention", p + "attn", [p + "qkv_v", p + "qkv_t", vshape[b], tlen[b]],
            [p + "a_v", p + "a_t"],
            f"0={HEADS} 1={HEAD_DIM} 2={TARGET[0]} 3={TARGET[1]} 4={TARGET[2]} 5={b % 2} "
            f"6=1.000000e-05 7={PAIRS} 8=0 9=0 10=0")
        add("SharedLinear", p + "out", [p + "a_v", p + "a_t"], [p + "o_v", p + "o_t"],
            f"0={HIDDEN} 1={HIDDEN} 2=1")
        add("DiTAdaOutIn", p + "ada_out_in",
            [rv1, rt1, p + "o_v", p + "o_t", mods[2][b], mods[3][b], mods[4][b]],
            [p + "r_v", p + "r_t", p + "m_v", p + "m_t"], f"0={HIDDEN} 1=1.000000e-05 2={sv}")
        add("SharedLinear", p + "up", [p + "m_v", p + "m_t"], [p + "u_v", p + "u_t"],
            f"0={MLP} 1={HIDDEN} 2=1")
        add("GELU", p + "gelu_v", [p + "u_v"], [p + "g_v"], "0=0")
        add("GELU", p + "gelu_t", [p + "u_t"], [p + "g_t"], "0=0")
        add("SharedLinear", p + "down", [p + "g_v", p + "g_t"], [p + "y_v", p + "y_t"],
            f"0={HIDDEN} 1={MLP} 2=1")
        last = b + 1 == blocks
        ov, ot = ("out0", "out1") if last else (p + "out_v", p + "out_t")
        add("DiTAdaOut", p + "ada_out", [p + "r_v", p + "r_t", p + "y_v", p + "y_t", mods[5][b]],
            [ov, ot], f"0={HIDDEN} 2={sv}")
        rv, rt = ov, ot
    blobs = set()
    for line in layers:
        f = line.split()
        nb, nt = int(f[2]), int(f[3])
        blobs.update(f[4 + nb:4 + nb + nt])
    return "7767517\n" + f"{len(layers)} {len(blobs)}\n" + "\n".join(layers) + "\n"


BUILTIN_PARAM_PATH = os.path.join(HERE, "dit_blocks_2_builtin.param")


def _with_splits(layers, first_free):
    """Inserts a Split after the producer of every blob read more than once
    (tops blob_s0, blob_s1, ... handed to the consumers in order), as ncnn
    exports write them."""
    uses = {}
    for _, _, bottoms, _, _ in layers:
        for b in bottoms:
            uses[b] = uses.get(b, 0) + 1
    taken = {}
    out = []
    for type_, name, bottoms, tops, params in layers:
        nb = []
        for b in bottoms:
            if uses[b] > 1:
                i = taken.get(b, 0)
                taken[b] = i + 1
                nb.append(f"{b}_s{i}")
            else:
                nb.append(b)
        out.append((type_, name, nb, tops, params))
        for t in tops:
            if uses.get(t, 0) > 1:
                out.append(("Split", f"split_{t}", [t], [f"{t}_s{i}" for i in range(uses[t])], ""))
    return out


def builtin_layers(blocks=BLOCKS):
    """The same blocks written with ncnn built-ins in place of DiTAdaIn,
    DiTAdaOut and DiTAdaOutIn: RMSNorm (block 0 as UnaryOp square ->
    Reduction mean -> BinaryOp add eps -> UnaryOp rsqrt -> BinaryOp mul,
    odd blocks as an RMSNorm layer without affine), the modulation as
    BinaryOp mul / add with the per-sample inputs (plus MemoryData vectors
    of the block's own, odd blocks), the gated residual as BinaryOp mul /
    add.  Per stream, as the exported graph keeps the streams apart."""
    L = []

    def add(type_, name, bottoms, tops, params=""):
        L.append((type_, name, list(bottoms), list(tops), params))

    for i in range(10):
        add("Input", f"in{i}", [], [f"in{i}"])
    rv, rt = "in0", "in1"
    for b in range(blocks):
        p = f"b{b}_"
        own = b % 2 == 1

        def mod(inp, vec_name):
            """in_k, or in_k + the block's MemoryData vector."""
            if not own:
                return inp
            add("MemoryData", p + vec_name, [], [p + vec_name], f"0={HIDDEN}")
            add("BinaryOp", p + vec_name + "_add", [inp, p + vec_name], [p + vec_name + "_sum"], "0=0")
            return p + vec_name + "_sum"

        def norm(x, tag):
            if b == 0:
                add("UnaryOp", p + tag + "_sq", [x], [p + tag + "_sq"], "0=4")
                add("Reduction", p + tag + "_ms", [p + tag + "_sq"], [p + tag + "_ms"],
                    "0=3 1=0 -23303=1,-1 4=1 5=1")
                add("BinaryOp", p + tag + "_eps", [p + tag + "_ms"], [p + tag + "_mse"],
                    "0=0 1=1 2=1.000000e-05")
                add("UnaryOp", p + tag + "_rs", [p + tag + "_mse"], [p + tag + "_rs"], "0=6")
                add("BinaryOp", p + tag + "_n", [x, p + tag + "_rs"], [p + tag + "_n"], "0=2")
            else:
                add("RMSNorm", p + tag + "_n", [x], [p + tag + "_n"], f"0={HIDDEN} 1=1.000000e-05 2=0")
            return p + tag + "_n"

        def modulate(x, tag, shift_in, scale_in, shift_vec, scale_vec):
            n = norm(x, tag)
            sc = mod(scale_in, scale_vec)
            sh = mod(shift_in, shift_vec)
            add("BinaryOp", p + tag + "_scale", [n, sc], [p + tag + "_m1"], "0=2")
            add("BinaryOp", p + tag + "_shift", [p + tag + "_m1", sh], [p + tag + "_h"], "0=0")
            return p + tag + "_h"

        def gated(x, y, tag, gate_in, gate_vec, top):
            g = mod(gate_in, gate_vec)
            add("BinaryOp", p + tag + "_gate", [y, g], [p + tag + "_g"], "0=2")
            add("BinaryOp", p + tag + "_res", [x, p + tag + "_g"], [top], "0=0")
            return top

        h_v = modulate(rv, "an_v", "in4", "in5", "vshift", "vscale")
        h_t = modulate(rt, "an_t", "in4", "in5", "tshift", "tscale")
        add("SharedLinear", p + "qkv", [h_v, h_t], [p + "qkv_v", p + "qkv_t"], f"0={3 * HIDDEN} 1={HIDDEN} 2=1")
        add("AdaptiveWindowAttention", p + "attn", [p + "qkv_v", p + "qkv_t", "in2", "in3"],
            [p + "a_v", p + "a_t"],
            f"0={HEADS} 1={HEAD_DIM} 2={TARGET[0]} 3={TARGET[1]} 4={TARGET[2]} 5={b % 2} "
            f"6=1.000000e-05 7={PAIRS} 8=0 9=0 10=0")
        add("SharedLinear", p + "out", [p + "a_v", p + "a_t"], [p + "o_v", p + "o_t"], f"0={HIDDEN} 1={HIDDEN} 2=1")
        r_v = gated(rv, p + "o_v", "ag_v", "in6", "vgate", p + "r_v")
        r_t = gated(rt, p + "o_t", "ag_t", "in6", "tgate", p + "r_t")
        m_v = modulate(r_v, "mn_v", "in7", "in8", "m_vshift", "m_vscale")
        m_t = modulate(r_t, "mn_t", "in7", "in8", "m_tshift", "m_tscale")
        add("SharedLinear", p + "up", [m_v, m_t], [p + "u_v", p + "u_t"], f"0={MLP} 1={HIDDEN} 2=1")
        add("GELU", p + "gelu_v", [p + "u_v"], [p + "g_v"], "0=0")
        add("GELU", p + "gelu_t", [p + "u_t"], [p + "g_t"], "0=0")
        add("SharedLinear", p + "down", [p + "g_v", p + "g_t"], [p + "y_v", p + "y_t"], f"0={HIDDEN} 1={MLP} 2=1")
        last = b + 1 == blocks
        ov, ot = ("out0", "out1") if last else (p + "out_v", p + "out_t")
        rv = gated(r_v, p + "y_v", "mg_v", "in9", "m_vgate", ov)
        rt = gated(r_t, p + "y_t", "mg_t", "in9", "m_tgate", ot)
    return _with_splits(L, 0)


def builtin_param_text(blocks=BLOCKS):
    layers = builtin_layers(blocks)
    lines = []
    blobs = set()
    for type_, name, bottoms, tops, params in layers:
        line = f"{type_:<24} {name:<16} {len(bottoms)} {len(tops)} " + " ".join(bottoms + tops)
        lines.append(line + (" " + params if params else ""))
        blobs.update(tops)
    return "7767517\n" + f"{len(lines)} {len(blobs)}\n" + "\n".join(lines) + "\n"


def builtin_model_bytes(weights, blocks=BLOCKS):
    """The .bin of builtin_param_text: each layer's weights in layer order
    (SharedLinear and attention as in model_bytes, MemoryData raw fp32)."""
    parts = []
    for type_, name, _, _, _ in builtin_layers(blocks):
        b = int(name[1:name.index("_")]) if name.startswith("b") and name[1].isdigit() else None
        if b is None:
            continue
        w = weights[b]
        key = name[name.index("_") + 1:]
        if type_ == "MemoryData":
            parts.append(w["stream"][key])
        elif type_ == "SharedLinear":
            k = {"qkv": "qkv", "out": "o", "up": "up", "down": "dn"}[key]
            parts += [w[k], w["b_" + k]]
        elif type_ == "AdaptiveWindowAttention":
            parts += [w["norms"][0], w["norms"][1], w["norms"][2], w["norms"][3], w["freqs"]]
    return b"".join(np.ascontiguousarray(p, dtype="<f4").tobytes() for p in parts)


V3_PARAM_PATH = os.path.join(HERE, "dit_blocks_2_v3.param")
V3_MLP = 384   # SwiGLU width: whole 128-column blocks, not a multiple of 256


def v3_block_weights(blocks=BLOCKS, seed=SEED + 3):
    """Weights of the v3-shaped blocks (seedvr2_pipeline.cpp:434-438): q, k
    and v projections of their own and a SwiGLU MLP (gate, up, down)."""
    g = np.random.default_rng(seed)
    out = []
    for b in range(blocks):
        w = {}
        for name, n, k in (("q", HIDDEN, HIDDEN), ("k", HIDDEN, HIDDEN), ("v", HIDDEN, HIDDEN),
                           ("o", HIDDEN, HIDDEN), ("gate", V3_MLP, HIDDEN), ("up", V3_MLP, HIDDEN),
                           ("dn", HIDDEN, V3_MLP)):
            w[name] = _bf16(0.02 * g.standard_normal((n, k)))
            w["b_" + name] = (0.02 * g.standard_normal(n)).astype(np.float32)
        w["norms"] = (1.0 + 0.02 * g.standard_normal((4, HEAD_DIM))).astype(np.float32)
        w["freqs"] = (10000.0 ** (-np.arange(PAIRS, dtype=np.float64) / PAIRS)).astype(np.float32)
        w["stream"] = None
        if b % 2 == 1:
            w["stream"] = {k: (0.05 * g.standard_normal(HIDDEN)).astype(np.float32)
                           for k in ("vshift", "vscale", "tshift", "tscale", "vgate", "tgate",
                                     "m_vshift", "m_vscale", "m_tshift", "m_tscale",
                                     "m_vgate", "m_tgate")}
        out.append(w)
    return out


def v3_layers(blocks=BLOCKS):
    """The v3 graph form: split q / k / v SharedLinear layers feeding the
    attention's 8-input form (adaptive_window_attention.cpp:783-797), and a
    SwiGLU MLP written as gate and up SharedLinear layers, Swish on the gate
    and a BinaryOp mul per stream; the norm / modulation layers as in
    param_text."""
    L = []

    def add(type_, name, bottoms, tops, params=""):
        L.append((type_, name, list(bottoms), list(tops), params))

    for i in range(10):
        add("Input", f"in{i}", [], [f"in{i}"])
    rv, rt = "in0", "in1"
    for b in range(blocks):
        p = f"b{b}_"
        sv = 1 if b % 2 == 1 else 0
        add("DiTAdaIn", p + "ada_in", [rv, rt, "in4", "in5"], [p + "h_v", p + "h_t"],
            f"0={HIDDEN} 1=1.000000e-05 2={sv}")
        for part in ("q", "k", "v"):
            add("SharedLinear", p + part, [p + "h_v", p + "h_t"], [p + part + "_v", p + part + "_t"],
                f"0={HIDDEN} 1={HIDDEN} 2=1")
        add("AdaptiveWindowAttention", p + "attn",
            [p + "q_v", p + "k_v", p + "v_v", p + "q_t", p + "k_t", p + "v_t", "in2", "in3"],
            [p + "a_v", p + "a_t"],
            f"0={HEADS} 1={HEAD_DIM} 2={TARGET[0]} 3={TARGET[1]} 4={TARGET[2]} 5={b % 2} "
            f"6=1.000000e-05 7={PAIRS} 8=0 9=0 10=0")
        add("SharedLinear", p + "out", [p + "a_v", p + "a_t"], [p + "o_v", p + "o_t"], f"0={HIDDEN} 1={HIDDEN} 2=1")
        add("DiTAdaOutIn", p + "ada_out_in", [rv, rt, p + "o_v", p + "o_t", "in6", "in7", "in8"],
            [p + "r_v", p + "r_t", p + "m_v", p + "m_t"], f"0={HIDDEN} 1=1.000000e-05 2={sv}")
        add("SharedLinear", p + "gate", [p + "m_v", p + "m_t"], [p + "gt_v", p + "gt_t"], f"0={V3_MLP} 1={HIDDEN} 2=1")
        add("SharedLinear", p + "up", [p + "m_v", p + "m_t"], [p + "u_v", p + "u_t"], f"0={V3_MLP} 1={HIDDEN} 2=1")
        for s_ in ("v", "t"):
            add("Swish", p + "silu_" + s_, [p + "gt_" + s_], [p + "sg_" + s_])
            add("BinaryOp", p + "glu_" + s_, [p + "sg_" + s_, p + "u_" + s_], [p + "gu_" + s_], "0=2")
        add("SharedLinear", p + "down", [p + "gu_v", p + "gu_t"], [p + "y_v", p + "y_t"], f"0={HIDDEN} 1={V3_MLP} 2=1")
        last = b + 1 == blocks
        ov, ot = ("out0", "out1") if last else (p + "out_v", p + "out_t")
        add("DiTAdaOut", p + "ada_out", [p + "r_v", p + "r_t", p + "y_v", p + "y_t", "in9"], [ov, ot],
            f"0={HIDDEN} 2={sv}")
        rv, rt = ov, ot
    return _with_splits(L, 0)


def v3_param_text(blocks=BLOCKS):
    lines = []
    blobs = set()
    for type_, name, bottoms, tops, params in v3_layers(blocks):
        line = f"{type_:<24} {name:<16} {len(bottoms)} {len(tops)} " + " ".join(bottoms + tops)
        lines.append(line + (" " + params if params else ""))
        blobs.update(tops)
    return "7767517\n" + f"{len(lines)} {len(blobs)}\n" + "\n".join(lines) + "\n"


def v3_model_bytes(weights):
    parts = []
    for w in weights:
        s = w["stream"]
        if s is not None:
            parts += [s["vshift"], s["vscale"], s["tshift"], s["tscale"]]
        for k in ("q", "k", "v"):
            parts += [w[k], w["b_" + k]]
        parts += [w["norms"][0], w["norms"][1], w["norms"][2], w["norms"][3], w["freqs"]]
        parts += [w["o"], w["b_o"]]
        if s is not None:
            parts += [s["vgate"], s["tgate"], s["m_vshift"], s["m_vscale"], s["m_tshift"], s["m_tscale"]]
        parts += [w["gate"], w["b_gate"], w["up"], w["b_up"], w["dn"], w["b_dn"]]
        if s is not None:
            parts += [s["m_vgate"], s["m_tgate"]]
    return b"".join(np.ascontiguousarray(p, dtype="<f4").tobytes() for p in parts)


def model_bytes(weights):
    """The .bin: each layer's load_model data in layer order, raw fp32 (the
    type-1 loads of SharedLinear, AdaptiveWindowAttention and the block ops)."""
    parts = []
    for b, w in enumerate(weights):
        s = w["stream"]
        if s is not None:   # DiTAdaIn: video_shift, video_scale, text_shift, text_scale
            parts += [s["vshift"], s["vscale"], s["tshift"], s["tscale"]]
        parts += [w["qkv"], w["b_qkv"]]
        parts += [w["norms"][0], w["norms"][1], w["norms"][2], w["norms"][3], w["freqs"]]
        parts += [w["o"], w["b_o"]]
        if s is not None:   # DiTAdaOutIn: gates, then the MLP's shift/scale vectors
            parts += [s["vgate"], s["tgate"], s["m_vshift"], s["m_vscale"], s["m_tshift"], s["m_tscale"]]
        parts += [w["up"], w["b_up"], w["dn"], w["b_dn"]]
        if s is not None:   # DiTAdaOut: the MLP's gates
            parts += [s["m_vgate"], s["m_tgate"]]
    return b"".join(np.ascontiguousarray(p, dtype="<f4").tobytes() for p in parts)


if __name__ == "__main__":
    with open(PARAM_PATH, "w") as f:
        f.write(param_text())
    with open(BUILTIN_PARAM_PATH, "w") as f:
        f.write(builtin_param_text())
    with open(V3_PARAM_PATH, "w") as f:
        f.write(v3_param_text())
    print("wrote", PARAM_PATH, BUILTIN_PARAM_PATH, V3_PARAM_PATH)
