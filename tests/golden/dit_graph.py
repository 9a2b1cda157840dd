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

Usage: python tests/golden/dit_graph.py  rewrites dit_blocks_2.param here.
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
    print("wrote", PARAM_PATH)
