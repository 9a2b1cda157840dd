"""Builds small ncnn .param graphs of built-in layers and runs them through
ncnn::Net (tests/harness h_net_run), on the host or on device blobs."""
from __future__ import annotations

import ctypes

import numpy as np

from common import HBlob, harness


def param(layers):
    """layers: (type, name, bottoms, tops, params) tuples -> .param text."""
    blobs = set()
    lines = []
    for type_, name, bottoms, tops, params in layers:
        blobs.update(tops)
        lines.append(f"{type_} {name} {len(bottoms)} {len(tops)} " + " ".join(bottoms + tops) +
                     (" " + params if params else ""))
    return "7767517\n" + f"{len(lines)} {len(blobs)}\n" + "\n".join(lines) + "\n"


def fp32(*arrays):
    """Raw fp32 weight bytes (ModelBin type 1)."""
    return b"".join(np.ascontiguousarray(a, "<f4").tobytes() for a in arrays)


def tagged(*arrays, fp16=False):
    """ModelBin type 0 weights: a 4-byte tag each, then fp32 or fp16 data
    (padded to 4 bytes)."""
    out = b""
    for a in arrays:
        if fp16:
            raw = np.ascontiguousarray(a, "<f2").tobytes()
            out += np.uint32(0x01306B47).tobytes() + raw + b"\0" * (-len(raw) % 4)
        else:
            out += np.uint32(0).tobytes() + np.ascontiguousarray(a, "<f4").tobytes()
    return out


def _lib():
    L = harness()
    P = ctypes.POINTER
    L.h_net_run.argtypes = [ctypes.c_char_p, ctypes.c_void_p, ctypes.c_long, ctypes.c_int, ctypes.c_int,
                            P(ctypes.c_char_p), P(HBlob), ctypes.c_int, P(ctypes.c_char_p), P(HBlob)]
    return L


def run(text, model, inputs, outputs, device=False):
    """inputs: {name: numpy fp32 (host) or torch tensor (device)}; outputs:
    {name: max element count}.  Returns (code, {name: numpy fp32 array of the
    blob's shape})."""
    names_in = list(inputs)
    ins = (HBlob * max(1, len(names_in)))()
    keep = []
    for i, n in enumerate(names_in):
        t = inputs[n]
        if isinstance(t, np.ndarray):
            a = np.ascontiguousarray(t, np.float32)
            keep.append(a)
            ins[i] = HBlob(a.ndim, a.shape[-1], a.shape[0] if a.ndim == 2 else 1, 4, 0, a.ctypes.data)
        else:
            ins[i] = HBlob(t.dim(), t.shape[-1], t.shape[0] if t.dim() == 2 else 1, t.element_size(), 1,
                           t.data_ptr())
    names_out = list(outputs)
    bufs = [np.zeros(outputs[n] + 8, np.float32) for n in names_out]
    outs = (HBlob * max(1, len(names_out)))()
    for i, b in enumerate(bufs):
        outs[i] = HBlob(1, b.size, 1, 4, 0, b.ctypes.data)
    model_buf = ctypes.create_string_buffer(model, max(1, len(model)))
    cin = (ctypes.c_char_p * max(1, len(names_in)))(*[n.encode() for n in names_in])
    cout = (ctypes.c_char_p * max(1, len(names_out)))(*[n.encode() for n in names_out])
    ret = _lib().h_net_run(text.encode(), model_buf, len(model), int(device), len(names_in), cin, ins,
                           len(names_out), cout, outs)
    res = {}
    if ret == 0:
        for i, n in enumerate(names_out):
            o = outs[i]
            count = o.w * o.h
            if o.elemsize == 4:
                a = bufs[i][:count].copy()
            else:   # 16-bit device blobs of this net are bf16 (no fp16 storage option)
                raw = bufs[i].view(np.uint16)[:count]
                a = (raw.astype(np.uint32) << 16).view(np.float32)
            res[n] = a.reshape((o.h, o.w) if o.dims == 2 else (o.w,))
    return ret, res
