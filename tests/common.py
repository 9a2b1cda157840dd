"""Shared helpers of the test suite: seeded inputs, parity metrics, and the
ctypes binding of the layer harness (tests/harness/layer_harness.cpp)."""
from __future__ import annotations

import ctypes
import os

import numpy as np

TESTS = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(TESTS)
HARNESS_PATH = os.path.join(TESTS, "harness", "liblayer_harness.so")

# Parity bar for floating point outputs: fp32 accumulation on the device,
# compared with the fp32 CPU oracle.
MAX_ABS_TOL = 2e-2
COSINE_TOL = 0.9999


def bf16_round(a) -> np.ndarray:
    """Round-to-nearest-even to bfloat16, returned as float32 (finite inputs)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    bits = a.view(np.uint32).astype(np.uint64)
    bits = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
    return bits.astype(np.uint32).view(np.float32).reshape(a.shape)


def metrics(got, ref):
    g = np.asarray(got, dtype=np.float64).ravel()
    r = np.asarray(ref, dtype=np.float64).ravel()
    max_abs = float(np.max(np.abs(g - r))) if g.size else 0.0
    denom = np.linalg.norm(g) * np.linalg.norm(r)
    cos = float(np.dot(g, r) / denom) if denom > 0 else 1.0
    return max_abs, cos


def assert_close(got, ref, what="", max_abs=MAX_ABS_TOL, cosine=COSINE_TOL):
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    ma, cs = metrics(got, ref)
    assert ma <= max_abs and cs >= cosine, f"{what}: max_abs={ma:.3e} cosine={cs:.7f}"
    return ma, cs


def rope_freqs(pairs):
    """rope_freqs[p] = 10000^(-p/P): this build's choice for the synthetic
    weights (the exported model's values are not available)."""
    if pairs == 0:
        return np.zeros(0, np.float32)
    return (10000.0 ** (-np.arange(pairs, dtype=np.float64) / pairs)).astype(np.float32)


def make_awa_inputs(seed, video_shapes, text_lengths, heads, head_dim, pairs, bf16=False,
                    peaky=True, shared_norm=False, fp16=False):
    """Seeded synthetic inputs of the layer: fused video_qkv [Lv, 3*inner] and
    text_qkv [Lt, 3*inner] ~ N(0,1); norm weights N(0,0.02) ("literal") or
    1+N(0,0.02) ("peaky", which makes the softmax far from uniform).  With
    bf16=True (fp16=True) the activations are rounded to bf16 (fp16) and the
    oracle consumes the same rounded values."""
    g = np.random.default_rng(seed)
    inner = heads * head_dim
    lv = int(sum(t * h * w for t, h, w in video_shapes))
    lt = int(sum(text_lengths))
    video = g.standard_normal((lv, 3 * inner), dtype=np.float32)
    text = g.standard_normal((lt, 3 * inner), dtype=np.float32)
    if bf16:
        video, text = bf16_round(video), bf16_round(text)
    if fp16:
        video = video.astype(np.float16).astype(np.float32)
        text = text.astype(np.float16).astype(np.float32)
    base = 1.0 if peaky else 0.0
    norms = (base + 0.02 * g.standard_normal((4, head_dim))).astype(np.float32)
    if shared_norm:
        norms[2], norms[3] = norms[0], norms[1]
    return dict(video=video, text=text, norms=norms, freqs=rope_freqs(pairs))


def oracle_awa(case, heads, head_dim, target, shifted, eps, pairs, video_shapes, text_lengths,
               official_bf16=False, window_subset=None, threads=None, fast=False):
    import oracle
    inner = heads * head_dim
    p = oracle.awa_params(heads, head_dim, target, shifted, eps, pairs, official_bf16)
    v, t, n = case["video"], case["text"], case["norms"]
    if threads is None:
        threads = min(16, os.cpu_count() or 1)
    return oracle.awa_forward(p, n[0], n[1], n[2], n[3], case["freqs"], video_shapes, text_lengths,
                              v[:, :inner], v[:, inner:2 * inner], v[:, 2 * inner:],
                              t[:, :inner], t[:, inner:2 * inner], t[:, 2 * inner:],
                              window_subset=window_subset, threads=threads, fast=fast)


# ---------------------------------------------------------------------------
# Layer harness binding

class HBlob(ctypes.Structure):
    _fields_ = [("dims", ctypes.c_int), ("w", ctypes.c_int), ("h", ctypes.c_int),
                ("elemsize", ctypes.c_int), ("device", ctypes.c_int), ("data", ctypes.c_void_p)]


_H = None


class HBlob4(ctypes.Structure):
    _fields_ = [("w", ctypes.c_int), ("h", ctypes.c_int), ("d", ctypes.c_int), ("c", ctypes.c_int),
                ("cstep", ctypes.c_long), ("elemsize", ctypes.c_int), ("device", ctypes.c_int),
                ("data", ctypes.c_void_p)]


def ncnn_cstep(w, h, d, elemsize):
    """ncnn's channel stride of a 4-D Mat: a channel rounded up to 16 bytes."""
    return ((w * h * d * elemsize + 15) // 16 * 16) // elemsize


def harness():
    global _H
    if _H is None:
        if not os.path.exists(HARNESS_PATH):
            import subprocess
            subprocess.run(["make", "-s", "-C", os.path.dirname(HARNESS_PATH)], check=True)
        L = ctypes.CDLL(HARNESS_PATH)
        P, vp, ci, cf = ctypes.POINTER, ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        L.h_layer_create.argtypes = [ctypes.c_char_p, ctypes.c_char_p, vp, ctypes.c_long, P(vp)]
        L.h_layer_create_pipeline.argtypes = [vp]
        L.h_layer_destroy.argtypes = [vp]
        L.h_awa_set_state.argtypes = [vp, P(ci), P(ci), ci]
        L.h_awa_configure_and_set_weights.argtypes = [vp, ci, ci, P(ci), ci, cf, ci, ci, ci,
                                                      P(cf), P(cf), P(cf), P(cf), P(cf)]
        L.h_layer_forward.argtypes = [vp, ci, P(HBlob), ci, P(HBlob)]
        L.h_layer_set_storage.argtypes = [vp, ci, ci]
        L.h_build_plan.argtypes = [P(ci), ci, P(ci), ci, ci, P(ci), P(ci), P(ci), P(ci), P(ci), P(ci)]
        L.h_set_vae_memory_state.argtypes = [ci]
        L.h_conv_memory.argtypes = [vp, ci]
        L.h_layer_forward4.argtypes = [vp, P(HBlob4), P(HBlob4)]
        L.h_layer_forward1.argtypes = [vp, P(HBlob), P(HBlob)]
        _H = L
    return _H


def _ip(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int))


def _fp(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


class Layer:
    """An ncnn-surface layer created through its creator, load_param (from a
    .param field string) and load_model (from raw fp32 weight bytes)."""

    def __init__(self, type_name, params, weights=None):
        self._keep = None
        data, nbytes = None, 0
        if weights is not None:
            self._keep = np.ascontiguousarray(np.concatenate([np.ravel(w) for w in weights]),
                                              dtype=np.float32)
            data, nbytes = self._keep.ctypes.data, self._keep.nbytes
        self.h = ctypes.c_void_p()
        self.create_code = harness().h_layer_create(type_name.encode(), params.encode(), data,
                                                    nbytes, ctypes.byref(self.h))

    def create_pipeline(self):
        return harness().h_layer_create_pipeline(self.h)

    def set_storage(self, fp16, bf16):
        """ncnn Option use_fp16_storage / use_bf16_storage for forward."""
        harness().h_layer_set_storage(self.h, int(bool(fp16)), int(bool(bf16)))

    def forward_planar(self, x, dims, out_dims, device=False, dtype=None):
        """One-blob forward over 4-D blobs.  x: numpy [c, d, h, w] (fp32
        values); dims = (w, h, d, c); out_dims = (w, h, d, c) expected.  With
        device=True the blob is a device Mat of the given torch dtype
        (elemsize 4 or 2).  Returns (code, numpy [c, d, h, w] fp32)."""
        import torch
        w, h, d, c = dims
        es = 4 if dtype in (None, torch.float32) else 2
        cs = ncnn_cstep(w, h, d, es)
        flat = np.zeros((c, cs), np.float32)
        flat[:, :w * h * d] = np.asarray(x, np.float32).reshape(c, -1)
        ow, oh, od, oc = out_dims
        ocs = ncnn_cstep(ow, oh, od, es)
        bi, bo = HBlob4(), HBlob4()
        bi.w, bi.h, bi.d, bi.c, bi.cstep, bi.elemsize = w, h, d, c, cs, es
        bo.w, bo.h, bo.d, bo.c, bo.cstep, bo.elemsize = ow, oh, od, oc, ocs, es
        if device:
            tin = torch.from_numpy(flat).cuda().to(dtype or torch.float32)
            tout = torch.zeros((oc, ocs), dtype=dtype or torch.float32, device="cuda")
            bi.device = bo.device = 1
            bi.data, bo.data = tin.data_ptr(), tout.data_ptr()
        else:
            hout = np.zeros((oc, ocs), np.float32)
            bi.device = bo.device = 0
            bi.data, bo.data = flat.ctypes.data, hout.ctypes.data
        code = harness().h_layer_forward4(self.h, ctypes.byref(bi), ctypes.byref(bo))
        if code != 0:
            return code, None
        res = tout.float().cpu().numpy() if device else hout
        assert (bo.w, bo.h, bo.d, bo.c) == (ow, oh, od, oc)
        return 0, res[:, :ow * oh * od].reshape(oc, od, oh, ow)

    def forward_rows(self, x, out_w, device=False, dtype=None):
        """One-blob forward over a 2-D blob x [h][w] (numpy fp32 values); with
        device=True a device Mat of the given torch dtype.  Returns (code,
        numpy [h][out_w] fp32)."""
        import torch
        h, w = x.shape
        es = 4 if dtype in (None, torch.float32) else 2
        bi, bo = HBlob(), HBlob()
        bi.dims, bi.w, bi.h, bi.elemsize = 2, w, h, es
        bo.dims, bo.w, bo.h, bo.elemsize = 2, out_w, h, es
        if device:
            tin = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda().to(dtype or torch.float32)
            tout = torch.zeros((h, out_w), dtype=dtype or torch.float32, device="cuda")
            bi.device = bo.device = 1
            bi.data, bo.data = tin.data_ptr(), tout.data_ptr()
        else:
            xin = np.ascontiguousarray(x, np.float32)
            hout = np.zeros((h, out_w), np.float32)
            bi.device = bo.device = 0
            bi.data, bo.data = xin.ctypes.data, hout.ctypes.data
        code = harness().h_layer_forward1(self.h, ctypes.byref(bi), ctypes.byref(bo))
        if code != 0:
            return code, None
        return 0, (tout.float().cpu().numpy() if device else hout)

    def conv_memory(self, reset):
        return harness().h_conv_memory(self.h, int(bool(reset)))

    def set_state(self, video_shapes, text_lengths):
        s = np.ascontiguousarray(np.asarray(video_shapes, np.int32).ravel())
        t = np.ascontiguousarray(np.asarray(text_lengths, np.int32))
        harness().h_awa_set_state(self.h, _ip(s), _ip(t), len(t))

    def forward(self, inputs, out_shapes, device_out=False):
        """inputs: list of numpy arrays (host blobs), torch device tensors
        (device blobs) or None (empty blob).  Returns (code, outputs)."""
        ins = (HBlob * len(inputs))()
        keep = []
        for i, x in enumerate(inputs):
            b = ins[i]
            if x is None:
                b.dims = 0
                continue
            if hasattr(x, "data_ptr"):   # torch device tensor
                b.device = 1
                b.data = x.data_ptr()
                b.elemsize = x.element_size()
                shape = tuple(x.shape)
            else:
                x = np.ascontiguousarray(x)
                keep.append(x)
                b.device = 0
                b.data = x.ctypes.data
                b.elemsize = x.itemsize
                shape = x.shape
            b.dims = len(shape)
            b.w = shape[-1]
            b.h = shape[0] if len(shape) == 2 else 1
        outs = (HBlob * len(out_shapes))()
        results = []
        for i, (shape, dtype) in enumerate(out_shapes):
            if device_out:
                import torch
                t = torch.zeros(shape, dtype=dtype, device="cuda")
                results.append(t)
                outs[i].data = t.data_ptr()
                outs[i].device = 1
                outs[i].elemsize = t.element_size()
            else:
                a = np.zeros(shape, dtype=dtype)
                results.append(a)
                outs[i].data = a.ctypes.data
                outs[i].elemsize = a.itemsize
            outs[i].w, outs[i].h = shape[1], shape[0]
        code = harness().h_layer_forward(self.h, len(inputs), ins, len(out_shapes), outs)
        return code, results

    def close(self):
        if self.h:
            harness().h_layer_destroy(self.h)
            self.h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def awa_param_string(heads, head_dim, target, shifted, eps, pairs, shared_norm=False,
                     int32_shapes=False, official_bf16=False):
    return (f"0={heads} 1={head_dim} 2={target[0]} 3={target[1]} 4={target[2]} "
            f"5={int(bool(shifted))} 6={eps:e} 7={pairs} 8={int(bool(shared_norm))} "
            f"9={int(bool(int32_shapes))} 10={int(bool(official_bf16))}")


def harness_plan(video_shapes, target, shifted):
    """seedvr2::build_adaptive_window_plan through the harness."""
    shapes = np.ascontiguousarray(np.asarray(video_shapes, np.int32).ravel())
    batch = len(shapes) // 3
    lv = int(sum(int(t) * int(h) * int(w) for t, h, w in np.asarray(video_shapes).reshape(-1, 3)))
    maxw = 4096
    n = ctypes.c_int()
    wins = np.zeros(maxw * 9, np.int32)
    counts = np.zeros(batch, np.int32)
    idx = np.zeros(lv, np.int32)
    inv = np.zeros(lv, np.int32)
    pos = np.zeros(lv * 3, np.int32)
    tgt = np.asarray(target, np.int32)
    code = harness().h_build_plan(_ip(shapes), batch, _ip(tgt), int(bool(shifted)), maxw,
                                  ctypes.byref(n), _ip(wins), _ip(counts), _ip(idx), _ip(inv), _ip(pos))
    if code != 0:
        raise ValueError(code)
    return wins[:9 * n.value].reshape(-1, 9), counts, idx, inv, pos.reshape(-1, 3)


def set_vae_memory_state(state):
    """seedvr2::set_vae_memory_state: 0 DISABLED, 1 INITIALIZING, 2 ACTIVE."""
    harness().h_set_vae_memory_state(int(state))
