"""ctypes wrapper of the CPU oracle (oracle.c) -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the reference result or the timed CPU baseline.  The product
path (seedvr2_ncnn_amd) never imports it.

The C code restates the reference CPU forward of AdaptiveWindowAttention
(src/seedvr2/adaptive_window_attention.cpp:434-655, 764-978) and of
SharedLinear (src/seedvr2/shared_linear.cpp:83-96); see oracle.h.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIBS: dict = {}


class Conv3dConfig(ctypes.Structure):
    """The 16 DecomposedConv3D configuration values (decomposed_conv3d.cpp:422-441)."""
    _fields_ = [(n, ctypes.c_int) for n in (
        "num_output", "num_input", "kernel_w", "kernel_h", "kernel_t", "stride_t", "dilation_t",
        "head_frames", "stride_w", "stride_h", "dilation_w", "dilation_h", "pad_w", "pad_h",
        "groups", "bias_term")]


def conv3d_config(**kw):
    c = Conv3dConfig()
    defaults = dict(stride_t=1, dilation_t=1, head_frames=0, stride_w=1, stride_h=1,
                    dilation_w=1, dilation_h=1, pad_w=0, pad_h=0, groups=1, bias_term=0)
    defaults.update(kw)
    for name, _ in Conv3dConfig._fields_:
        setattr(c, name, int(defaults[name]))
    return c


class Slice(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "sample_index", "t0", "t1", "h0", "h1", "w0", "w1",
        "partition_offset", "token_count")]


class AwaParams(ctypes.Structure):
    _fields_ = [
        ("heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("target_windows", ctypes.c_int * 3),
        ("shifted", ctypes.c_int),
        ("epsilon", ctypes.c_float),
        ("rope_pairs_per_axis", ctypes.c_int),
        ("official_bf16_attention", ctypes.c_int),
    ]


def build() -> None:
    """Compile liboracle.so / liboracle_fast.so with the committed Makefile."""
    import subprocess
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib(fast: bool = False) -> ctypes.CDLL:
    name = "liboracle_fast.so" if fast else "liboracle.so"
    if name not in _LIBS:
        path = os.path.join(_HERE, name)
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        P = ctypes.POINTER
        ci, cf = ctypes.c_int, ctypes.c_float
        L.orc_plan_count.argtypes = [P(ci), ci, P(ci), ci, P(ci), P(ci)]
        L.orc_plan_build.argtypes = [P(ci), ci, P(ci), ci, P(Slice), ci, P(ci), P(ci),
                                     P(ci), P(ci)]
        L.orc_round_bf16.argtypes = [cf]
        L.orc_round_bf16.restype = cf
        L.orc_round_bf16_array.argtypes = [P(cf), P(cf), ctypes.c_long]
        L.orc_rms_norm.argtypes = [P(cf), P(cf), ci, cf, P(cf)]
        L.orc_apply_mm_rope.argtypes = [P(cf), ci, P(cf), ci, P(ci)]
        L.orc_sdpa.argtypes = [P(cf), P(cf), P(cf), ci, ci, ci, P(cf), ci]
        L.orc_awa_forward.argtypes = [P(AwaParams), P(cf), P(cf), P(cf), P(cf), P(cf),
                                      P(ci), P(ci), ci,
                                      P(cf), P(cf), P(cf), ctypes.c_long,
                                      P(cf), P(cf), P(cf), ctypes.c_long,
                                      P(cf), P(cf), P(ci), ci, ci]
        L.orc_linear.argtypes = [P(cf), ci, ci, P(cf), P(cf), ci, ci, P(cf), P(ci), ci, ci]
        cl = ctypes.c_long
        L.orc_patchify_video.argtypes = [P(cf), cl, P(ci), ci, P(cf)]
        L.orc_timestep_embedding.argtypes = [P(cf), ci, P(cf)]
        L.orc_unpatchify_prediction.argtypes = [P(cf), cl, P(ci), ci, P(cf)]
        L.orc_apply_cfg.argtypes = [P(cf), P(cf), cl, cf, cf, P(cf)]
        L.orc_euler_step.argtypes = [P(cf), cl, P(cf), cl, cf]
        L.orc_video_tokens.argtypes = [P(cf), P(cf), cl, cl, P(cf)]
        L.orc_ada_in.argtypes = [P(cf), ci, cf, P(ci), ci, P(cf), P(cf), P(cf), P(cf), P(cf)]
        L.orc_ada_out.argtypes = [P(cf), P(cf), ci, P(ci), ci, P(cf), P(cf)]
        L.orc_mha.argtypes = [P(cf), ci, ci, ci, ci, cf, P(cf), P(cf), P(cf), P(cf), P(cf), P(cf),
                              P(cf), P(cf), P(ci), ci, P(cf), ci]
        L.orc_vae_pixel_shuffle.argtypes = [P(cf), ci, ci, ci, ci, cl, ci, ci, ci, P(cf), cl]
        L.orc_decomposed_conv3d.argtypes = [P(Conv3dConfig), P(cf), ci, ci, ci, cl, P(cf), ci, cl,
                                            P(cf), P(cf), P(cf), cl, P(cf), cl, ci]
        _LIBS[name] = L
    return _LIBS[name]


def _i32(a):
    a = np.ascontiguousarray(a, dtype=np.int32)
    return a, a.ctypes.data_as(ctypes.POINTER(ctypes.c_int))


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


@dataclass
class Plan:
    """Mirror of the reference AdaptiveWindowPlan (adaptive_window_attention.h:29-36)."""
    windows: np.ndarray                # [nwin, 9] int32, WindowSlice fields in order
    sample_window_count: np.ndarray    # [batch]
    video_indices: np.ndarray          # [L]
    inverse_video_indices: np.ndarray  # [L]
    local_positions: np.ndarray        # [L, 3]


def plan(video_shapes, target_windows, shifted) -> Plan:
    L = lib()
    shapes, ps = _i32(np.asarray(video_shapes).reshape(-1, 3))
    tgt, pt = _i32(target_windows)
    batch = shapes.shape[0]
    nwin, ntok = ctypes.c_int(), ctypes.c_int()
    ret = L.orc_plan_count(ps, batch, pt, int(bool(shifted)), ctypes.byref(nwin), ctypes.byref(ntok))
    if ret != 0:
        raise ValueError(f"orc_plan_count returned {ret}")
    slices = (Slice * max(nwin.value, 1))()
    counts, pc = _i32(np.zeros(batch))
    idx, pi = _i32(np.zeros(ntok.value))
    inv, pv = _i32(np.zeros(ntok.value))
    pos, pp = _i32(np.zeros((ntok.value, 3)))
    ret = L.orc_plan_build(ps, batch, pt, int(bool(shifted)), slices, nwin.value, pc, pi, pv, pp)
    if ret != 0:
        raise ValueError(f"orc_plan_build returned {ret}")
    win = np.array([[getattr(slices[i], f) for f, _ in Slice._fields_]
                    for i in range(nwin.value)], dtype=np.int32).reshape(-1, 9)
    return Plan(win, counts, idx, inv, pos)


def round_bf16(x) -> np.ndarray:
    L = lib()
    x, px = _f32(x)
    out = np.empty_like(x)
    L.orc_round_bf16_array(px, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), x.size)
    return out


def rms_norm(x, w, eps) -> np.ndarray:
    L = lib()
    x, px = _f32(x)
    w, pw = _f32(w)
    out = np.zeros_like(x)
    _, po = _f32(out)
    po = out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    L.orc_rms_norm(px, pw, x.size, eps, po)
    return out


def apply_mm_rope(x, freqs, pairs, position) -> np.ndarray:
    L = lib()
    out = np.array(x, dtype=np.float32, copy=True)
    po = out.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    f, pf = _f32(freqs)
    pos, pp = _i32(position)
    L.orc_apply_mm_rope(po, out.size, pf, pairs, pp)
    return out


def sdpa(q, k, v, threads=1) -> np.ndarray:
    """q,k,v: [heads, seq, d] float32."""
    L = lib()
    q, pq = _f32(q)
    k, pk = _f32(k)
    v, pv = _f32(v)
    out = np.zeros_like(q)
    L.orc_sdpa(pq, pk, pv, q.shape[0], q.shape[1], q.shape[2],
               out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), threads)
    return out


def awa_params(heads, head_dim, target_windows, shifted, epsilon, rope_pairs, official_bf16):
    p = AwaParams()
    p.heads, p.head_dim = heads, head_dim
    for i in range(3):
        p.target_windows[i] = int(target_windows[i])
    p.shifted = int(bool(shifted))
    p.epsilon = float(epsilon)
    p.rope_pairs_per_axis = rope_pairs
    p.official_bf16_attention = int(bool(official_bf16))
    return p


def awa_forward(params: AwaParams, norm_vq, norm_vk, norm_tq, norm_tk, freqs,
                video_shapes, text_lengths, video_q, video_k, video_v, text_q, text_k, text_v,
                window_subset=None, threads=1, fast=False):
    """Reference-equivalent CPU forward.  video_q/k/v: [Lv, inner] float32 arrays
    (views into a fused [Lv, 3*inner] array are fine: the row stride is taken
    from the array).  Returns (out_video [Lv, inner], out_text [Lt, inner]) or
    raises ValueError with the reference return code."""
    L = lib(fast)
    inner = params.heads * params.head_dim
    shapes, ps = _i32(np.asarray(video_shapes).reshape(-1, 3))
    tl, ptl = _i32(text_lengths)

    def rows(a):
        a = np.asarray(a)
        assert a.dtype == np.float32 and a.ndim == 2 and a.strides[1] == 4
        return a, a.strides[0] // 4

    vq, vs = rows(video_q)
    vk, vs2 = rows(video_k)
    vv, vs3 = rows(video_v)
    tq, ts = rows(text_q)
    tk, ts2 = rows(text_k)
    tv, ts3 = rows(text_v)
    assert vs == vs2 == vs3 and ts == ts2 == ts3
    fp = lambda a: ctypes.cast(a.ctypes.data, ctypes.POINTER(ctypes.c_float))
    lv = int(np.prod(shapes, axis=1).sum())
    lt = int(tl.sum())
    out_v = np.zeros((lv, inner), np.float32)
    out_t = np.zeros((lt, inner), np.float32)
    ws = None
    if window_subset is not None:
        ws, pws = _i32(window_subset)
    norms = [_f32(a) for a in (norm_vq, norm_vk, norm_tq, norm_tk, freqs)]
    ret = L.orc_awa_forward(ctypes.byref(params), *[n[1] for n in norms], ps, ptl, shapes.shape[0],
                            fp(vq), fp(vk), fp(vv), vs, fp(tq), fp(tk), fp(tv), ts,
                            fp(out_v), fp(out_t),
                            pws if ws is not None else None, 0 if ws is None else len(ws),
                            threads)
    if ret != 0:
        raise ValueError(ret)
    return out_v, out_t


def linear(x, w, bias=None, activation=0, rows=None, threads=1, fast=False) -> np.ndarray:
    """Y = X W^T + b (erf-GELU when activation == 1); rows selects rows of X."""
    L = lib(fast)
    x, px = _f32(x)
    w, pw = _f32(w)
    m, k = x.shape
    n = w.shape[0]
    pb = None
    if bias is not None:
        bias, pb = _f32(bias)
    pr, nr = None, m
    if rows is not None:
        rr, pr = _i32(rows)
        nr = len(rr)
    y = np.zeros((nr, n), np.float32)
    L.orc_linear(px, m, k, pw, pb, n, activation,
                 y.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), pr, nr if rows is not None else 0,
                 threads)
    return y


# ---- DiT frontend and tail ---------------------------------------------------------

def patchify_video(source, video_shapes):
    """seedvr2_dit.cpp:167-230: [tokens][33] -> [patches][132]; (code, out)."""
    src, ps = _f32(source)
    shapes, pshp = _i32(np.asarray(video_shapes).reshape(-1, 3))
    patches = int(sum(int(t) * (int(h) // 2) * (int(w) // 2) for t, h, w in shapes))
    out = np.zeros((patches, 132), np.float32)
    code = lib().orc_patchify_video(ps, src.shape[0], pshp, shapes.shape[0],
                                    out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    return code, out


def timestep_embedding(timesteps):
    """seedvr2_dit.cpp:232-253: [count][256]."""
    ts, pt = _f32(np.asarray(timesteps, np.float32).ravel())
    out = np.zeros((ts.shape[0], 256), np.float32)
    lib().orc_timestep_embedding(pt, ts.shape[0], out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    return out


def unpatchify_prediction(source, video_shapes):
    """seedvr2_dit.cpp:255-326: [patches][64] -> [tokens][16]; (code, out)."""
    src, ps = _f32(source)
    shapes, pshp = _i32(np.asarray(video_shapes).reshape(-1, 3))
    tokens = int(sum(int(t) * int(h) * int(w) for t, h, w in shapes))
    out = np.zeros((tokens, 16), np.float32)
    code = lib().orc_unpatchify_prediction(ps, src.shape[0], pshp, shapes.shape[0],
                                           out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    return code, out


def apply_cfg(positive, negative, scale, rescale):
    """seedvr2_pipeline.cpp:171-210."""
    pos, pp = _f32(np.ravel(positive))
    neg, pn = _f32(np.ravel(negative))
    out = np.zeros_like(pos)
    lib().orc_apply_cfg(pp, pn, pos.shape[0], float(scale), float(rescale),
                        out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    return out.reshape(np.shape(positive))


def euler_step(latent, prediction, delta):
    """seedvr2_pipeline.cpp:575-588 on a copy of latent [16][stride] (the
    first tokens entries of each channel row are the tokens)."""
    lat = np.array(latent, dtype=np.float32, copy=True, order="C")
    pred, pp = _f32(prediction)
    lib().orc_euler_step(lat.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), lat.shape[1], pp,
                         pred.shape[0], float(delta))
    return lat


def video_tokens(latent, condition, tokens):
    """seedvr2_pipeline.cpp:296-317: planes [16][stride] x2 -> [tokens][33]."""
    lat, pl = _f32(latent)
    cond, pc = _f32(condition)
    assert lat.shape == cond.shape and lat.shape[0] == 16 and lat.shape[1] >= tokens
    out = np.zeros((tokens, 33), np.float32)
    lib().orc_video_tokens(pl, pc, lat.shape[1], tokens,
                           out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    return out


def _opt_vec(v, dim):
    """None -> (None, NULL); else a float32 [dim] vector and its pointer."""
    if v is None:
        return None, ctypes.POINTER(ctypes.c_float)()
    a, p = _f32(np.ravel(v))
    assert a.shape == (dim,)
    return a, p


def ada_in(x, sample_rows, shift_a, scale_a, shift_b=None, scale_b=None, eps=1e-5):
    """Norm + AdaSingle "in" of the DiT block (seedvr2_dit.cpp:441-448): x
    [rows][dim] with rows = sum(sample_rows); shift_a/scale_a [batch][dim]."""
    xs, px = _f32(x)
    rows, dim = xs.shape
    counts = np.ascontiguousarray(sample_rows, dtype=np.int32)
    assert int(counts.sum()) == rows
    sa, psa = _f32(np.reshape(shift_a, (len(counts), dim)))
    ca, pca = _f32(np.reshape(scale_a, (len(counts), dim)))
    sb, psb = _opt_vec(shift_b, dim)
    cb, pcb = _opt_vec(scale_b, dim)
    out = np.zeros_like(xs)
    lib().orc_ada_in(px, dim, float(eps), counts.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
                     len(counts), psa, pca, psb, pcb,
                     out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
    return out


def ada_out(x, y, sample_rows, gate_a, gate_b=None):
    """AdaSingle "out" and the residual sum: returns x + y * (gate_a[b] + gate_b)."""
    xs = np.array(x, dtype=np.float32, copy=True, order="C")
    ys, py = _f32(y)
    rows, dim = xs.shape
    assert ys.shape == xs.shape
    counts = np.ascontiguousarray(sample_rows, dtype=np.int32)
    assert int(counts.sum()) == rows
    ga, pga = _f32(np.reshape(gate_a, (len(counts), dim)))
    gb, pgb = _opt_vec(gate_b, dim)
    lib().orc_ada_out(xs.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), py, dim,
                      counts.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), len(counts), pga, pgb)
    return xs


def _planar(a, pad):
    """[C, F, H, W] -> [C, F*H*W + pad] (channel stride with padding)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    c = a.shape[0]
    flat = a.reshape(c, -1)
    if pad:
        flat = np.concatenate([flat, np.full((c, pad), np.nan, np.float32)], axis=1)
    return np.ascontiguousarray(flat)


def decomposed_conv3d(cfg, x, weights, bias=None, memory=None, want_memory=False, threads=8,
                      cstep_pad=0, fast=False):
    """decomposed_conv3d.cpp:605-755.  x [Cin, F, H, W]; weights [kt, Cout,
    Cin, kh, kw]; memory [Cin, M, H, W] or None.  Returns (out_t or -1,
    out [Cout, To, Ho, Wo], next_memory [Cin, kt - st, H, W] or None)."""
    cin, frames, h, w = x.shape
    xin = _planar(x, cstep_pad)
    pxin = xin.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
    mem = None
    pm, mframes, mcs = None, 0, 0
    if memory is not None:
        mem = _planar(memory, cstep_pad)
        pm, mframes, mcs = mem.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), memory.shape[1], mem.shape[1]
    wts, pw_ = _f32(weights)
    pb = None
    if bias is not None:
        b, pb = _f32(bias)
    prefix = mframes if mframes else cfg.head_frames
    extent = cfg.dilation_t * (cfg.kernel_t - 1) + 1
    out_t = max((frames + prefix - extent) // cfg.stride_t + 1, 1)
    ow = (w + 2 * cfg.pad_w - cfg.dilation_w * (cfg.kernel_w - 1) - 1) // cfg.stride_w + 1
    oh = (h + 2 * cfg.pad_h - cfg.dilation_h * (cfg.kernel_h - 1) - 1) // cfg.stride_h + 1
    out = np.zeros((cfg.num_output, max(out_t * oh * ow, 1)), np.float32)
    cache = cfg.kernel_t - cfg.stride_t
    nxt = None
    pn, ncs = None, 0
    if want_memory and cache > 0:
        nxt = np.zeros((cin, cache * h * w), np.float32)
        pn, ncs = nxt.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), nxt.shape[1]
    code = lib(fast).orc_decomposed_conv3d(ctypes.byref(cfg), pxin, frames, h, w, xin.shape[1], pm,
                                       mframes, mcs, pw_, pb,
                                       out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                       out.shape[1], pn, ncs, threads)
    if code < 0:
        return code, None, None
    out = out[:, :code * oh * ow].reshape(cfg.num_output, code, oh, ow)
    if nxt is not None:
        nxt = nxt.reshape(cin, cache, h, w)
    return code, out, nxt


def mha(x, heads, wq, bq, wk, bk, wv, bv, wo, bo, scale=None, rows=None, threads=8, fast=False):
    """vae_chunked_mha.cpp:223-235 (ncnn MultiHeadAttention, self attention).
    x [seq][qdim]; wq/wk/wv [embed][qdim]; wo [qdim][embed].  Returns
    [seq or len(rows)][qdim]."""
    xs, px = _f32(x)
    seq, qdim = xs.shape
    embed = np.asarray(wq).shape[0]
    if scale is None:
        scale = 1.0 / float(np.sqrt(np.float32(embed // heads)))
    arrs = [_f32(a) for a in (wq, bq, wk, bk, wv, bv, wo, bo)]
    pr, n = None, seq
    if rows is not None:
        r, pr = _i32(np.asarray(rows))
        n = r.shape[0]
    out = np.zeros((n, qdim), np.float32)
    lib(fast).orc_mha(px, seq, qdim, embed, heads, float(scale), *[a[1] for a in arrs], pr, n,
                      out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), threads)
    return out


def vae_pixel_shuffle(packed, channels, tr, sr, remove_head):
    """vae_upsample3d.cpp:270-318.  packed [channels*tr*sr*sr, F, H, W] ->
    [channels, F*tr - remove_head, H*sr, W*sr]."""
    pk = np.ascontiguousarray(packed, np.float32)
    _, frames, h, w = pk.shape
    out_t = frames * tr - (1 if remove_head else 0)
    out = np.zeros((channels, out_t, h * sr, w * sr), np.float32)
    lib().orc_vae_pixel_shuffle(pk.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), channels,
                                frames, h, w, frames * h * w, tr, sr, int(bool(remove_head)),
                                out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                out_t * h * sr * w * sr)
    return out


def vae_upsample3d(post, post_w, post_b, up, up_w, up_b, x, channels, tr, sr, remove_head,
                   threads=8):
    """VAEUpsample3D::forward (vae_upsample3d.cpp:258-320) without temporal
    memory: upscale conv, shuffle, post conv."""
    code, packed, _ = decomposed_conv3d(up, x, up_w, up_b, threads=threads)
    assert code > 0
    sh = vae_pixel_shuffle(packed, channels, tr, sr, remove_head)
    code, out, _ = decomposed_conv3d(post, sh, post_w, post_b, threads=threads)
    assert code > 0
    return out


def vae_downsample3d(conv, conv_w, conv_b, x, pad_right, pad_bottom, threads=8):
    """VAEDownsample3D::forward (vae_downsample3d.cpp:145-172): zero padding
    on the right and bottom, then the conv."""
    c, f, h, w = x.shape
    xp = np.zeros((c, f, h + pad_bottom, w + pad_right), np.float32)
    xp[:, :, :h, :w] = x
    code, out, _ = decomposed_conv3d(conv, xp, conv_w, conv_b, threads=threads)
    assert code > 0
    return out
