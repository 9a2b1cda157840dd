"""ctypes binding of the C-ABI in include/seedvr2_hip.h (libseedvr2_hip.so).

torch supplies device memory and the current HIP stream; every computation
happens in the gfx950 kernels behind the C-ABI.  There is no fallback: if the
library is missing, or no gfx950 device is visible, calls raise.
"""
from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "lib", "libseedvr2_hip.so")
LAYERS_PATH = os.path.join(_PKG, "lib", "libseedvr2_layers.so")

S2_OK = 0
S2_ERR_INVALID = -1
S2_ERR_PLAN = -2
S2_ERR_ALLOC = -100
S2_ERR_DEVICE = -200

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2
ACT_NONE = 0
ACT_GELU = 1
ACT_SWIGLU = 2

# Every symbol include/seedvr2_hip.h declares.
EXPORTS = (
    "s2_device_count", "s2_malloc", "s2_free", "s2_memcpy_h2d", "s2_memcpy_d2h",
    "s2_memcpy_d2d", "s2_stream_synchronize", "s2_last_error", "s2_awa_plan_windows",
    "s2_awa_plan_create", "s2_awa_plan_get_info", "s2_awa_plan_get_windows",
    "s2_awa_plan_destroy", "s2_awa_plan_tables", "s2_awa_forward", "s2_cast_f32_to_bf16",
    "s2_cast_bf16_to_f32", "s2_shared_linear_forward", "s2_awa_stage_timing",
    "s2_awa_stage_times", "s2_patchify_video", "s2_latent_patches", "s2_timestep_embedding",
    "s2_unpatchify_prediction", "s2_apply_cfg", "s2_euler_step", "s2_denoise_update",
    "s2_conv3d_output_shape", "s2_conv3d_packed_weight_bytes", "s2_conv3d_pack_weights",
    "s2_conv3d_memory_bytes", "s2_conv3d_workspace_bytes", "s2_conv3d_forward",
    "s2_mha_weight_bytes", "s2_mha_prepare_weights", "s2_mha_workspace_bytes", "s2_mha_forward",
    "s2_conv3d_forward_padded", "s2_vae_pixel_shuffle", "s2_dit_ada_in", "s2_dit_ada_out",
    "s2_dit_ada_out_in", "s2_conv3d_workspace_bytes_padded", "s2_shared_linear_forward_noalloc",
    "s2_awa_qkv_forward", "s2_gelu", "s2_swiglu_pack_weight", "s2_awa_plan_cache_rope",
    "s2_stream_wait", "s2_stream_scratch_acquire", "s2_stream_scratch_release",
    "s2_binary_op", "s2_unary_op", "s2_reduce", "s2_rms_norm", "s2_copy_2d",
    "s2_shared_linear_residual",
)


class S2Error(RuntimeError):
    def __init__(self, code, what=""):
        super().__init__(f"{what} returned {code}: {last_error()}")
        self.code = code


class WindowSlice(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "sample_index", "t0", "t1", "h0", "h1", "w0", "w1", "partition_offset", "token_count")]


class AwaConfig(ctypes.Structure):
    _fields_ = [
        ("heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("target_windows", ctypes.c_int * 3),
        ("shifted", ctypes.c_int),
        ("epsilon", ctypes.c_float),
        ("rope_pairs_per_axis", ctypes.c_int),
        ("shared_norm", ctypes.c_int),
        ("official_bf16_attention", ctypes.c_int),
    ]


class Conv3dConfig(ctypes.Structure):
    """s2_conv3d_config: the 16 DecomposedConv3D config values in blob order."""
    _fields_ = [(n, ctypes.c_int) for n in (
        "num_output", "num_input", "kernel_w", "kernel_h", "kernel_t", "stride_t", "dilation_t",
        "head_frames", "stride_w", "stride_h", "dilation_w", "dilation_h", "pad_w", "pad_h",
        "groups", "bias_term")]


def conv3d_config(**kw) -> Conv3dConfig:
    c = Conv3dConfig()
    values = dict(stride_t=1, dilation_t=1, head_frames=0, stride_w=1, stride_h=1, dilation_w=1,
                  dilation_h=1, pad_w=0, pad_h=0, groups=1, bias_term=0)
    values.update(kw)
    for name, _ in Conv3dConfig._fields_:
        setattr(c, name, int(values[name]))
    return c


class MhaConfig(ctypes.Structure):
    """s2_mha_config: VAEChunkedMHA's embed_dim, num_heads, qdim and scale."""
    _fields_ = [("embed_dim", ctypes.c_int), ("num_heads", ctypes.c_int), ("qdim", ctypes.c_int),
                ("scale", ctypes.c_float)]


class PlanInfo(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int),
        ("num_windows", ctypes.c_int),
        ("video_tokens", ctypes.c_int),
        ("text_tokens", ctypes.c_int),
        ("workspace_bytes", ctypes.c_size_t),
    ]


_LIB = None


def lib() -> ctypes.CDLL:
    """Loads libseedvr2_hip.so (built by seedvr2_ncnn_amd.build); raises if absent."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run python -m seedvr2_ncnn_amd.build")
        L = ctypes.CDLL(LIB_PATH)
        P, vp, ci, cf = ctypes.POINTER, ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        sz, cl = ctypes.c_size_t, ctypes.c_long
        L.s2_last_error.restype = ctypes.c_char_p
        L.s2_device_count.argtypes = [P(ci)]
        L.s2_malloc.argtypes = [P(vp), sz]
        L.s2_free.argtypes = [vp]
        for f in ("s2_memcpy_h2d", "s2_memcpy_d2h", "s2_memcpy_d2d"):
            getattr(L, f).argtypes = [vp, vp, sz, vp]
        L.s2_stream_synchronize.argtypes = [vp]
        L.s2_awa_plan_windows.argtypes = [P(ci), ci, P(ci), ci, P(WindowSlice), ci, P(ci), P(ci), P(ci)]
        L.s2_awa_plan_create.argtypes = [P(AwaConfig), P(ci), P(ci), ci, P(vp)]
        L.s2_awa_plan_get_info.argtypes = [vp, P(PlanInfo)]
        L.s2_awa_plan_get_windows.argtypes = [vp, P(WindowSlice), ci, P(ci)]
        L.s2_awa_plan_destroy.argtypes = [vp]
        L.s2_awa_plan_tables.argtypes = [vp, vp, vp, vp, vp]
        L.s2_awa_plan_cache_rope.argtypes = [vp, vp, vp]
        L.s2_awa_forward.argtypes = [vp, vp, vp, vp, vp, vp, cl, vp, vp, vp, cl, ci, vp, vp, ci,
                                     vp, sz, vp]
        L.s2_awa_qkv_forward.argtypes = [vp, vp, vp, ci, vp, vp, vp, vp, vp, vp, ci, vp, sz, vp]
        L.s2_cast_f32_to_bf16.argtypes = [vp, vp, sz, vp]
        L.s2_gelu.argtypes = [vp, vp, sz, ci, vp]
        L.s2_swiglu_pack_weight.argtypes = [vp, vp, vp, vp, ci, ci, vp, vp, vp]
        L.s2_cast_bf16_to_f32.argtypes = [vp, vp, sz, vp]
        L.s2_shared_linear_forward.argtypes = [vp, ci, vp, ci, ci, vp, vp, ci, ci, ci, vp, vp, ci, vp]
        L.s2_shared_linear_forward_noalloc.argtypes = L.s2_shared_linear_forward.argtypes
        L.s2_awa_stage_timing.argtypes = [ci]
        L.s2_awa_stage_times.argtypes = [P(ctypes.c_float)]
        L.s2_patchify_video.argtypes = [vp, cl, P(ci), ci, vp, vp]
        L.s2_latent_patches.argtypes = [vp, vp, cl, ci, ci, ci, vp, vp]
        L.s2_timestep_embedding.argtypes = [P(cf), ci, vp, vp]
        L.s2_unpatchify_prediction.argtypes = [vp, cl, P(ci), ci, vp, vp]
        L.s2_apply_cfg.argtypes = [vp, vp, cl, cf, cf, vp, vp]
        L.s2_euler_step.argtypes = [vp, cl, vp, cl, cf, vp]
        L.s2_denoise_update.argtypes = [vp, vp, ci, ci, ci, cf, cf, cf, vp, cl, vp]
        C3 = P(Conv3dConfig)
        L.s2_conv3d_output_shape.argtypes = [C3, ci, ci, ci, ci, P(ci)]
        L.s2_conv3d_packed_weight_bytes.argtypes = [C3, P(sz)]
        L.s2_conv3d_pack_weights.argtypes = [C3, vp, vp, vp]
        L.s2_conv3d_memory_bytes.argtypes = [C3, ci, ci, P(sz), P(ci)]
        L.s2_conv3d_workspace_bytes.argtypes = [C3, ci, ci, ci, ci, P(sz)]
        L.s2_conv3d_workspace_bytes_padded.argtypes = [C3, ci, ci, ci, ci, ci, ci, P(sz)]
        M3 = P(MhaConfig)
        L.s2_mha_weight_bytes.argtypes = [M3, P(sz)]
        L.s2_mha_prepare_weights.argtypes = [M3, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
        L.s2_mha_workspace_bytes.argtypes = [M3, ci, P(sz)]
        L.s2_mha_forward.argtypes = [M3, vp, vp, ci, ci, vp, ci, vp, sz, vp]
        L.s2_conv3d_forward_padded.argtypes = [C3, vp, vp, vp, ci, ci, ci, ci, cl, ci, ci, vp, ci,
                                               vp, ci, cl, vp, vp, sz, vp]
        L.s2_vae_pixel_shuffle.argtypes = [vp, ci, ci, ci, ci, ci, cl, ci, ci, ci, vp, cl, vp]
        L.s2_conv3d_forward.argtypes = [C3, vp, vp, vp, ci, ci, ci, ci, cl, vp, ci, vp, ci, cl, vp,
                                        vp, sz, vp]
        L.s2_dit_ada_in.argtypes = [ci, cf, ci, P(ci), P(ci), vp, vp, ci, cl, vp, vp, vp, vp, vp,
                                    vp, vp, vp, ci, cl, vp]
        L.s2_dit_ada_out.argtypes = [ci, ci, P(ci), P(ci), vp, vp, ci, cl, vp, vp, ci, cl, vp, vp,
                                     vp, vp, vp, cl, vp]
        L.s2_dit_ada_out_in.argtypes = [ci, ci, P(ci), P(ci), vp, vp, ci, cl, vp, vp, ci, cl, vp,
                                        vp, vp, vp, vp, cl, cf, vp, vp, vp, vp, vp, vp, vp, vp,
                                        ci, cl, vp]
        L.s2_shared_linear_residual.argtypes = [vp, ci, vp, ci, vp, vp, ci, ci, ci, P(ci), P(ci),
                                                vp, vp, ci, vp, vp, vp, vp, vp, vp]
        _LIB = L
    return _LIB


def last_error() -> str:
    if _LIB is None:
        return ""
    return (_LIB.s2_last_error() or b"").decode()


def check(code, what=""):
    if code != S2_OK:
        raise S2Error(code, what)


def device_count() -> int:
    n = ctypes.c_int()
    check(lib().s2_device_count(ctypes.byref(n)), "s2_device_count")
    return n.value


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _ints(values):
    values = [int(v) for v in values]
    return (ctypes.c_int * max(1, len(values)))(*values)


def plan_windows(video_shapes, target_windows, shifted):
    """Window list of the host plan: (list of 9-int tuples, sample_window_count, video_tokens)."""
    L = lib()
    shapes = [int(x) for s in video_shapes for x in s]
    batch = len(shapes) // 3
    n, tokens = ctypes.c_int(), ctypes.c_int()
    counts = (ctypes.c_int * max(1, batch))()
    check(L.s2_awa_plan_windows(_ints(shapes), batch, _ints(target_windows), int(bool(shifted)),
                                None, 0, ctypes.byref(n), counts, ctypes.byref(tokens)),
          "s2_awa_plan_windows")
    buf = (WindowSlice * max(1, n.value))()
    check(L.s2_awa_plan_windows(_ints(shapes), batch, _ints(target_windows), int(bool(shifted)),
                                buf, n.value, ctypes.byref(n), None, None), "s2_awa_plan_windows")
    wins = [tuple(getattr(buf[i], f) for f, _ in WindowSlice._fields_) for i in range(n.value)]
    return wins, [counts[i] for i in range(batch)], tokens.value


def awa_config(heads=20, head_dim=128, target_windows=(4, 3, 3), shifted=False, epsilon=1e-5,
               rope_pairs=21, shared_norm=False, official_bf16=False) -> AwaConfig:
    c = AwaConfig()
    c.heads, c.head_dim = heads, head_dim
    for i in range(3):
        c.target_windows[i] = int(target_windows[i])
    c.shifted = int(bool(shifted))
    c.epsilon = float(epsilon)
    c.rope_pairs_per_axis = rope_pairs
    c.shared_norm = int(bool(shared_norm))
    c.official_bf16_attention = int(bool(official_bf16))
    return c


class AwaPlan:
    """Device-resident window plan (s2_awa_plan_create / _destroy)."""

    def __init__(self, config: AwaConfig, video_shapes, text_lengths):
        self.config = config
        self._h = ctypes.c_void_p()
        shapes = [int(x) for s in video_shapes for x in s]
        batch = len(text_lengths)
        check(lib().s2_awa_plan_create(ctypes.byref(config), _ints(shapes), _ints(text_lengths),
                                       batch, ctypes.byref(self._h)), "s2_awa_plan_create")
        self.info = PlanInfo()
        check(lib().s2_awa_plan_get_info(self._h, ctypes.byref(self.info)), "s2_awa_plan_get_info")

    @property
    def handle(self):
        return self._h

    def windows(self):
        n = self.info.num_windows
        buf = (WindowSlice * max(1, n))()
        counts = (ctypes.c_int * max(1, self.info.batch))()
        check(lib().s2_awa_plan_get_windows(self._h, buf, n, counts), "s2_awa_plan_get_windows")
        wins = [tuple(getattr(buf[i], f) for f, _ in WindowSlice._fields_) for i in range(n)]
        return wins, [counts[i] for i in range(self.info.batch)]

    def tables(self, device="cuda"):
        """(video_indices, inverse_video_indices, local_positions) computed on the device."""
        import torch
        L = self.info.video_tokens
        idx = torch.full((L,), -7, dtype=torch.int32, device=device)
        inv = torch.full((L,), -7, dtype=torch.int32, device=device)
        pos = torch.full((L, 3), -7, dtype=torch.int32, device=device)
        check(lib().s2_awa_plan_tables(self._h, _ptr(idx), _ptr(inv), _ptr(pos), _stream()),
              "s2_awa_plan_tables")
        return idx, inv, pos

    def cache_rope(self, rope_freqs):
        """s2_awa_plan_cache_rope: the plan keeps the cos/sin table of these
        frequencies (a device fp32 tensor; None clears the cache).  Forwards
        given the same tensor then skip recomputing it."""
        check(lib().s2_awa_plan_cache_rope(self._h, _ptr(rope_freqs), _stream()),
              "s2_awa_plan_cache_rope")

    def close(self):
        if self._h:
            lib().s2_awa_plan_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def _dtype_code(t):
    import torch
    if t.dtype == torch.bfloat16:
        return DTYPE_BF16
    if t.dtype == torch.float16:
        return DTYPE_F16
    if t.dtype == torch.float32:
        return DTYPE_F32
    raise TypeError(f"unsupported dtype {t.dtype}")


def awa_forward(plan: AwaPlan, norm_weights, rope_freqs, video_q, video_k, video_v, text_q,
                text_k, text_v, out_dtype=None, workspace=None, out_video=None, out_text=None,
                stream=None):
    """Runs s2_awa_forward on torch device tensors.  video_* / text_* are 2-D
    row views (unit column stride, shared row stride: views into one fused
    [L, 3*inner] tensor are fine).  Returns (out_video, out_text)."""
    import torch
    inner = plan.config.heads * plan.config.head_dim
    ins = (video_q, video_k, video_v, text_q, text_k, text_v)
    for t in ins:
        assert t.is_cuda and t.dim() == 2 and t.stride(1) == 1 and t.shape[1] == inner
    dt = _dtype_code(video_q)
    assert all(_dtype_code(t) == dt for t in ins)
    vs, ts = video_q.stride(0), text_q.stride(0)
    assert video_k.stride(0) == vs and video_v.stride(0) == vs
    assert text_k.stride(0) == ts and text_v.stride(0) == ts
    odt = out_dtype or video_q.dtype
    dev = video_q.device
    if out_video is None:
        out_video = torch.empty((plan.info.video_tokens, inner), dtype=odt, device=dev)
    if out_text is None:
        out_text = torch.empty((plan.info.text_tokens, inner), dtype=odt, device=dev)
    if workspace is None:
        workspace = torch.empty(plan.info.workspace_bytes, dtype=torch.uint8, device=dev)
    check(lib().s2_awa_forward(plan.handle, _ptr(norm_weights), _ptr(rope_freqs),
                               _ptr(video_q), _ptr(video_k), _ptr(video_v), vs,
                               _ptr(text_q), _ptr(text_k), _ptr(text_v), ts, dt,
                               _ptr(out_video), _ptr(out_text), _dtype_code(out_video),
                               _ptr(workspace), workspace.numel(), _stream(stream)),
          "s2_awa_forward")
    return out_video, out_text


def awa_qkv_forward(plan: AwaPlan, x_video, x_text, qkv_weight_bf16, qkv_bias, norm_weights,
                    rope_freqs, out_dtype=None, workspace=None, out_video=None, out_text=None,
                    stream=None):
    """s2_awa_qkv_forward: the QKV projection (bf16 activations x_* [L][hidden],
    weight [3*inner][hidden]) and the attention layer in one call.  Returns
    (out_video, out_text)."""
    import torch
    inner = plan.config.heads * plan.config.head_dim
    assert x_video.dtype == torch.bfloat16 and x_text.dtype == torch.bfloat16
    assert x_video.is_contiguous() and x_text.is_contiguous()
    hidden = x_video.shape[1]
    assert x_text.shape[1] == hidden and qkv_weight_bf16.shape == (3 * inner, hidden)
    assert qkv_weight_bf16.dtype == torch.bfloat16 and qkv_weight_bf16.is_contiguous()
    odt = out_dtype or torch.bfloat16
    dev = x_video.device
    if out_video is None:
        out_video = torch.empty((plan.info.video_tokens, inner), dtype=odt, device=dev)
    if out_text is None:
        out_text = torch.empty((plan.info.text_tokens, inner), dtype=odt, device=dev)
    if workspace is None:
        workspace = torch.empty(plan.info.workspace_bytes, dtype=torch.uint8, device=dev)
    check(lib().s2_awa_qkv_forward(plan.handle, _ptr(x_video), _ptr(x_text), hidden,
                                   _ptr(qkv_weight_bf16), _ptr(qkv_bias), _ptr(norm_weights),
                                   _ptr(rope_freqs), _ptr(out_video), _ptr(out_text),
                                   _dtype_code(out_video), _ptr(workspace), workspace.numel(),
                                   _stream(stream)), "s2_awa_qkv_forward")
    return out_video, out_text


AWA_STAGES = ("rope_table", "prologue", "attention", "text_pool")


def awa_stage_timing(enable: bool) -> None:
    """s2_awa_stage_timing: record events around the four kernels of every
    awa_forward on this thread (a diagnostic)."""
    check(lib().s2_awa_stage_timing(1 if enable else 0), "s2_awa_stage_timing")


def awa_stage_times() -> dict:
    """s2_awa_stage_times: milliseconds of the last timed awa_forward's
    RoPE table, prologue, attention and text-pool kernels."""
    out = (ctypes.c_float * 4)()
    check(lib().s2_awa_stage_times(out), "s2_awa_stage_times")
    return dict(zip(AWA_STAGES, (float(v) for v in out)))


def cast_f32_to_bf16(src, dst=None, stream=None):
    import torch
    if dst is None:
        dst = torch.empty(src.shape, dtype=torch.bfloat16, device=src.device)
    check(lib().s2_cast_f32_to_bf16(_ptr(src), _ptr(dst), src.numel(), _stream(stream)),
          "s2_cast_f32_to_bf16")
    return dst


def swiglu_pack_weight(gate_bf16, up_bf16, gate_bias=None, up_bias=None, stream=None):
    """s2_swiglu_pack_weight: the interleaved [2n][k] weight (and [2n] bias)
    of a SwiGLU shared_linear from gate and up projections [n][k]."""
    import torch
    n, k = gate_bf16.shape
    packed = torch.empty(2 * n, k, dtype=torch.bfloat16, device=gate_bf16.device)
    pb = None if gate_bias is None else torch.empty(2 * n, device=gate_bf16.device)
    check(lib().s2_swiglu_pack_weight(_ptr(gate_bf16), _ptr(up_bf16), _ptr(gate_bias),
                                      _ptr(up_bias), n, k, _ptr(packed), _ptr(pb), _stream(stream)),
          "s2_swiglu_pack_weight")
    return packed, pb


def gelu(x, y=None, stream=None):
    """s2_gelu: elementwise erf-GELU of a device tensor (fp32, bf16 or fp16)."""
    import torch
    if y is None:
        y = torch.empty_like(x)
    assert x.is_contiguous() and y.is_contiguous() and y.dtype == x.dtype
    check(lib().s2_gelu(_ptr(x), _ptr(y), x.numel(), _dtype_code(x), _stream(stream)), "s2_gelu")
    return y


def shared_linear(x_video, x_text, weight_bf16, bias=None, activation=ACT_NONE, out_dtype=None,
                  y_video=None, y_text=None, stream=None, noalloc=False):
    """s2_shared_linear_forward: y = act(x W^T + b) for both streams
    (s2_shared_linear_forward_noalloc with noalloc=True)."""
    import torch
    n, k = weight_bf16.shape
    if activation == ACT_SWIGLU:
        n //= 2   # the interleaved gate/up weight has two rows per output column
    assert weight_bf16.dtype == torch.bfloat16 and weight_bf16.is_contiguous()
    xd = _dtype_code(x_video)
    assert x_text is None or _dtype_code(x_text) == xd
    odt = out_dtype or x_video.dtype
    m0 = x_video.shape[0]
    m1 = 0 if x_text is None else x_text.shape[0]
    dev = x_video.device
    if y_video is None:
        y_video = torch.empty((m0, n), dtype=odt, device=dev)
    if y_text is None and m1:
        y_text = torch.empty((m1, n), dtype=odt, device=dev)
    name = "s2_shared_linear_forward_noalloc" if noalloc else "s2_shared_linear_forward"
    check(getattr(lib(), name)(_ptr(x_video), m0, _ptr(x_text) if m1 else None, m1, xd,
                               _ptr(weight_bf16), _ptr(bias), n, k, activation, _ptr(y_video),
                               _ptr(y_text) if m1 else None, _dtype_code(y_video),
                               _stream(stream)), name)
    return y_video, y_text


# ---- DiT block: norm and AdaSingle modulation -------------------------------

def _row_stride(*ts):
    strides = {t.stride(0) for t in ts if t is not None and t.shape[0] > 0}
    assert len(strides) <= 1, "the two streams must share one row stride"
    for t in ts:
        assert t is None or (t.dim() == 2 and t.stride(1) == 1)
    return strides.pop() if strides else 0


def ada_in(x_video, x_text, video_rows, text_rows, shift, scale, video_shift=None,
           video_scale=None, text_shift=None, text_scale=None, eps=1e-5, out_dtype=None,
           out_video=None, out_text=None, stream=None):
    """s2_dit_ada_in: rmsnorm(x) * (scale[b] + *_scale) + (shift[b] + *_shift)
    for both streams.  x_*: [rows, hidden] row views; shift/scale [batch, hidden]
    fp32; video_rows/text_rows: rows per sample.  Returns (out_video, out_text)."""
    import torch
    hidden = x_video.shape[1]
    batch = len(video_rows)
    assert text_rows is None or len(text_rows) == batch
    nt = 0 if text_rows is None else sum(int(r) for r in text_rows)
    odt = out_dtype or x_video.dtype
    if out_video is None:
        out_video = torch.empty((x_video.shape[0], hidden), dtype=odt, device=x_video.device)
    if out_text is None and nt:
        out_text = torch.empty((nt, hidden), dtype=odt, device=x_video.device)
    xs = _row_stride(x_video, x_text if nt else None)
    os_ = _row_stride(out_video, out_text if nt else None)
    check(lib().s2_dit_ada_in(hidden, float(eps), batch, _ints(video_rows),
                              _ints(text_rows) if text_rows is not None else None,
                              _ptr(x_video), _ptr(x_text) if nt else None,
                              _dtype_code(x_video), xs or hidden, _ptr(shift), _ptr(scale),
                              _ptr(video_shift), _ptr(video_scale), _ptr(text_shift),
                              _ptr(text_scale), _ptr(out_video), _ptr(out_text) if nt else None,
                              _dtype_code(out_video), os_ or hidden, _stream(stream)),
          "s2_dit_ada_in")
    return out_video, out_text


def ada_out(x_video, x_text, y_video, y_text, video_rows, text_rows, gate, video_gate=None,
            text_gate=None, out_video=None, out_text=None, stream=None):
    """s2_dit_ada_out: x + y * (gate[b] + *_gate) for both streams; by
    default in place (out = x).  Returns (out_video, out_text)."""
    hidden = x_video.shape[1]
    batch = len(video_rows)
    nt = 0 if text_rows is None else sum(int(r) for r in text_rows)
    if out_video is None:
        out_video = x_video
    if out_text is None and nt:
        out_text = x_text
    assert out_video.dtype == x_video.dtype
    xs = _row_stride(x_video, x_text if nt else None)
    ys = _row_stride(y_video, y_text if nt else None)
    os_ = _row_stride(out_video, out_text if nt else None)
    check(lib().s2_dit_ada_out(hidden, batch, _ints(video_rows),
                               _ints(text_rows) if text_rows is not None else None,
                               _ptr(x_video), _ptr(x_text) if nt else None,
                               _dtype_code(x_video), xs or hidden, _ptr(y_video),
                               _ptr(y_text) if nt else None, _dtype_code(y_video), ys or hidden,
                               _ptr(gate), _ptr(video_gate), _ptr(text_gate), _ptr(out_video),
                               _ptr(out_text) if nt else None, os_ or hidden, _stream(stream)),
          "s2_dit_ada_out")
    return out_video, out_text


def ada_out_in(x_video, x_text, y_video, y_text, video_rows, text_rows, gate, shift, scale,
               video_gate=None, text_gate=None, video_shift=None, video_scale=None,
               text_shift=None, text_scale=None, eps=1e-5, h_dtype=None, h_video=None,
               h_text=None, out_video=None, out_text=None, stream=None):
    """s2_dit_ada_out_in: x += y * gate (in place by default), then
    h = rmsnorm(x) * scale + shift.  Returns (out_video, out_text, h_video, h_text)."""
    import torch
    hidden = x_video.shape[1]
    batch = len(video_rows)
    nt = 0 if text_rows is None else sum(int(r) for r in text_rows)
    hdt = h_dtype or torch.bfloat16
    if out_video is None:
        out_video = x_video
    if out_text is None and nt:
        out_text = x_text
    if h_video is None:
        h_video = torch.empty((x_video.shape[0], hidden), dtype=hdt, device=x_video.device)
    if h_text is None and nt:
        h_text = torch.empty((nt, hidden), dtype=hdt, device=x_video.device)
    xs = _row_stride(x_video, x_text if nt else None)
    ys = _row_stride(y_video, y_text if nt else None)
    os_ = _row_stride(out_video, out_text if nt else None)
    hs = _row_stride(h_video, h_text if nt else None)
    check(lib().s2_dit_ada_out_in(hidden, batch, _ints(video_rows),
                                  _ints(text_rows) if text_rows is not None else None,
                                  _ptr(x_video), _ptr(x_text) if nt else None,
                                  _dtype_code(x_video), xs or hidden, _ptr(y_video),
                                  _ptr(y_text) if nt else None, _dtype_code(y_video),
                                  ys or hidden, _ptr(gate), _ptr(video_gate), _ptr(text_gate),
                                  _ptr(out_video), _ptr(out_text) if nt else None, os_ or hidden,
                                  float(eps), _ptr(shift), _ptr(scale), _ptr(video_shift),
                                  _ptr(video_scale), _ptr(text_shift), _ptr(text_scale),
                                  _ptr(h_video), _ptr(h_text) if nt else None,
                                  _dtype_code(h_video), hs or hidden, _stream(stream)),
          "s2_dit_ada_out_in")
    return out_video, out_text, h_video, h_text


def shared_linear_residual(x_video, x_text, weight_bf16, bias, video_rows, text_rows, res_video,
                           res_text, gate, video_gate=None, text_gate=None, out_video=None,
                           out_text=None, stream=None):
    """s2_shared_linear_residual: out = res + (x W^T + b, rounded to bf16) *
    (gate[b] + *_gate); in place (out = res) by default.  Returns
    (out_video, out_text)."""
    import torch
    n, k = weight_bf16.shape
    assert weight_bf16.dtype == torch.bfloat16 and weight_bf16.is_contiguous()
    m0 = x_video.shape[0]
    m1 = 0 if x_text is None else x_text.shape[0]
    if out_video is None:
        out_video = res_video
    if out_text is None and m1:
        out_text = res_text
    for t in (x_video, x_text, res_video, res_text, out_video, out_text):
        assert t is None or t.shape[0] == 0 or t.is_contiguous()
    check(lib().s2_shared_linear_residual(
        _ptr(x_video), m0, _ptr(x_text) if m1 else None, m1, _ptr(weight_bf16), _ptr(bias), n, k,
        len(video_rows), _ints(video_rows), _ints(text_rows) if text_rows is not None else None,
        _ptr(res_video), _ptr(res_text) if m1 else None, _dtype_code(res_video), _ptr(gate),
        _ptr(video_gate), _ptr(text_gate), _ptr(out_video), _ptr(out_text) if m1 else None,
        _stream(stream)), "s2_shared_linear_residual")
    return out_video, out_text


# ---- DiT frontend and tail, sampler step -------------------------------------

def _shape_ints(video_shapes):
    flat = [int(x) for s in video_shapes for x in s]
    return _ints(flat), len(flat) // 3


def patchify_video(video, video_shapes, patches=None, stream=None):
    """s2_patchify_video: [tokens, 33] fp32 -> [patches, 132]."""
    import torch
    shapes, batch = _shape_ints(video_shapes)
    n = sum(int(t) * (int(h) // 2) * (int(w) // 2) for t, h, w in video_shapes)
    if patches is None:
        patches = torch.empty((n, 132), dtype=torch.float32, device=video.device)
    check(lib().s2_patchify_video(_ptr(video), video.shape[0], shapes, batch, _ptr(patches),
                                  _stream(stream)), "s2_patchify_video")
    return patches


def latent_patches(latent, condition, frames, height, width, channel_stride, patches=None,
                   stream=None):
    """s2_latent_patches: 16-plane latent and condition -> [patches, 132]."""
    import torch
    if patches is None:
        patches = torch.empty((frames * (height // 2) * (width // 2), 132), dtype=torch.float32,
                              device=latent.device)
    check(lib().s2_latent_patches(_ptr(latent), _ptr(condition), channel_stride, frames, height,
                                  width, _ptr(patches), _stream(stream)), "s2_latent_patches")
    return patches


def timestep_embedding(timesteps, device="cuda", embedding=None, stream=None):
    """s2_timestep_embedding: host timesteps -> device [count, 256]."""
    import torch
    ts = [float(t) for t in timesteps]
    if embedding is None:
        embedding = torch.empty((len(ts), 256), dtype=torch.float32, device=device)
    arr = (ctypes.c_float * max(1, len(ts)))(*ts)
    check(lib().s2_timestep_embedding(arr, len(ts), _ptr(embedding), _stream(stream)),
          "s2_timestep_embedding")
    return embedding


def unpatchify_prediction(patches, video_shapes, prediction=None, stream=None):
    """s2_unpatchify_prediction: [patches, 64] -> [tokens, 16]."""
    import torch
    shapes, batch = _shape_ints(video_shapes)
    n = sum(int(t) * int(h) * int(w) for t, h, w in video_shapes)
    if prediction is None:
        prediction = torch.empty((n, 16), dtype=torch.float32, device=patches.device)
    check(lib().s2_unpatchify_prediction(_ptr(patches), patches.shape[0], shapes, batch,
                                         _ptr(prediction), _stream(stream)),
          "s2_unpatchify_prediction")
    return prediction


def apply_cfg(positive, negative, scale, rescale, output=None, stream=None):
    """s2_apply_cfg over all elements of positive/negative (contiguous fp32)."""
    import torch
    if output is None:
        output = torch.empty_like(positive)
    check(lib().s2_apply_cfg(_ptr(positive), _ptr(negative), positive.numel(), float(scale),
                             float(rescale), _ptr(output), _stream(stream)), "s2_apply_cfg")
    return output


def euler_step(latent, channel_stride, prediction, delta, stream=None):
    """s2_euler_step: latent planes += delta * prediction^T, in place."""
    check(lib().s2_euler_step(_ptr(latent), channel_stride, _ptr(prediction),
                              prediction.shape[0], float(delta), _stream(stream)),
          "s2_euler_step")
    return latent


def denoise_update(positive_patches, negative_patches, frames, height, width, cfg_scale,
                   cfg_rescale, delta, latent, channel_stride, stream=None):
    """s2_denoise_update: one sampler step from patchified predictions, in place."""
    check(lib().s2_denoise_update(_ptr(positive_patches), _ptr(negative_patches), frames, height,
                                  width, float(cfg_scale), float(cfg_rescale), float(delta),
                                  _ptr(latent), channel_stride, _stream(stream)),
          "s2_denoise_update")
    return latent


# ---- DecomposedConv3D ------------------------------------------------------------

class Conv3d:
    """Device state of one DecomposedConv3D: packed bf16 weights, bias and the
    temporal memory (s2_conv3d_*)."""

    def __init__(self, config: Conv3dConfig, weights, bias=None, stream=None):
        import torch
        self.config = config
        n = ctypes.c_size_t()
        check(lib().s2_conv3d_packed_weight_bytes(ctypes.byref(config), ctypes.byref(n)),
              "s2_conv3d_packed_weight_bytes")
        self.packed = torch.empty(n.value // 2, dtype=torch.int16, device=weights.device)
        check(lib().s2_conv3d_pack_weights(ctypes.byref(config), _ptr(weights.contiguous()),
                                           _ptr(self.packed), _stream(stream)),
              "s2_conv3d_pack_weights")
        self.bias = bias
        self.memory = None
        self.memory_frames = 0

    def output_shape(self, frames, height, width, memory_frames=0):
        out = (ctypes.c_int * 3)()
        check(lib().s2_conv3d_output_shape(ctypes.byref(self.config), frames, height, width,
                                           memory_frames, out), "s2_conv3d_output_shape")
        return tuple(out)

    def forward(self, x, frames, height, width, cstep=None, use_memory=False, keep_memory=False,
                out_dtype=None, out_cstep=None, reuse_memory_buffer=False, stream=None,
                staged_only_workspace=False):
        """x: device [num_input, cstep] planar (cstep >= frames*height*width).
        Returns the output as [num_output, out_cstep].  reuse_memory_buffer
        writes the new memory over the one this call reads.
        staged_only_workspace passes a workspace that holds only the staged
        frames (no partial tiles), which runs the k loop unsplit."""
        import torch
        cfg = self.config
        mem = self.memory if use_memory and self.memory is not None else None
        mframes = self.memory_frames if mem is not None else 0
        to, ho, wo = self.output_shape(frames, height, width, mframes)
        odt = out_dtype or x.dtype
        ocs = out_cstep or to * ho * wo
        out = torch.empty((cfg.num_output, ocs), dtype=odt, device=x.device)
        ws_n = ctypes.c_size_t()
        check(lib().s2_conv3d_workspace_bytes(ctypes.byref(cfg), frames, height, width, mframes,
                                              ctypes.byref(ws_n)), "s2_conv3d_workspace_bytes")
        if staged_only_workspace:
            cin = cfg.num_input
            cpad = 8 if cin <= 8 else 16 if cin <= 16 else 32 if cin <= 32 else (cin + 63) // 64 * 64
            staged = (frames + mframes) * height * width * cpad * 2
            ws_n.value = min(ws_n.value, (staged + 255) // 256 * 256)
        ws = torch.empty(ws_n.value, dtype=torch.uint8, device=x.device)
        nxt = None
        if keep_memory:
            nb, nf = ctypes.c_size_t(), ctypes.c_int()
            check(lib().s2_conv3d_memory_bytes(ctypes.byref(cfg), height, width, ctypes.byref(nb),
                                               ctypes.byref(nf)), "s2_conv3d_memory_bytes")
            if nf.value > 0:
                if reuse_memory_buffer and mem is not None and mem.numel() == nb.value:
                    nxt = mem
                else:
                    nxt = torch.empty(nb.value, dtype=torch.uint8, device=x.device)
        check(lib().s2_conv3d_forward(ctypes.byref(cfg), _ptr(self.packed), _ptr(self.bias), _ptr(x),
                                      _dtype_code(x), frames, height, width,
                                      cstep or x.shape[1], _ptr(mem), mframes, _ptr(out),
                                      _dtype_code(out), ocs, _ptr(nxt), _ptr(ws), ws.numel(),
                                      _stream(stream)), "s2_conv3d_forward")
        if keep_memory:
            self.memory = nxt
            self.memory_frames = cfg.kernel_t - cfg.stride_t if nxt is not None else 0
        return out, (to, ho, wo)


# ---- VAEChunkedMHA -------------------------------------------------------------

class Mha:
    """Device weights of one VAEChunkedMHA (s2_mha_*).  Weights are device
    fp32 tensors in the reference load_model order."""

    def __init__(self, heads, wq, bq, wk, bk, wv, bv, wo, bo, scale=None, stream=None):
        import math
        import torch
        embed, qdim = wq.shape
        self.config = MhaConfig(embed, heads, qdim,
                                scale if scale is not None else 1.0 / math.sqrt(embed // heads))
        n = ctypes.c_size_t()
        check(lib().s2_mha_weight_bytes(ctypes.byref(self.config), ctypes.byref(n)),
              "s2_mha_weight_bytes")
        self.prepared = torch.empty(n.value, dtype=torch.uint8, device=wq.device)
        ws = [t.contiguous() for t in (wq, bq, wk, bk, wv, bv, wo, bo)]
        check(lib().s2_mha_prepare_weights(ctypes.byref(self.config), *[_ptr(t) for t in ws],
                                           _ptr(self.prepared), _stream(stream)),
              "s2_mha_prepare_weights")

    def forward(self, x, out_dtype=None, stream=None):
        """x: device [seq, qdim]; returns [seq, qdim]."""
        import torch
        seq = x.shape[0]
        n = ctypes.c_size_t()
        check(lib().s2_mha_workspace_bytes(ctypes.byref(self.config), seq, ctypes.byref(n)),
              "s2_mha_workspace_bytes")
        ws = torch.empty(n.value, dtype=torch.uint8, device=x.device)
        out = torch.empty((seq, self.config.qdim), dtype=out_dtype or x.dtype, device=x.device)
        check(lib().s2_mha_forward(ctypes.byref(self.config), _ptr(self.prepared), _ptr(x),
                                   _dtype_code(x), seq, _ptr(out), _dtype_code(out), _ptr(ws),
                                   ws.numel(), _stream(stream)), "s2_mha_forward")
        return out
