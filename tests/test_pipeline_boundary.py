"""Argument checks of the DiT frontend/tail entry points, which return
S2_ERR_INVALID (the reference's -1, src/seedvr2/seedvr2_dit.cpp:173-191,
262-283) before any device work, so they run without a GPU."""
import ctypes

import pytest

from seedvr2_ncnn_amd import capi

INVALID = capi.S2_ERR_INVALID
FAKE = ctypes.c_void_p(0x10000)   # never dereferenced: the checks fail first


def _shapes(*s):
    flat = [x for t in s for x in t]
    return (ctypes.c_int * len(flat))(*flat)


@pytest.fixture(scope="module")
def L():
    return capi.lib()


def test_patchify_rejects_bad_shapes(L):
    assert L.s2_patchify_video(FAKE, 24, _shapes((2, 3, 4)), 1, FAKE, None) == INVALID   # odd h
    assert L.s2_patchify_video(FAKE, 24, _shapes((2, 4, 3)), 1, FAKE, None) == INVALID   # odd w
    assert L.s2_patchify_video(FAKE, 24, _shapes((0, 4, 4)), 1, FAKE, None) == INVALID
    assert L.s2_patchify_video(FAKE, 31, _shapes((2, 4, 4)), 1, FAKE, None) == INVALID   # count
    assert L.s2_patchify_video(FAKE, 0, None, 0, FAKE, None) == INVALID                  # empty
    assert L.s2_patchify_video(None, 32, _shapes((2, 4, 4)), 1, FAKE, None) == INVALID
    assert L.s2_patchify_video(ctypes.c_void_p(0x10004), 32, _shapes((2, 4, 4)), 1, FAKE,
                               None) == INVALID                                           # align


def test_unpatchify_rejects_bad_shapes(L):
    assert L.s2_unpatchify_prediction(FAKE, 7, _shapes((2, 4, 4)), 1, FAKE, None) == INVALID
    assert L.s2_unpatchify_prediction(FAKE, 8, _shapes((2, 4, 5)), 1, FAKE, None) == INVALID
    assert L.s2_unpatchify_prediction(FAKE, 8, _shapes((2, 4, 4)), 1, ctypes.c_void_p(0x10008),
                                      None) == INVALID


def test_latent_patches_and_steps_reject_bad_arguments(L):
    assert L.s2_latent_patches(FAKE, FAKE, 31, 2, 4, 4, FAKE, None) == INVALID   # stride < tokens
    assert L.s2_latent_patches(FAKE, FAKE, 32, 2, 4, 5, FAKE, None) == INVALID
    assert L.s2_latent_patches(FAKE, None, 32, 2, 4, 4, FAKE, None) == INVALID
    assert L.s2_timestep_embedding(None, 1, FAKE, None) == INVALID
    ts = (ctypes.c_float * 1)(1.0)
    assert L.s2_timestep_embedding(ts, 0, FAKE, None) == INVALID
    assert L.s2_apply_cfg(FAKE, FAKE, -1, 2.0, 0.0, FAKE, None) == INVALID
    assert L.s2_apply_cfg(FAKE, FAKE, 0, 2.0, 0.0, FAKE, None) == capi.S2_OK    # nothing to do
    assert L.s2_apply_cfg(FAKE, ctypes.c_void_p(0x10004), 8, 2.0, 0.0, FAKE, None) == INVALID
    assert L.s2_euler_step(FAKE, 9, FAKE, 10, 0.1, None) == INVALID
    assert L.s2_euler_step(FAKE, 10, FAKE, 0, 0.1, None) == capi.S2_OK
    assert L.s2_denoise_update(FAKE, None, 2, 4, 4, 1.0, 0.0, 0.1, FAKE, 31, None) == INVALID
    assert L.s2_denoise_update(FAKE, None, 2, 3, 4, 1.0, 0.0, 0.1, FAKE, 32, None) == INVALID
    assert L.s2_denoise_update(FAKE, ctypes.c_void_p(0x10004), 2, 4, 4, 1.0, 0.0, 0.1, FAKE, 32,
                               None) == INVALID


def test_block_modulation_rejects_bad_arguments(L):
    rows = _shapes((4,))
    F32, BF16 = capi.DTYPE_F32, capi.DTYPE_BF16

    def ada_in(hidden=64, batch=1, vr=rows, x=FAKE, xs=64, shift=FAKE, out=FAKE, os_=64, eps=1e-5):
        return L.s2_dit_ada_in(hidden, eps, batch, vr, None, x, None, F32, xs, shift, FAKE, None,
                               None, None, None, out, None, BF16, os_, None)

    assert ada_in(hidden=62, xs=62, os_=62) == INVALID      # hidden not a multiple of 4
    assert ada_in(hidden=4100, xs=4100, os_=4100) == INVALID   # wider than 4096
    assert ada_in(batch=0) == INVALID
    assert ada_in(batch=65, vr=_shapes(tuple([1] * 65))) == INVALID
    assert ada_in(vr=_shapes((-1,))) == INVALID
    assert ada_in(xs=60) == INVALID                         # stride below hidden
    assert ada_in(x=ctypes.c_void_p(0x10008)) == INVALID    # fp32 rows need 16 bytes
    assert ada_in(shift=None) == INVALID
    assert ada_in(eps=-1.0) == INVALID
    assert ada_in(vr=_shapes((0,))) == capi.S2_OK           # no rows: nothing to do

    def ada_out(x=FAKE, xs=64, out=FAKE, os_=64, gate=FAKE, y=FAKE):
        return L.s2_dit_ada_out(64, 1, rows, None, x, None, F32, xs, y, None, BF16, 64, gate,
                                None, None, out, None, os_, None)

    assert ada_out(gate=None) == INVALID
    assert ada_out(y=None) == INVALID
    assert ada_out(out=FAKE, xs=64, os_=128) == INVALID     # in place with another stride
    assert ada_out(gate=ctypes.c_void_p(0x10004)) == INVALID


def test_fused_block_modulation_rejects_bad_arguments(L):
    rows = _shapes((4,))
    F32, BF16 = capi.DTYPE_F32, capi.DTYPE_BF16

    def call(gate=FAKE, shift=FAKE, h=FAKE, hs=64, eps=1e-5, hidden=64):
        return L.s2_dit_ada_out_in(hidden, 1, rows, None, FAKE, None, F32, 64, FAKE, None, BF16,
                                   64, gate, None, None, FAKE, None, 64, eps, shift, FAKE, None,
                                   None, None, None, h, None, BF16, hs, None)

    assert call(gate=None) == INVALID
    assert call(shift=None) == INVALID
    assert call(h=None) == INVALID
    assert call(hs=60) == INVALID
    assert call(eps=float("nan")) == INVALID
    assert call(hidden=66) == INVALID
