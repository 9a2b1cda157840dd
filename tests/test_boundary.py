"""The drop-in boundary without a GPU: the C-ABI library loads and exports
every symbol include/seedvr2_hip.h declares, argument validation returns the
reference's codes, and the ncnn-surface layers reject bad blobs and weights
with the reference's return codes (src/seedvr2/adaptive_window_attention.cpp:
700-831, src/seedvr2/shared_linear.cpp:27-96) before touching a device."""
import ctypes
import os
import re

import numpy as np
import pytest

from common import ROOT, Layer, awa_param_string
from seedvr2_ncnn_amd import capi


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "seedvr2_hip.h")).read()
    return sorted(set(re.findall(r"\b(s2_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert _declared_symbols() == sorted(capi.EXPORTS)


def test_library_exports_every_declared_symbol():
    L = capi.lib()
    for name in _declared_symbols():
        assert hasattr(L, name), name


def test_library_exports_only_declared_functions():
    """libseedvr2_hip.so is built with hidden visibility: its dynamic symbol
    table holds the functions of include/seedvr2_hip.h and no internals."""
    import shutil
    import subprocess
    if shutil.which("nm") is None:
        pytest.skip("nm not available")
    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    funcs = sorted(line.split()[-1] for line in out.splitlines() if line.split()[1:2] == ["T"])
    assert funcs == _declared_symbols()


def test_layers_library_loads():
    ctypes.CDLL(capi.LAYERS_PATH)


def _no_device():
    return capi.device_count() == 0


def test_plan_create_validates_before_the_device():
    c = capi.awa_config(heads=20, head_dim=128, rope_pairs=22)   # 6*22 > 128
    with pytest.raises(capi.S2Error) as e:
        capi.AwaPlan(c, [(1, 8, 8)], [4])
    assert e.value.code == capi.S2_ERR_INVALID
    with pytest.raises(capi.S2Error) as e:
        capi.AwaPlan(capi.awa_config(), [(1, 8, 8)], [0])        # text length 0
    assert e.value.code == capi.S2_ERR_INVALID
    with pytest.raises(capi.S2Error) as e:
        capi.AwaPlan(capi.awa_config(head_dim=96, rope_pairs=16), [(1, 8, 8)], [4])
    assert e.value.code == capi.S2_ERR_INVALID


def test_shared_linear_validates_before_the_device():
    L = capi.lib()
    dummy = ctypes.c_void_p(256)
    # k not a multiple of 8
    assert L.s2_shared_linear_forward(dummy, 4, None, 0, 1, dummy, None, 16, 12, 0, dummy, None, 1,
                                      None) == capi.S2_ERR_INVALID
    # unknown activation
    assert L.s2_shared_linear_forward(dummy, 4, None, 0, 1, dummy, None, 16, 16, 7, dummy, None, 1,
                                      None) == capi.S2_ERR_INVALID
    # null weight
    assert L.s2_shared_linear_forward(dummy, 4, None, 0, 1, None, None, 16, 16, 0, dummy, None, 1,
                                      None) == capi.S2_ERR_INVALID


# ---- AdaptiveWindowAttention layer surface -----------------------------------------

HEADS, D, PAIRS = 2, 64, 10
INNER = HEADS * D


def _awa_weights(d=D, pairs=PAIRS, shared=False):
    g = np.random.default_rng(0)
    n = 2 if shared else 4
    return [g.standard_normal(d).astype(np.float32) for _ in range(n)] + [np.ones(pairs, np.float32)]


def _awa(shifted=0, shared=False, int32=False, pairs=PAIRS, weights=True):
    params = awa_param_string(HEADS, D, (1, 2, 2), shifted, 1e-5, pairs, shared_norm=shared,
                              int32_shapes=int32)
    return Layer("AdaptiveWindowAttention", params, _awa_weights(pairs=pairs, shared=shared) if weights else None)


def _blobs(lv=16, lt=3, shape=(1, 4, 4)):
    video = np.zeros((lv, 3 * INNER), np.float32)
    text = np.zeros((lt, 3 * INNER), np.float32)
    vs = np.asarray(shape, np.float32)
    tl = np.asarray([lt], np.float32)
    return [video, text, vs, tl]


OUTS = [((16, INNER), np.float32), ((3, INNER), np.float32)]


def test_awa_load_param_and_model_codes():
    layer = _awa()
    assert layer.create_code == 0
    # truncated weights: load_model returns -100 (reference :720-737)
    w = _awa_weights()
    short = Layer("AdaptiveWindowAttention", awa_param_string(HEADS, D, (1, 2, 2), 0, 1e-5, PAIRS),
                  [np.concatenate(w)[:-1]])
    assert short.create_code == -100
    # shared_norm consumes only two norm vectors plus the frequencies
    assert _awa(shared=True).create_code == 0


def test_awa_forward_rejects_bad_arity():
    layer = _awa()
    code, _ = layer.forward(_blobs()[:3], OUTS)
    assert code == -1
    code, _ = layer.forward(_blobs(), OUTS[:1])
    assert code == -1


def test_awa_forward_rejects_bad_widths_and_counts():
    layer = _awa()
    b = _blobs()
    b[0] = np.zeros((16, 3 * INNER - 8), np.float32)
    assert layer.forward(b, OUTS)[0] == -1
    b = _blobs()
    b[1] = np.zeros((4, 3 * INNER), np.float32)      # text rows != text length
    assert layer.forward(b, OUTS)[0] == -1
    b = _blobs(shape=(1, 4, 5))                        # video rows != t*h*w
    assert layer.forward(b, OUTS)[0] == -1
    b = _blobs()
    b[2] = np.asarray([1, 4], np.float32)              # shape blob width != 3
    assert layer.forward(b, OUTS)[0] == -1


def test_awa_forward_rejects_nonpositive_text_length():
    layer = _awa()
    b = _blobs()
    b[3] = np.asarray([0], np.float32)
    assert layer.forward(b, OUTS)[0] == -1


def test_awa_forward_rejects_too_many_rope_pairs():
    layer = _awa(pairs=11)                               # 6*11 > 64
    assert layer.forward(_blobs(), OUTS)[0] == -1


def test_awa_forward_rejects_missing_weights():
    layer = _awa(weights=False)
    assert layer.forward(_blobs(), OUTS)[0] == -1


def test_awa_split_form_checks_each_part():
    layer = _awa()
    parts = [np.zeros((16, INNER), np.float32)] * 3 + [np.zeros((3, INNER), np.float32)] * 3
    parts = list(parts) + [np.asarray([1, 4, 4], np.float32), np.asarray([3], np.float32)]
    bad = list(parts)
    bad[4] = np.zeros((3, INNER + 8), np.float32)
    assert layer.forward(bad, OUTS)[0] == -1
    bad = list(parts)
    bad[1] = np.zeros((15, INNER), np.float32)
    assert layer.forward(bad, OUTS)[0] == -1


@pytest.mark.skipif("not _no_device()")
def test_awa_forward_without_device_fails_loudly():
    # no device: the reference's -100, never the C-ABI's S2_ERR_DEVICE
    layer = _awa()
    assert layer.forward(_blobs(), OUTS)[0] == -100


def test_awa_rejects_head_dims_the_kernels_lack():
    """Stated deviation: the attention kernels exist for head_dim 64 and 128
    only (the SeedVR2 DiTs use 128).  The reference accepts any head_dim with
    6 * rope_pairs <= head_dim (adaptive_window_attention.cpp:770); here other
    widths return -1 before any device work."""
    heads, d, pairs = 2, 96, 16
    params = awa_param_string(heads, d, (1, 2, 2), 0, 1e-5, pairs)
    g = np.random.default_rng(1)
    w = [g.standard_normal(d).astype(np.float32) for _ in range(4)] + [np.ones(pairs, np.float32)]
    layer = Layer("AdaptiveWindowAttention", params, w)
    assert layer.create_code == 0
    inner = heads * d
    blobs = [np.zeros((16, 3 * inner), np.float32), np.zeros((3, 3 * inner), np.float32),
             np.asarray([1, 4, 4], np.float32), np.asarray([3], np.float32)]
    outs = [((16, inner), np.float32), ((3, inner), np.float32)]
    assert layer.forward(blobs, outs)[0] == -1


# ---- SharedLinear layer surface ------------------------------------------------------

def test_shared_linear_param_codes():
    assert Layer("SharedLinear", "0=0 1=16 2=1").create_code == -1
    assert Layer("SharedLinear", "0=16 1=0 2=1").create_code == -1
    w = np.zeros(16 * 8, np.float32)
    assert Layer("SharedLinear", "0=16 1=8 2=1", [w]).create_code == -100      # bias missing
    assert Layer("SharedLinear", "0=16 1=8 2=0", [w]).create_code == 0
    assert Layer("SharedLinear", "0=16 1=8 2=0", [w[:-1]]).create_code == -100  # truncated


def test_shared_linear_forward_codes():
    w = np.zeros(16 * 8, np.float32)
    layer = Layer("SharedLinear", "0=16 1=8 2=0", [w])
    outs = [((4, 16), np.float32), ((2, 16), np.float32)]
    assert layer.forward([np.zeros((4, 8), np.float32)], outs)[0] == -1
    assert layer.forward([np.zeros((4, 8), np.float32), np.zeros((2, 9), np.float32)], outs)[0] == -1
    assert layer.forward([np.zeros((4, 8), np.float32), np.zeros(8, np.float32)], outs)[0] == -1
    if _no_device():
        assert layer.forward([np.zeros((4, 8), np.float32), np.zeros((2, 8), np.float32)],
                             outs)[0] == -100


def test_shared_linear_rejects_input_widths_not_a_multiple_of_8():
    """Stated deviation: operand rows are read as 16-byte chunks, so
    num_input must be a multiple of 8 (the SeedVR2 widths 2560, 3072, 5120,
    10240 and 3456 are).  The reference computes any width
    (shared_linear.cpp:83-96); here the forward returns -1."""
    w = np.zeros(16 * 12, np.float32)
    layer = Layer("SharedLinear", "0=16 1=12 2=0", [w])
    assert layer.create_code == 0
    outs = [((4, 16), np.float32), ((2, 16), np.float32)]
    assert layer.forward([np.zeros((4, 12), np.float32), np.zeros((2, 12), np.float32)],
                         outs)[0] == -1


def test_awa_c_abi_rejects_row_strides_not_a_multiple_of_8():
    """Stated deviation of the C-ABI (the layers always pass strides of
    heads * head_dim or 3 * heads * head_dim, multiples of 8): q/k/v rows are
    read as 16-byte chunks, so a row stride that is not a multiple of 8
    elements returns S2_ERR_INVALID before any device work."""
    L = capi.lib()
    dummy = ctypes.c_void_p(256)
    for vstride, tstride in ((3 * 128 * 2 + 4, 3 * 128 * 2), (3 * 128 * 2, 3 * 128 * 2 + 2)):
        assert L.s2_awa_forward(dummy, dummy, dummy, dummy, dummy, dummy, vstride, dummy, dummy,
                                dummy, tstride, 1, dummy, dummy, 1, dummy, 1 << 20,
                                None) == capi.S2_ERR_INVALID


def test_param_text_parser_accepts_ncnn_fields():
    # float in exponent form and an int id beyond the layer's range are fine
    layer = Layer("AdaptiveWindowAttention", "0=2 1=64 6=1.000000e-05 7=10 9=1 30=5",
                  _awa_weights())
    assert layer.create_code == 0
    bad = Layer("SharedLinear", "0=x")
    assert bad.create_code == -1


def test_awa_one_dim_text_length_blob_reads_column_zero_for_every_sample():
    # The reference reads text_lengths[sample] = read_shape_value(blob, sample, 0)
    # (adaptive_window_attention.cpp:812, :475-485): a 1-D blob of width B
    # answers column 0 for every sample, so batches need a [B][1] blob.
    layer = _awa()
    video = np.zeros((16 + 4, 3 * INNER), np.float32)
    text = np.zeros((3 + 2, 3 * INNER), np.float32)
    shapes = np.asarray([[1, 4, 4], [1, 2, 2]], np.float32)
    outs = [((20, INNER), np.float32), ((5, INNER), np.float32)]
    one_dim = layer.forward([video, text, shapes, np.asarray([3, 2], np.float32)], outs)[0]
    assert one_dim == -1          # lengths read as (3, 3): 6 text rows expected, 5 given
    two_dim = layer.forward([video, text, shapes, np.asarray([[3], [2]], np.float32)], outs)[0]
    assert two_dim in (0, -100)
