"""The ncnn built-in layers of exported graphs on device blobs (the C-ABI's
s2_binary_op, s2_unary_op, s2_reduce, s2_rms_norm, s2_copy_2d and the
single-stream s2_shared_linear_forward behind Gemm), through ncnn::Net with a
device blob allocator, against the same graphs run on the host
(tests/test_graph_builtins.py holds those to numpy) and, for Gemm, against
the fp32 product of the bf16-rounded operands.  Inputs come both as host
blobs (uploaded by the extractor) and as device fp32 / bf16 tensors."""
import numpy as np
import pytest

import graph_ops as G
from common import bf16_round

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(31)


def _x(*shape, lo=-2.0, hi=2.0):
    return RNG.uniform(lo, hi, shape).astype(np.float32)


def _both(layers, model, inputs, outs, rtol=4e-6, atol=1e-6, dev_inputs=None):
    """Runs the graph on the host and on the device; returns the device results."""
    text = G.param(layers)
    ret_h, host = G.run(text, model, inputs, outs)
    assert ret_h == 0
    ret_d, dev = G.run(text, model, dev_inputs if dev_inputs is not None else inputs, outs, device=True)
    assert ret_d == 0
    for k in outs:
        assert dev[k].shape == host[k].shape, k
        np.testing.assert_allclose(dev[k], host[k], rtol=rtol, atol=atol, err_msg=k)
    return dev


@pytest.mark.parametrize("op", range(12))
@pytest.mark.parametrize("bshape", [(64, 96), (96,), (64, 1)])
def test_binary_op(op, bshape):
    pos = op in (6, 9)
    a = _x(64, 96, lo=0.5 if pos else -2)
    b = _x(*bshape, lo=0.5 if pos else -2)
    layers = [("Input", "a", [], ["a"], ""), ("Input", "b", [], ["b"], ""),
              ("BinaryOp", "op", ["a", "b"], ["y"], f"0={op}"),
              ("BinaryOp", "op2", ["b", "a"], ["y2"], f"0={op}"),
              ("BinaryOp", "op3", ["a"], ["y3"], f"0={op} 1=1 2=1.500000e+00")]
    _both(layers, b"", {"a": a, "b": b}, {"y": a.size, "y2": a.size, "y3": a.size})


def test_binary_op_on_bf16_device_blobs():
    import torch
    a = bf16_round(_x(33, 80))
    b = bf16_round(_x(80))
    layers = [("Input", "a", [], ["a"], ""), ("Input", "b", [], ["b"], ""),
              ("BinaryOp", "op", ["a", "b"], ["y"], "0=2")]
    ret, dev = G.run(G.param(layers), b"", {"a": torch.from_numpy(a).cuda().to(torch.bfloat16),
                                            "b": torch.from_numpy(b).cuda()}, {"y": a.size},
                     device=True)
    assert ret == 0
    # the output takes the bf16 full-shape operand's type
    np.testing.assert_array_equal(dev["y"], bf16_round(a * b))


@pytest.mark.parametrize("op", list(range(20)) + ["Sigmoid", "Swish"])
def test_unary_ops(op):
    lo, hi = (0.1, 0.9) if op in (5, 6, 8, 12, 13, 17) else (-3, 3)
    x = _x(50, 70, lo=lo, hi=hi)
    if op == 18:
        x[0, :4] = [0.5, 1.5, 2.5, -0.5]
    layer = ("UnaryOp", "u", ["x"], ["y"], f"0={op}") if isinstance(op, int) else (op, "u", ["x"], ["y"], "")
    _both([("Input", "x", [], ["x"], ""), layer], b"", {"x": x}, {"y": x.size})


@pytest.mark.parametrize("op", range(11))
@pytest.mark.parametrize("axes, keep", [("-1", 1), ("0", 0), (None, 1)])
def test_reduction(op, axes, keep):
    x = _x(300, 257, lo=0.9, hi=1.1)   # products and exp sums stay finite
    params = f"0={op} 2=1.500000e+00 4={keep} 5=1" + (f" 1=0 -23303=1,{axes}" if axes else " 1=1")
    # device sums run in a different order than the host's: relative 1e-5
    _both([("Input", "x", [], ["x"], ""), ("Reduction", "r", ["x"], ["y"], params)], b"", {"x": x},
          {"y": x.size}, rtol=2e-5, atol=1e-5)


@pytest.mark.parametrize("affine", [0, 1])
def test_rms_norm(affine):
    x = _x(333, 2560)
    gamma = _x(2560, lo=0.5, hi=1.5)
    _both([("Input", "x", [], ["x"], ""), ("RMSNorm", "n", ["x"], ["y"], f"0=2560 1=1.000000e-05 2={affine}")],
          G.fp32(gamma) if affine else b"", {"x": x}, {"y": x.size}, rtol=1e-5, atol=1e-5)


def test_memory_data_reshape_slice_concat_crop():
    v = _x(96)
    x = _x(40, 96)
    layers = [("Input", "x", [], ["x"], ""), ("MemoryData", "v", [], ["v"], "0=96"),
              ("BinaryOp", "add", ["x", "v"], ["s"], "0=0"),
              ("Reshape", "r", ["s"], ["s2"], "0=48 1=-1"),
              ("Slice", "sl", ["s2"], ["p0", "p1", "p2"], "-23300=3,10,-233,-233 1=1"),
              ("Concat", "c", ["p2", "p0", "p1"], ["y"], "0=1"),
              ("Crop", "cr", ["y"], ["z"], "-23309=2,3,5 -23310=2,-4,40 -23311=2,0,1")]
    outs = {"s2": x.size, "p0": x.size, "p1": x.size, "p2": x.size, "y": x.size, "z": x.size}
    _both(layers, G.fp32(v), {"x": x}, outs, rtol=0, atol=0)


@pytest.mark.parametrize("transB", [0, 1])
@pytest.mark.parametrize("ctype", [-1, 0, 4])
def test_gemm_on_the_matrix_cores(transB, ctype):
    """Device Gemm is the SharedLinear GEMM with one token stream: bf16
    operands, fp32 accumulation, beta C as the bias."""
    import torch
    M, K, N = 777, 320, 448
    a = _x(M, K)
    w = _x(N, K, lo=-0.1, hi=0.1)
    c = _x(N if ctype == 4 else 1)
    model = G.tagged(w if transB else w.T.copy()) + (G.tagged(c) if ctype != -1 else b"")
    params = f"1=5.000000e-01 3={transB} 5=1 6={1 if ctype != -1 else 0} 8={N} 9={K} 10={ctype}"
    layers = [("Input", "a", [], ["a"], ""), ("Gemm", "g", ["a"], ["y"], params)]
    text = G.param(layers)
    want = bf16_round(a).astype(np.float64) @ bf16_round(w).T.astype(np.float64)
    if ctype != -1:
        want = want + 0.5 * c
    for inp in ({"a": a}, {"a": torch.from_numpy(a).cuda()}):
        ret, dev = G.run(text, model, inp, {"y": M * N}, device=True)
        assert ret == 0
        np.testing.assert_allclose(dev["y"], want, rtol=1e-4, atol=1e-4)
    # bf16 activations in, bf16 out
    ret, dev = G.run(text, model, {"a": torch.from_numpy(a).cuda().to(torch.bfloat16)}, {"y": M * N},
                     device=True)
    assert ret == 0
    np.testing.assert_allclose(dev["y"], want, rtol=1e-2, atol=1e-2)


def test_gemm_with_alpha_is_refused_on_the_device():
    text = G.param([("Input", "a", [], ["a"], ""), ("Gemm", "g", ["a"], ["y"], "0=2.0 3=1 5=1 8=8 9=64")])
    ret, _ = G.run(text, G.tagged(np.zeros((8, 64), np.float32)), {"a": _x(4, 64)}, {"y": 32},
                   device=True)
    assert ret == -1
