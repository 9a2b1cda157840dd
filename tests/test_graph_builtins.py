"""The ncnn built-in layers of exported graphs (csrc/ncnn/builtin_layers.cpp)
on host blobs, through ncnn::Net, against numpy: MemoryData, BinaryOp (all
twelve op types, numpy broadcasting, the scalar form), UnaryOp (all twenty),
Sigmoid, Swish, Reduction (eleven operations, last / first / all axes,
keepdims), RMSNorm, Reshape, Slice, Concat, Crop and Gemm (both B layouts,
the C broadcast types, alpha and beta, fp16-tagged weights).  Their ParamDict
ids, defaults and weight layouts are ncnn's; the reference loads graphs of
these layers at src/seedvr2/seedvr2_dit.cpp:603-633.  The device paths are
tests/test_gpu_graph_builtins.py."""
import numpy as np
import pytest

import graph_ops as G

RNG = np.random.default_rng(20)


def _x(*shape, lo=-2.0, hi=2.0):
    return RNG.uniform(lo, hi, shape).astype(np.float32)


def _run1(layers, model, inputs, out, count):
    ret, res = G.run(G.param(layers), model, inputs, {out: count})
    assert ret == 0, ret
    return res[out]


BINARY = {0: np.add, 1: np.subtract, 2: np.multiply, 3: np.divide, 4: np.maximum, 5: np.minimum,
          6: np.power, 7: lambda a, b: b - a, 8: lambda a, b: b / a, 9: lambda a, b: np.power(b, a),
          10: np.arctan2, 11: lambda a, b: np.arctan2(b, a)}


@pytest.mark.parametrize("op", range(12))
@pytest.mark.parametrize("bshape", [(4, 6), (6,), (1, 6), (4, 1)])
def test_binary_op_broadcasts_numpy_style(op, bshape):
    pos = op in (6, 9)   # powers of positive bases
    a = _x(4, 6, lo=0.5 if pos else -2, hi=2)
    b = _x(*bshape, lo=0.5 if pos else -2, hi=2)
    layers = [("Input", "a", [], ["a"], ""), ("Input", "b", [], ["b"], ""),
              ("BinaryOp", "op", ["a", "b"], ["y"], f"0={op}")]
    y = _run1(layers, b"", {"a": a, "b": b}, "y", 24)
    np.testing.assert_allclose(y, BINARY[op](a, b), rtol=2e-6, atol=1e-6)
    # the broadcast operand first
    layers[-1] = ("BinaryOp", "op", ["b", "a"], ["y"], f"0={op}")
    y = _run1(layers, b"", {"a": a, "b": b}, "y", 24)
    np.testing.assert_allclose(y, BINARY[op](np.broadcast_to(b, a.shape), a), rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("op", [0, 1, 2, 3, 6, 7])
def test_binary_op_with_scalar(op):
    a = _x(3, 5, lo=0.5, hi=2)
    layers = [("Input", "a", [], ["a"], ""),
              ("BinaryOp", "op", ["a"], ["y"], f"0={op} 1=1 2=1.250000e+00")]
    y = _run1(layers, b"", {"a": a}, "y", 15)
    np.testing.assert_allclose(y, BINARY[op](a, np.float32(1.25)), rtol=2e-6)


def test_binary_op_rejects_shapes_that_do_not_broadcast():
    layers = [("Input", "a", [], ["a"], ""), ("Input", "b", [], ["b"], ""),
              ("BinaryOp", "op", ["a", "b"], ["y"], "0=0")]
    ret, _ = G.run(G.param(layers), b"", {"a": _x(4, 6), "b": _x(5)}, {"y": 24})
    assert ret == -1


UNARY = {0: np.abs, 1: np.negative, 2: np.floor, 3: np.ceil, 4: np.square, 5: np.sqrt,
         6: lambda x: 1 / np.sqrt(x), 7: np.exp, 8: np.log, 9: np.sin, 10: np.cos, 11: np.tan,
         12: np.arcsin, 13: np.arccos, 14: np.arctan, 15: lambda x: 1 / x, 16: np.tanh,
         17: np.log10, 18: np.rint, 19: np.trunc}


@pytest.mark.parametrize("op", range(20))
def test_unary_op(op):
    lo, hi = (0.1, 0.9) if op in (5, 6, 8, 12, 13, 17) else (-3, 3)
    x = _x(3, 7, lo=lo, hi=hi)
    if op == 18:
        x[0, :4] = [0.5, 1.5, 2.5, -0.5]   # ties go to even
    y = _run1([("Input", "x", [], ["x"], ""), ("UnaryOp", "u", ["x"], ["y"], f"0={op}")], b"",
              {"x": x}, "y", 21)
    np.testing.assert_allclose(y, UNARY[op](x.astype(np.float64)), rtol=3e-6, atol=1e-6)


@pytest.mark.parametrize("kind", ["Sigmoid", "Swish"])
def test_sigmoid_and_swish(kind):
    x = _x(64, lo=-9, hi=9)
    y = _run1([("Input", "x", [], ["x"], ""), (kind, "u", ["x"], ["y"], "")], b"", {"x": x}, "y", 64)
    s = 1 / (1 + np.exp(-x.astype(np.float64)))
    np.testing.assert_allclose(y, s if kind == "Sigmoid" else x * s, rtol=2e-6, atol=1e-7)


def _np_reduce(op, x, axis, keepdims, coeff):
    x = x.astype(np.float64)
    f = {0: lambda a: np.sum(a, axis, keepdims=keepdims),
         1: lambda a: np.sum(np.abs(a), axis, keepdims=keepdims),
         2: lambda a: np.sum(a * a, axis, keepdims=keepdims),
         3: lambda a: np.mean(a, axis, keepdims=keepdims),
         4: lambda a: np.max(a, axis, keepdims=keepdims),
         5: lambda a: np.min(a, axis, keepdims=keepdims),
         6: lambda a: np.prod(a, axis, keepdims=keepdims),
         7: lambda a: np.sum(np.abs(a), axis, keepdims=keepdims),
         8: lambda a: np.sqrt(np.sum(a * a, axis, keepdims=keepdims)),
         9: lambda a: np.log(np.sum(a, axis, keepdims=keepdims)),
         10: lambda a: np.log(np.sum(np.exp(a), axis, keepdims=keepdims))}[op]
    return f(x) * coeff


@pytest.mark.parametrize("op", range(11))
@pytest.mark.parametrize("axes, keep", [("-1", 1), ("1", 0), ("0", 1), ("-2", 0), (None, 0), (None, 1)])
def test_reduction(op, axes, keep):
    x = _x(5, 9, lo=0.5, hi=1.5)   # positive: logsum and prod stay finite
    params = f"0={op} 2=1.500000e+00 4={keep} 5=1" + (f" 1=0 -23303=1,{axes}" if axes else " 1=1")
    y = _run1([("Input", "x", [], ["x"], ""), ("Reduction", "r", ["x"], ["y"], params)], b"",
              {"x": x}, "y", 45)
    axis = None if axes is None else int(axes)
    want = _np_reduce(op, x, axis, bool(keep), 1.5)
    if axis is None and keep:
        want = want.reshape(1, 1)
    np.testing.assert_allclose(y, np.asarray(want, np.float32).reshape(y.shape), rtol=5e-6, atol=1e-6)
    assert y.shape == np.shape(want) or (axis is None and y.size == 1)


def test_reduction_legacy_axes_are_refused():
    # fixbug0 = 0 with explicit axes: ncnn's legacy axis numbering, not run here
    layers = [("Input", "x", [], ["x"], ""), ("Reduction", "r", ["x"], ["y"], "0=3 1=0 -23303=1,-1")]
    ret, _ = G.run(G.param(layers), b"", {"x": _x(2, 3)}, {"y": 6})
    assert ret == -1


@pytest.mark.parametrize("affine", [0, 1])
def test_rms_norm(affine):
    x = _x(7, 48)
    gamma = _x(48, lo=0.5, hi=1.5)
    params = f"0=48 1=1.000000e-05 2={affine}"
    y = _run1([("Input", "x", [], ["x"], ""), ("RMSNorm", "n", ["x"], ["y"], params)],
              G.fp32(gamma) if affine else b"", {"x": x}, "y", 7 * 48)
    xd = x.astype(np.float64)
    want = xd / np.sqrt(np.mean(xd * xd, -1, keepdims=True) + 1e-5) * (gamma if affine else 1)
    np.testing.assert_allclose(y, want, rtol=2e-6, atol=1e-6)


def test_memory_data_and_reshape():
    v = _x(12)
    m = _x(3, 4)
    layers = [("MemoryData", "v", [], ["v"], "0=12"), ("MemoryData", "m", [], ["m"], "0=4 1=3"),
              ("Reshape", "r1", ["v"], ["v2"], "0=4 1=-1"), ("Reshape", "r2", ["m"], ["m1"], "0=-1"),
              ("BinaryOp", "add", ["v2", "m"], ["y"], "0=0")]
    ret, res = G.run(G.param(layers), G.fp32(v, m), {}, {"y": 12, "m1": 12, "v2": 12})
    assert ret == 0
    np.testing.assert_array_equal(res["v2"], v.reshape(3, 4))
    np.testing.assert_array_equal(res["m1"], m.reshape(-1))
    np.testing.assert_array_equal(res["y"], v.reshape(3, 4) + m)


@pytest.mark.parametrize("axis", [0, 1, -1])
def test_slice_and_concat(axis):
    x = _x(6, 10)
    ax = axis % 2
    n = x.shape[ax]
    sizes = [2, -233, -233] if ax == 0 else [3, 2, -233]   # -233: an even share of the rest
    layers = [("Input", "x", [], ["x"], ""),
              ("Slice", "s", ["x"], ["p0", "p1", "p2"], f"-23300=3,{','.join(map(str, sizes))} 1={axis}"),
              ("Concat", "c", ["p2", "p0", "p1"], ["y"], f"0={axis}")]
    ret, res = G.run(G.param(layers), b"", {"x": x}, {"p0": 60, "p1": 60, "p2": 60, "y": 60})
    assert ret == 0
    first = 2 if ax == 0 else 3
    second = (n - first) // 2 if ax == 0 else 2
    parts = np.split(x, [first, first + second], axis=ax)
    for i in range(3):
        np.testing.assert_array_equal(res[f"p{i}"], parts[i])
    np.testing.assert_array_equal(res["y"], np.concatenate([parts[2], parts[0], parts[1]], axis=ax))
    # split points instead of sizes
    layers[1] = ("Slice", "s", ["x"], ["p0", "p1", "p2"], f"-23302=2,2,-1 1={axis}")
    ret, res = G.run(G.param(layers), b"", {"x": x}, {"p0": 60, "p1": 60, "p2": 60})
    assert ret == 0
    parts = np.split(x, [2, n - 1], axis=ax)
    for i in range(3):
        np.testing.assert_array_equal(res[f"p{i}"], parts[i])


def test_crop():
    x = _x(8, 12)
    layers = [("Input", "x", [], ["x"], ""),
              ("Crop", "c1", ["x"], ["y1"], "-23309=2,1,3 -23310=2,-2,100 -23311=2,0,1"),
              ("Crop", "c2", ["x"], ["y2"], "-23309=1,4 -23310=1,9 -23311=1,-1"),
              ("Crop", "c3", ["x"], ["y3"], "0=2 1=1 3=5 4=3"),
              ("Crop", "c4", ["x"], ["y4"], "0=1 1=2 6=3 7=1")]
    ret, res = G.run(G.param(layers), b"", {"x": x}, {f"y{i}": 96 for i in range(1, 5)})
    assert ret == 0
    np.testing.assert_array_equal(res["y1"], x[1:-2, 3:])
    np.testing.assert_array_equal(res["y2"], x[:, 4:9])
    np.testing.assert_array_equal(res["y3"], x[1:4, 2:7])
    np.testing.assert_array_equal(res["y4"], x[2:7, 1:9])


@pytest.mark.parametrize("transB", [0, 1])
@pytest.mark.parametrize("ctype", [-1, 0, 4])
@pytest.mark.parametrize("fp16", [False, True])
def test_gemm(transB, ctype, fp16):
    M, K, N = 5, 16, 7
    a = _x(M, K)
    w = _x(N, K)          # [N][K]
    c = _x(N if ctype == 4 else 1)
    alpha, beta = 1.0, 0.5
    bmat = w if transB else w.T.copy()
    model = G.tagged(bmat, fp16=fp16) + (G.tagged(c, fp16=fp16) if ctype != -1 else b"")
    if fp16:
        w = w.astype(np.float16).astype(np.float32)
        c = c.astype(np.float16).astype(np.float32)
    params = (f"0={alpha:e} 1={beta:e} 3={transB} 5=1 6={1 if ctype != -1 else 0} 8={N} 9={K} "
              f"10={ctype}")
    y = _run1([("Input", "a", [], ["a"], ""), ("Gemm", "g", ["a"], ["y"], params)], model, {"a": a},
              "y", M * N)
    want = alpha * (a.astype(np.float64) @ w.T.astype(np.float64))
    if ctype != -1:
        want = want + beta * c
    np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-5)


def test_gemm_refuses_forms_it_does_not_run():
    for params in ("3=1 5=0 8=4 9=8", "2=1 3=1 5=1 8=4 9=8", "3=1 4=1 5=1 8=4 9=8", "3=1 5=1 8=4 9=8 14=1"):
        ret, _ = G.run(G.param([("Input", "a", [], ["a"], ""), ("Gemm", "g", ["a"], ["y"], params)]),
                       G.tagged(np.zeros(32, np.float32)), {"a": _x(2, 8)}, {"y": 8})
        assert ret == -1, params
