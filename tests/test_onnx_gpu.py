"""The reference's ONNX model files through the device Session: tbn.Model(path)
(the reference's Python Model, tbn-runtime/python/bindings.cpp:53-110, over
the C++ reader) against the CPU executor (models.run_oracle) run on the
weights decoded by the independent codec (onnx_proto.py).

Both modes: F32 (use_quantization=False) and the reference Session's
quantized branches (use_quantization=True).  Tolerance as for every fp32
path: rel-L2 <= 1e-5 and max-abs <= 1e-4 * sqrt(K) * max|x| for the last
layer's K and input."""
import os

import numpy as np
import pytest

import models
import onnx_proto as op
import refmath as rm

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "onnx")

# model -> (input seed, input distribution, last layer's K, the value feeding it)
CASES = {
    "simple_matmul": (1, "normal", 4, "X"),
    "simple_conv": (2, "normal", 27, "X"),
    "simple_mlp": (3, "normal", 32, "temp3"),
    "binary_weights": (4, "normal", 8, "X"),
    "ternary_weights": (5, "normal", 8, "X"),
    "simple_cnn": (6, "uniform", 84, "relu_3"),
    "mnist_tbn": (5, "uniform", 512, "view"),
}


def _input(shape, seed, dist):
    rng = np.random.default_rng(seed)
    x = rng.random(shape) if dist == "uniform" else rng.standard_normal(shape)
    return x.astype(np.float32)


def _mnist_thresholds_clear(orc, decoded, rec, quant):
    """The +-0.5 comparisons after conv2 cannot flip under fp32 rounding:
    every conv2 output is further from +-0.5 than K * 2^-23 * sum|terms|."""
    w = decoded["inits"]["conv2_w"]
    b = decoded["inits"]["conv2_b"]
    mags = np.ones_like(w) if quant else np.abs(w)
    terms = orc.conv2d_f64(np.abs(rec["max_pool2d"]), mags.astype(np.float32), None, (1, 1), (2, 2), (1, 1))
    terms = terms + np.abs(b)[None, :, None, None]
    margin = np.abs(np.abs(rec["conv2d_1"].astype(np.float64)) - 0.5)
    assert np.all(margin > 400 * 2.0 ** -23 * terms)


@pytest.mark.parametrize("quant", [False, True])
@pytest.mark.parametrize("name", list(CASES))
def test_reference_onnx_model(dev, tbn, orc, name, quant):
    seed, dist, K, feed = CASES[name]
    path = os.path.join(GOLDEN, name + ".onnx")
    decoded = op.load(path)
    spec = models.spec_from_onnx(decoded)
    (in_name, shape), = spec.inputs.items()
    (out_name, _), = spec.outputs.items()
    x = _input(shape, seed, dist)
    rec = {}
    ref = models.run_oracle(spec, {in_name: x}, quant, orc, record=rec)[out_name]
    if name == "mnist_tbn":
        _mnist_thresholds_clear(orc, decoded, rec, quant)
    model = tbn.Model(path)
    print("%s quant=%s: input %s %s" % (name, quant, in_name, shape), flush=True)
    out = model.run(x, use_quantization=quant)
    assert out.shape == ref.shape and np.all(np.isfinite(out))
    rm.assert_within_tolerance(out, ref, K, np.abs(rec[feed]).max())
    again = model.run(x, use_quantization=quant)  # the same Session, second run
    assert np.array_equal(out, again)


def test_buffer_and_file_loads_agree(dev, tbn):
    path = os.path.join(GOLDEN, "simple_cnn.onnx")
    x = _input([1, 1, 28, 28], 11, "uniform")
    a = tbn.Model(path).run(x)
    p = tbn.OnnxParser()
    p.parse_from_buffer(open(path, "rb").read(), GOLDEN)
    s = tbn.TBNModel(p.get_graph()).create_session()
    s.set_input("input", x)
    s.run()
    assert np.array_equal(a, s.get_output("output"))
