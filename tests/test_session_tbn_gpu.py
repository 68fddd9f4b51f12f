"""The Session in TBN arithmetic (QuantArithmetic::TBN): the reference's own
quantized Session, bit for bit, against the CPU executor in tests/models.py
(run_oracle(..., arithmetic="tbn")).

Reference: tbn-runtime/include/tbn/runtime/model.hpp:414-564 (the quantized
conv: cached (float(C) + b) * s, or quantize_to_binary then conv2d_binary's
float(C) + b), :763-870 (the quantized Gemm: float(C) * alpha, then
+= beta * C), conv2d.cpp:195-316; the integers C come from ternarizing the
activations at +-0.1.  Layers the reference keeps in fp32 (MatMul, Gemm with
transB, nodes marked tbn_quantize = 0) are compared within the north_star
tolerance; every value computed only from TBN layers is compared bitwise."""
import os

import numpy as np
import pytest

import models
import tbn_hip
import onnx_proto as op
import refmath as rm

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "onnx")


def _session(tbn, spec, quant=True, replay=False, extra_outputs=()):
    g = models.build_graph(spec, tbn)
    for name in extra_outputs:
        g.add_output(name, list(spec.value_info[name]))
    model = tbn.TBNModel(g)
    model.validate()
    s = model.create_session()
    s.set_quantization(quant)
    s.set_quant_arithmetic("tbn")
    if replay:
        s.set_graph_replay(True)
    return model, s


def _bits_equal(a, b, what):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    assert a.shape == b.shape, what
    diff = np.count_nonzero(a.view(np.uint32) != b.view(np.uint32))
    assert diff == 0, f"{what}: {diff} of {a.size} values differ"


@pytest.mark.parametrize("prebinarized", [True, False])
@pytest.mark.parametrize("replay", [False, True], ids=["eager", "graph"])
def test_lenet_tbn_bit_exact(dev, tbn, orc, prebinarized, replay):
    """Config 1: both convs and the Gemm in TBN arithmetic (the cached conv
    path with prebinarized weights, quantize_to_binary without), so the whole
    forward is exact; graph replay gives the same bits on every replay."""
    spec = models.lenet(seed=1, prebinarized=prebinarized)
    x = models.lenet_input(1)
    _, s = _session(tbn, spec, replay=replay)
    ref = models.run_oracle(spec, {"input": x}, True, orc, arithmetic="tbn")["output"]
    for _ in range(4 if replay else 1):  # eager, capture, replays
        s.set_input("input", x)
        s.run()
        _bits_equal(s.get_output("output"), ref, "lenet output")
    assert s.planned_launches() == 3  # conv+relu+pool twice, then the Gemm


def test_lenet_tbn_differs_from_f32(dev, tbn, orc):
    """The two arithmetics are different computations (ternarized vs fp32
    activations): same Session, switching the arithmetic recompiles."""
    spec = models.lenet(seed=4)
    x = models.lenet_input(4)
    _, s = _session(tbn, spec)
    s.set_input("input", x)
    s.run()
    a = s.get_output("output")
    s.set_quant_arithmetic("f32")
    s.run()
    b = s.get_output("output")
    assert s.quant_arithmetic() == "f32"
    assert not np.array_equal(a, b)
    rm.assert_within_tolerance(b, models.run_oracle(spec, {"input": x}, True, orc)["output"], 256, 10.0)


def test_tbn_gemm_alpha_beta_relu_and_runtime_b(dev, tbn, orc):
    """The quantized Gemm's alpha / beta steps (float(C) * alpha, then one
    fused beta * C), a 2-D C, a fused Relu, and a B supplied at run time
    (packed on every run) -- bit-exact."""
    rng = np.random.default_rng(12)
    M, K, N = 6, 200, 40
    w = np.where(rng.random((K, N)) < 0.5, 1.0, -1.0).astype(np.float32)
    c2 = (rng.standard_normal((M, N)) * 2).astype(np.float32)
    nodes = [models.Node("g1", "Gemm", ["a", "w", "c"], ["y1"], {"alpha": 0.37, "beta": -1.3}),
             models.Node("r", "Relu", ["y1"], ["y2"]),
             models.Node("g2", "Gemm", ["a", "b", "c"], ["y3"], {"alpha": 1.0, "beta": 0.7})]
    spec = models.Spec(nodes, {"w": w, "c": c2}, {"w": "float32", "c": "float32"}, {"a": (M, K), "b": (K, N)},
                       {"y2": (M, N), "y3": (M, N)}, {"y1": (M, N), "y2": (M, N), "y3": (M, N), "a": (M, K),
                                                      "b": (K, N)})
    _, s = _session(tbn, spec)
    for seed in (1, 2):
        r2 = np.random.default_rng(seed)
        a = (r2.standard_normal((M, K)) * 0.2).astype(np.float32)
        b = (r2.standard_normal((K, N))).astype(np.float32)  # not already binary: quantize_to_binary
        feeds = {"a": a, "b": b}
        for k, v in feeds.items():
            s.set_input(k, v)
        s.run()
        ref = models.run_oracle(spec, feeds, True, orc, arithmetic="tbn")
        _bits_equal(s.get_output("y2"), ref["y2"], "alpha/beta + relu")
        _bits_equal(s.get_output("y3"), ref["y3"], "runtime B")


def _resnet_tbn(tbn, orc, batch, check_oracle):
    spec = models.resnet18(batch=batch, seed=5)
    x = models.resnet_input(batch, seed=5)
    _, s = _session(tbn, spec, extra_outputs=("pool_out", "flat"))
    s.set_input("input", x)
    s.run()
    outs = {k: s.get_output(k) for k in ("pool_out", "flat", "logits")}
    if check_oracle:
        # the fp32 stem's device output feeds the oracle's TBN body, so every
        # binary conv, residual add and the average pool are compared bitwise
        rec = {}
        ref = models.run_oracle(spec, {"input": x}, True, orc, record=rec, arithmetic="tbn",
                                overrides={"pool_out": outs["pool_out"]})
        _bits_equal(outs["flat"], rec["flat"], "resnet18 body (GlobalAveragePool output)")
        rm.assert_within_tolerance(outs["logits"], ref["logits"], 512, np.abs(rec["flat"]).max())
    return s, outs


def test_resnet18_tbn_batch2_bit_exact(dev, tbn, orc):
    s, outs = _resnet_tbn(tbn, orc, 2, True)
    # stem(+relu+pool), 16 binary convs with relu or residual fused, 3 projections, gap, fc; a projection
    # runs in its block's first conv's launch where the library takes the pair
    fused = 0
    for c, hw in ((64, 56), (128, 28), (256, 14)):
        d = tbn_hip.conv_desc(2, c, hw, hw, 2 * c, 3, 3, 2, 2, 1, 1)
        try:
            tbn_hip.call("tbn_hip_conv2d_tbn_prepacked_pair", None, d, None, None, 1.0, None, None, tbn_hip.EPI_RELU,
                         -0.1, 0.1, None, None, None, 1.0, None, 0, None, 2, None)
            fused += 1
        except tbn_hip.TbnError as e:
            assert e.code == tbn_hip.NOT_IMPLEMENTED
    assert fused >= 1
    assert s.planned_launches() == 1 + 16 + 3 + 1 + 1 - fused


def test_resnet18_tbn_batch32_batch_invariant(dev, tbn):
    """Config 5 at batch 32 in TBN arithmetic: every sample's values equal
    the same sample's in a batch of 2, bit for bit."""
    _, o32 = _resnet_tbn(tbn, None, 32, False)
    spec2 = models.resnet18(batch=2, seed=5)
    _, s2 = _session(tbn, spec2, extra_outputs=("flat",))
    x32 = models.resnet_input(32, seed=5)
    for i0 in (0, 30):
        s2.set_input("input", x32[i0:i0 + 2].copy())
        s2.run()
        assert np.array_equal(s2.get_output("flat"), o32["flat"][i0:i0 + 2]), f"samples {i0}..{i0 + 1}"
        assert np.array_equal(s2.get_output("logits"), o32["logits"][i0:i0 + 2]), f"samples {i0}..{i0 + 1}"


# ONNX models: (input seed, distribution, the last value computed only by TBN
# layers (bitwise), the last layer's K and input for the tolerance check)
ONNX = {
    "simple_conv": (2, "normal", "Y", None, None),
    "simple_cnn": (6, "uniform", "view", 84, "relu_3"),
    "mnist_tbn": (5, "uniform", "view", 512, "view"),
}


@pytest.mark.parametrize("name", list(ONNX))
def test_reference_onnx_models_tbn(dev, tbn, orc, name):
    """The reference's ONNX models through Model(path, arithmetic="tbn")
    .run_quantized (bindings.cpp:68-96): the TBN part bitwise (an extra
    graph output exposes it), the layers the reference keeps fp32 (Gemm with
    transB) within tolerance."""
    seed, dist, exact_value, K, feed = ONNX[name]
    path = os.path.join(GOLDEN, name + ".onnx")
    spec = models.spec_from_onnx(op.load(path))
    (in_name, shape), = spec.inputs.items()
    (out_name, _), = spec.outputs.items()
    rng = np.random.default_rng(seed)
    x = (rng.random(shape) if dist == "uniform" else rng.standard_normal(shape)).astype(np.float32)
    rec = {}
    ref = models.run_oracle(spec, {in_name: x}, True, orc, record=rec, arithmetic="tbn")[out_name]
    out = tbn.Model(path, arithmetic="tbn").run_quantized(x)
    if exact_value == out_name:
        _bits_equal(out, ref, name)
    else:
        rm.assert_within_tolerance(out, ref, K, np.abs(rec[feed]).max())
        p = tbn.OnnxParser()
        p.parse_from_file(path)
        g = p.get_graph()
        g.add_output(exact_value, list(spec.value_info[exact_value]))
        s = tbn.TBNModel(g).create_session()
        s.set_quantization(True)
        s.set_quant_arithmetic("tbn")
        s.set_input(in_name, x)
        s.run()
        _bits_equal(s.get_output(exact_value), rec[exact_value], f"{name} {exact_value}")
        assert np.array_equal(s.get_output(out_name), out)
