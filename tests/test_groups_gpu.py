"""Grouped / depthwise convolution and BatchNormalization on the GPU against
the oracle executor (tests/models.py, itself pinned against torch's CPU
routines in test_groups_cpu.py).  The reference throws for groups > 1
(conv2d.cpp:372-393) and has no BatchNormalization, so the semantics are the
textbook ones: the quantized Session rules (sign(w) * mean|w| per output
channel, or w > 0 with no scale) apply to grouped weights as to dense ones.
Tolerance as for every fp32 path: rel-L2 <= 1e-5 and max-abs <= 1e-4 *
sqrt(K) * max|x| for the last layer's K and input."""
import ctypes
import os

import numpy as np
import pytest
import torch

import models
import onnx_proto as op
import refmath as rm
import tbn_hip
from gpu_util import P, empty, host, to_dev
from models import Node, Spec

pytestmark = pytest.mark.gpu


# ---- C ABI -------------------------------------------------------------------------------

@pytest.mark.parametrize("flags,with_scale,with_res", [(0, False, False), (tbn_hip.EPI_RELU, True, False),
                                                       (tbn_hip.EPI_BIAS_THEN_SCALE, True, True),
                                                       (tbn_hip.EPI_BIAS_THEN_SCALE | tbn_hip.EPI_RELU, True, True)])
def test_depthwise_entry_point_epilogues(dev, orc, flags, with_scale, with_res):
    rng = np.random.default_rng(flags * 4 + with_scale * 2 + with_res)
    n, c, h, w, mult, k = 2, 24, 37, 70, 2, 3
    x = rng.standard_normal((n, c, h, w)).astype(np.float32)
    wt = np.where(rng.random((c * mult, 1, k, k)) < 0.5, -1.0, 1.0).astype(np.float32)
    scale = rng.uniform(0.5, 1.5, c * mult).astype(np.float32)
    bias = rng.standard_normal(c * mult).astype(np.float32)
    d = tbn_hip.conv_desc(n, c, h, w, c * mult, k, k, 2, 1, 1, 2)
    oh, ow = (h + 2 - k) // 2 + 1, (w + 4 - k) // 1 + 1
    res = rng.standard_normal((n, c * mult, oh, ow)).astype(np.float32)
    y = empty((n, c * mult, oh, ow), torch.float32)
    tbn_hip.call("tbn_hip_conv2d_depthwise", P(to_dev(x)), ctypes.byref(d), P(to_dev(wt)),
                 P(to_dev(scale)) if with_scale else None, 0.75, P(to_dev(bias)),
                 P(to_dev(res)) if with_res else None, flags, P(y), None)
    acc = models._Grouped(orc, c).conv2d_f64(x, wt, None, (2, 1), (1, 2), (1, 1))
    s = 0.75 * (scale.astype(np.float64) if with_scale else 1.0)
    b = bias.astype(np.float64)[None, :, None, None]
    s = np.broadcast_to(s, (c * mult,))[None, :, None, None]
    ref = (acc + b) * s if flags & tbn_hip.EPI_BIAS_THEN_SCALE else acc * s + b
    if with_res:
        ref = ref + res
    if flags & tbn_hip.EPI_RELU:
        ref = np.maximum(ref, 0)
    rm.assert_within_tolerance(host(y), ref, k * k, np.abs(x).max() * 1.5)


@pytest.mark.parametrize("stride,h,w,mult,flags", [(1, 13, 11, 1, tbn_hip.EPI_RELU), (2, 14, 14, 2, 0),
                                                   (1, 56, 56, 1, tbn_hip.EPI_BIAS_THEN_SCALE),
                                                   (2, 29, 30, 1, tbn_hip.EPI_RELU), (1, 27, 28, 2, tbn_hip.EPI_RELU),
                                                   (1, 6, 256, 1, 0), (1, 9, 8, 1, tbn_hip.EPI_BIAS_THEN_SCALE),
                                                   (1, 14, 14, 1, tbn_hip.EPI_RELU), (2, 15, 17, 1, tbn_hip.EPI_RELU),
                                                   (1, 5, 300, 1, 0), (2, 56, 112, 1, tbn_hip.EPI_RELU)])
def test_depthwise_3x3_register_blocked(dev, orc, stride, h, w, mult, flags):
    """The 3x3 kernels: the row kernel (stride 1, or 2 on even widths; 4, 2
    or 1 output columns per lane; several row groups and planes per wave,
    partial row groups) and the 4x4-patch kernel (odd widths at stride 2,
    rows wider than 256); residual throughout."""
    rng = np.random.default_rng(stride * 100 + h)
    n, c = 3, 20
    x = rng.standard_normal((n, c, h, w)).astype(np.float32)
    wt = rng.standard_normal((c * mult, 1, 3, 3)).astype(np.float32)
    scale = rng.uniform(0.5, 1.5, c * mult).astype(np.float32)
    bias = rng.standard_normal(c * mult).astype(np.float32)
    d = tbn_hip.conv_desc(n, c, h, w, c * mult, 3, 3, stride, stride, 1, 1)
    oh, ow = (h - 1) // stride + 1, (w - 1) // stride + 1
    res = rng.standard_normal((n, c * mult, oh, ow)).astype(np.float32)
    y = empty((n, c * mult, oh, ow), torch.float32)
    tbn_hip.call("tbn_hip_conv2d_depthwise", P(to_dev(x)), ctypes.byref(d), P(to_dev(wt)), P(to_dev(scale)), 1.0,
                 P(to_dev(bias)), P(to_dev(res)), flags, P(y), None)
    acc = models._Grouped(orc, c).conv2d_f64(x, wt, None, (stride, stride), (1, 1), (1, 1))
    s = scale.astype(np.float64)[None, :, None, None]
    b = bias.astype(np.float64)[None, :, None, None]
    ref = ((acc + b) * s if flags & tbn_hip.EPI_BIAS_THEN_SCALE else acc * s + b) + res
    if flags & tbn_hip.EPI_RELU:
        ref = np.maximum(ref, 0)
    rm.assert_within_tolerance(host(y), ref, 9, np.abs(x).max() * 3)


def test_copy_channels_and_channel_affine_exact(dev):
    rng = np.random.default_rng(3)
    src = rng.standard_normal((3, 10, 7, 5)).astype(np.float32)
    dst = empty((3, 6, 7, 5), torch.float32)
    dst.fill_(7.0)
    tbn_hip.call("tbn_hip_copy_channels", P(to_dev(src)), 3, 10, 4, 5, 35, P(dst), 6, 1, None)
    out = host(dst)
    assert np.array_equal(out[:, 1:6], src[:, 4:9]) and np.all(out[:, 0] == 7.0)
    k = rng.standard_normal(10).astype(np.float32)
    t = rng.standard_normal(10).astype(np.float32)
    y = empty(src.shape, torch.float32)
    tbn_hip.call("tbn_hip_channel_affine", P(to_dev(src)), 3, 10, 35, P(to_dev(k)), P(to_dev(t)),
                 tbn_hip.EPI_RELU, P(y), None)
    # one fma per element: the product is exact in float64, then one rounding
    fma = (src.astype(np.float64) * k[None, :, None, None] + t[None, :, None, None]).astype(np.float32)
    assert np.array_equal(host(y), np.maximum(fma, 0))
    src4 = rng.standard_normal((2, 10, 8, 6)).astype(np.float32)  # rows of 48 floats: the float4 path
    y4 = empty(src4.shape, torch.float32)
    tbn_hip.call("tbn_hip_channel_affine", P(to_dev(src4)), 2, 10, 48, P(to_dev(k)), P(to_dev(t)), 0, P(y4), None)
    fma4 = (src4.astype(np.float64) * k[None, :, None, None] + t[None, :, None, None]).astype(np.float32)
    assert np.array_equal(host(y4), fma4)


# ---- operators ----------------------------------------------------------------------------

@pytest.mark.parametrize("n,c,m,g,k,stride,pad", [(1, 32, 32, 32, 3, 1, 1), (3, 16, 32, 16, 3, 2, 1),
                                                  (1, 64, 64, 4, 3, 1, 1), (3, 64, 96, 2, 1, 1, 0),
                                                  (2, 12, 12, 3, 5, 1, 2)])
def test_conv2d_grouped_operator(dev, tbn, orc, n, c, m, g, k, stride, pad):
    rng = np.random.default_rng(n + c + m + g)
    x = rng.standard_normal((n, c, 15, 13)).astype(np.float32)
    w = (rng.standard_normal((m, c // g, k, k)) * 0.2).astype(np.float32)
    b = rng.standard_normal(m).astype(np.float32)
    y = tbn.conv2d(x, w, b, [stride, stride], [pad, pad], [1, 1], g).numpy()
    ref = models._Grouped(orc, g).conv2d_f64(x, w, b, (stride, stride), (pad, pad), (1, 1))
    rm.assert_within_tolerance(y, ref, c // g * k * k, np.abs(x).max() * 0.2 * 4)
    if g == c:
        assert np.array_equal(tbn.depthwise_conv2d(x, w, b, [stride, stride], [pad, pad]).numpy(), y)


def test_batch_norm_operator(dev, tbn, orc):
    rng = np.random.default_rng(9)
    x = rng.standard_normal((2, 6, 5, 5)).astype(np.float32)
    sc, bb, mu = (rng.standard_normal(6).astype(np.float32) for _ in range(3))
    var = (rng.random(6) + 0.2).astype(np.float32)
    y = tbn.batch_norm(x, sc, bb, mu, var, 1e-5).numpy()
    shp = (1, 6, 1, 1)
    ref = (x.astype(np.float64) - mu.reshape(shp)) / np.sqrt(var.astype(np.float64).reshape(shp) + np.float32(1e-5)) \
        * sc.reshape(shp) + bb.reshape(shp)
    rm.assert_within_tolerance(y, ref, 1, np.abs(ref).max())


# ---- Session ----------------------------------------------------------------------------

def _bn_params(rng, c, prefix):
    return {prefix + "_s": rng.uniform(0.5, 1.5, c).astype(np.float32),
            prefix + "_b": rng.standard_normal(c).astype(np.float32) * 0.1,
            prefix + "_m": rng.standard_normal(c).astype(np.float32) * 0.1,
            prefix + "_v": rng.uniform(0.5, 2.0, c).astype(np.float32)}


def separable_block(n=2, c=32, h=14, w=14, mult=1, cout=64, seed=1, dw_dtype="float32", stride=1, dil=1):
    """Depthwise 3x3 (group = C) + BN + Relu, pointwise 1x1 + BN + Relu
    (a MobileNet block), weights He-scaled fp32 or BINARY / TERNARY bytes."""
    rng = np.random.default_rng(seed)
    cm = c * mult
    if dw_dtype == "binary":
        wdw = (rng.random((cm, 1, 3, 3)) < 0.5).astype(np.uint8)
    elif dw_dtype == "ternary":
        wdw = rng.integers(-1, 2, (cm, 1, 3, 3)).astype(np.int8)
    else:
        wdw = (rng.standard_normal((cm, 1, 3, 3)) * np.sqrt(2 / 9)).astype(np.float32)
    inits = {"wdw": wdw, "bdw": rng.standard_normal(cm).astype(np.float32) * 0.1,
             "wpw": (rng.standard_normal((cout, cm, 1, 1)) * np.sqrt(2 / cm)).astype(np.float32)}
    inits.update(_bn_params(rng, cm, "bn1"))
    inits.update(_bn_params(rng, cout, "bn2"))
    dtypes = {k: "float32" for k in inits}
    dtypes["wdw"] = dw_dtype
    oh = (h + 2 * dil - 2 * dil - 1) // stride + 1
    ow = (w + 2 * dil - 2 * dil - 1) // stride + 1
    nodes = [Node("dw", "Conv", ["x", "wdw", "bdw"], ["d"],
                  {"group": c, "pads": [dil] * 4, "strides": [stride, stride], "dilations": [dil, dil]}),
             Node("bn1", "BatchNormalization", ["d", "bn1_s", "bn1_b", "bn1_m", "bn1_v"], ["e"], {"epsilon": 1e-5}),
             Node("r1", "Relu", ["e"], ["f"]),
             Node("pw", "Conv", ["f", "wpw"], ["p"]),
             Node("bn2", "BatchNormalization", ["p", "bn2_s", "bn2_b", "bn2_m", "bn2_v"], ["q"], {"epsilon": 1e-5}),
             Node("r2", "Relu", ["q"], ["y"])]
    shapes = {"d": [n, cm, oh, ow], "e": [n, cm, oh, ow], "f": [n, cm, oh, ow], "p": [n, cout, oh, ow],
              "q": [n, cout, oh, ow], "y": [n, cout, oh, ow]}
    spec = Spec(nodes, inits, dtypes, {"x": [n, c, h, w]}, {"y": shapes["y"]}, shapes)
    x = rng.standard_normal((n, c, h, w)).astype(np.float32)
    return spec, x


def _run(tbn, spec, x, quant):
    s = tbn.TBNModel(models.build_graph(spec, tbn)).create_session()
    s.set_quantization(quant)
    s.set_input("x", x)
    s.run()
    (out,) = spec.outputs
    return s, s.get_output(out)


@pytest.mark.parametrize("dw_dtype,quant", [("float32", False), ("float32", True), ("binary", False),
                                            ("ternary", True)])
def test_separable_block_session(dev, tbn, orc, dw_dtype, quant):
    seed = {"float32": 10, "binary": 20, "ternary": 30}[dw_dtype] + quant
    spec, x = separable_block(dw_dtype=dw_dtype, seed=seed)
    s, out = _run(tbn, spec, x, quant)
    rec = {}
    ref = models.run_oracle(spec, {"x": x}, quant, orc, record=rec)["y"]
    rm.assert_within_tolerance(out, ref, 32, np.abs(rec["f"]).max())
    # both BatchNormalizations fold into their convs and both Relus fuse
    assert s.planned_launches() == 2


@pytest.mark.parametrize("mult,stride,dil", [(2, 2, 1), (1, 1, 2)])
def test_depthwise_multiplier_stride_dilation(dev, tbn, orc, mult, stride, dil):
    spec, x = separable_block(n=3, c=16, h=21, w=19, mult=mult, cout=24, seed=5 + mult, stride=stride, dil=dil)
    for quant in (False, True):
        _, out = _run(tbn, spec, x, quant)
        rec = {}
        ref = models.run_oracle(spec, {"x": x}, quant, orc, record=rec)["y"]
        rm.assert_within_tolerance(out, ref, 16 * mult, np.abs(rec["f"]).max())


def grouped_spec(n, c, m, g, k=3, stride=1, pad=1, h=12, w=12, seed=2, bn=True, wdtype="float32"):
    rng = np.random.default_rng(seed)
    if wdtype == "binary":
        wt = (rng.random((m, c // g, k, k)) < 0.5).astype(np.uint8)
    else:
        wt = (rng.standard_normal((m, c // g, k, k)) * np.sqrt(2 / (c // g * k * k))).astype(np.float32)
    inits = {"w": wt, "b": rng.standard_normal(m).astype(np.float32) * 0.1}
    inits.update(_bn_params(rng, m, "bn"))
    dtypes = {kk: "float32" for kk in inits}
    dtypes["w"] = wdtype
    oh, ow = (h + 2 * pad - k) // stride + 1, (w + 2 * pad - k) // stride + 1
    nodes = [Node("gc", "Conv", ["x", "w", "b"], ["c"], {"group": g, "pads": [pad] * 4, "strides": [stride] * 2})]
    last = "c"
    if bn:
        nodes.append(Node("bn", "BatchNormalization", ["c", "bn_s", "bn_b", "bn_m", "bn_v"], ["e"]))
        last = "e"
    nodes.append(Node("r", "Relu", [last], ["y"]))
    shp = [n, m, oh, ow]
    spec = Spec(nodes, inits, dtypes, {"x": [n, c, h, w]}, {"y": shp}, {"c": shp, "e": shp, "y": shp})
    return spec, rng.standard_normal((n, c, h, w)).astype(np.float32)


@pytest.mark.parametrize("n,c,m,g,stride,wdtype", [(1, 64, 64, 2, 1, "float32"),   # 32 channels/group: patch conv
                                                   (3, 64, 96, 2, 1, "float32"),   # batch 3: gather / scatter
                                                   (2, 16, 32, 4, 2, "float32"),   # 4 channels/group
                                                   (3, 96, 48, 3, 1, "binary")])
def test_grouped_conv_session(dev, tbn, orc, n, c, m, g, stride, wdtype):
    spec, x = grouped_spec(n, c, m, g, stride=stride, seed=n + g, wdtype=wdtype)
    for quant in ((False, True) if wdtype == "float32" else (False,)):
        s, out = _run(tbn, spec, x, quant)
        rec = {}
        ref = models.run_oracle(spec, {"x": x}, quant, orc, record=rec)["y"]
        rm.assert_within_tolerance(out, ref, c // g * 9, np.abs(x).max())
        assert s.planned_launches() == g * (1 if n == 1 else 3)


def test_batchnorm_unfolded_and_standalone(dev, tbn, orc):
    """BN on a graph input (nothing to fold into, Relu fused into the affine
    kernel) and BN after a conv whose output has a second reader."""
    rng = np.random.default_rng(11)
    n, c, h = 2, 8, 9
    inits = {"w": (rng.standard_normal((c, c, 3, 3)) * 0.3).astype(np.float32)}
    inits.update(_bn_params(rng, c, "a"))
    inits.update(_bn_params(rng, c, "b"))
    shp = [n, c, h, h]
    nodes = [Node("bna", "BatchNormalization", ["x", "a_s", "a_b", "a_m", "a_v"], ["xa"]),
             Node("ra", "Relu", ["xa"], ["xr"]),
             Node("cv", "Conv", ["xr", "w"], ["cv_out"], {"pads": [1, 1, 1, 1]}),
             Node("bnb", "BatchNormalization", ["cv_out", "b_s", "b_b", "b_m", "b_v"], ["z"]),
             Node("add", "Add", ["z", "cv_out"], ["y"])]
    spec = Spec(nodes, inits, {k: "float32" for k in inits}, {"x": shp}, {"y": shp},
                {k: shp for k in ("xa", "xr", "cv_out", "z", "y")})
    x = rng.standard_normal(shp).astype(np.float32)
    s, out = _run(tbn, spec, x, False)
    rec = {}
    ref = models.run_oracle(spec, {"x": x}, False, orc, record=rec)["y"]
    rm.assert_within_tolerance(out, ref, c * 9, np.abs(rec["xr"]).max())
    assert s.planned_launches() == 4  # affine+relu, conv, affine, add


def test_mobilenet_style_onnx_model(dev, tbn, orc, tmp_path):
    """A separable block written as an ONNX file (weights in an external data
    file) through tbn.Model(path), both modes."""
    spec, x = separable_block(n=1, c=32, h=16, w=16, cout=48, seed=21)
    blob, inits = b"", []
    for name, arr in spec.inits.items():
        inits.append(op.encode_tensor(name, arr, "external", ("w.bin", len(blob), arr.nbytes)))
        blob += arr.tobytes()
    (tmp_path / "w.bin").write_bytes(blob)
    nodes = [op.encode_node(nd.op, nd.inputs, nd.outputs, nd.name, nd.attrs) for nd in spec.nodes]
    model = op.encode_model(nodes, inits, [op.encode_value_info("x", spec.inputs["x"])],
                            [op.encode_value_info("y", spec.outputs["y"])])
    path = os.path.join(str(tmp_path), "block.onnx")
    with open(path, "wb") as f:
        f.write(model)
    m = tbn.Model(path)
    for quant in (False, True):
        rec = {}
        ref = models.run_oracle(spec, {"x": x}, quant, orc, record=rec)["y"]
        rm.assert_within_tolerance(m.run(x, use_quantization=quant), ref, 32, np.abs(rec["f"]).max())
