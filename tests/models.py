"""Seeded model graphs for the Session tests and the bench, and the CPU
reference executor that runs them through the oracle.

A graph is described once as plain data (`Spec`) and then either built into
a `_tbn.ModelGraph` (the device path) or executed by `run_oracle` on the CPU
with the oracle's operators, following the reference Session's per-node
semantics (tbn-runtime/include/tbn/runtime/model.hpp:277-1300) in mode F32:
fp32 activations, exact +-1 weights, per-channel scale where the reference
applies one.

Configs:
  lenet     config 1, x[1,1,28,28] ~ U[0,1): Conv 1->6 5x5, Relu, MaxPool 2x2,
            Conv 6->16 5x5, Relu, MaxPool 2x2, Flatten, Gemm 256->10 + bias.
            Weights N(0, 0.1) auto-quantized to sign(w) * mean|w| per output
            channel (`prebinarized=True`, the Session's cached binary path), or
            left raw (`prebinarized=False`, the quantize_to_binary path).
  resnet18  config 5, x[B,3,224,224] ~ N(0,1): fp32 7x7/2 stem + Relu +
            MaxPool 3x3/2 p1, four stages of two basic blocks (64/128/256/512,
            stride-2 3x3 and 1x1 projection at each stage change) whose convs
            are binary (sign(w) * mean|w| per channel, He-scaled w), residual
            Add + Relu, GlobalAveragePool, Flatten, fp32 Gemm 512->1000 + bias.
            The stem and the FC carry the attribute tbn_quantize=0, so a
            Session with quantization on keeps them fp32.
"""
from dataclasses import dataclass, field

import numpy as np


@dataclass
class Node:
    name: str
    op: str
    inputs: list
    outputs: list
    attrs: dict = field(default_factory=dict)


@dataclass
class Spec:
    nodes: list
    inits: dict          # name -> np.ndarray (float32, or uint8 'binary' / int8 'ternary')
    init_dtypes: dict    # name -> tbn dtype string
    inputs: dict         # name -> shape
    outputs: dict        # name -> shape
    value_info: dict     # name -> shape (every node output)


def prebinarize(w):
    """sign(w) * mean|w| per output channel (channel = first dim), float32."""
    w = np.asarray(w, np.float32)
    flat = w.reshape(w.shape[0], -1)
    s = np.abs(flat).mean(axis=1, dtype=np.float64).astype(np.float32)
    return (np.where(flat >= 0, 1.0, -1.0).astype(np.float32) * s[:, None]).reshape(w.shape)


def _out_hw(h, w, k, s, p):
    return (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1


def lenet(seed=1, prebinarized=True):
    rng = np.random.default_rng(seed)
    w1 = (rng.standard_normal((6, 1, 5, 5)) * 0.1).astype(np.float32)
    b1 = (rng.standard_normal(6) * 0.01).astype(np.float32)
    w2 = (rng.standard_normal((16, 6, 5, 5)) * 0.1).astype(np.float32)
    b2 = (rng.standard_normal(16) * 0.01).astype(np.float32)
    wf = (rng.standard_normal((256, 10)) * 0.1).astype(np.float32)
    bf = (rng.standard_normal(10) * 0.01).astype(np.float32)
    if prebinarized:
        w1, w2 = prebinarize(w1), prebinarize(w2)
        # Gemm B is [K, N]: one scale per output column n
        wf = prebinarize(wf.T).T.copy()
    nodes = [
        Node("conv1", "Conv", ["input", "w1", "b1"], ["conv1_out"], {"kernel_shape": [5, 5]}),
        Node("relu1", "Relu", ["conv1_out"], ["relu1_out"]),
        Node("pool1", "MaxPool", ["relu1_out"], ["pool1_out"], {"kernel_shape": [2, 2], "strides": [2, 2]}),
        Node("conv2", "Conv", ["pool1_out", "w2", "b2"], ["conv2_y"], {"kernel_shape": [5, 5]}),
        Node("relu2", "Relu", ["conv2_y"], ["relu2_out"]),
        Node("pool2", "MaxPool", ["relu2_out"], ["pool2_out"], {"kernel_shape": [2, 2], "strides": [2, 2]}),
        Node("flatten", "Flatten", ["pool2_out"], ["flat"], {"axis": 1}),
        Node("fc", "Gemm", ["flat", "wf", "bf"], ["output"], {"alpha": 1.0, "beta": 1.0}),
    ]
    vi = {"conv1_out": (1, 6, 24, 24), "relu1_out": (1, 6, 24, 24), "pool1_out": (1, 6, 12, 12),
          "conv2_y": (1, 16, 8, 8), "relu2_out": (1, 16, 8, 8), "pool2_out": (1, 16, 4, 4),
          "flat": (1, 256), "output": (1, 10), "input": (1, 1, 28, 28)}
    inits = {"w1": w1, "b1": b1, "w2": w2, "b2": b2, "wf": wf, "bf": bf}
    return Spec(nodes, inits, {k: "float32" for k in inits}, {"input": (1, 1, 28, 28)}, {"output": (1, 10)}, vi)


def lenet_input(seed=1):
    return np.random.default_rng(seed + 1000).random((1, 1, 28, 28)).astype(np.float32)


def resnet18(batch=32, seed=5, classes=1000):
    rng = np.random.default_rng(seed)
    nodes, inits, vi = [], {}, {}

    def he(shape):
        fan_in = int(np.prod(shape[1:]))
        return (rng.standard_normal(shape) * np.sqrt(2.0 / fan_in)).astype(np.float32)

    def conv(name, x, cin, cout, k, s, p, h, w, binary=True):
        wname = name + "_w"
        inits[wname] = prebinarize(he((cout, cin, k, k))) if binary else he((cout, cin, k, k))
        attrs = {"kernel_shape": [k, k], "strides": [s, s], "pads": [p, p, p, p]}
        if not binary:
            attrs["tbn_quantize"] = 0
        oh, ow = _out_hw(h, w, k, s, p)
        out = name + "_out"
        nodes.append(Node(name, "Conv", [x, wname], [out], attrs))
        vi[out] = (batch, cout, oh, ow)
        return out, oh, ow

    def relu(name, x):
        out = name + "_out"
        nodes.append(Node(name, "Relu", [x], [out]))
        vi[out] = vi[x]
        return out

    x, h, w = conv("stem", "input", 3, 64, 7, 2, 3, 224, 224, binary=False)
    x = relu("stem_relu", x)
    nodes.append(Node("stem_pool", "MaxPool", [x], ["pool_out"],
                      {"kernel_shape": [3, 3], "strides": [2, 2], "pads": [1, 1, 1, 1]}))
    h, w = _out_hw(h, w, 3, 2, 1)
    vi["pool_out"] = (batch, 64, h, w)
    x, cin = "pool_out", 64
    for stage, cout in enumerate([64, 128, 256, 512]):
        for blk in range(2):
            s = 2 if (stage > 0 and blk == 0) else 1
            pre = f"l{stage + 1}b{blk}"
            y, oh, ow = conv(pre + "_c1", x, cin, cout, 3, s, 1, h, w)
            y = relu(pre + "_r1", y)
            y, oh, ow = conv(pre + "_c2", y, cout, cout, 3, 1, 1, oh, ow)
            if s != 1 or cin != cout:
                sc, _, _ = conv(pre + "_ds", x, cin, cout, 1, s, 0, h, w)
            else:
                sc = x
            nodes.append(Node(pre + "_add", "Add", [y, sc], [pre + "_sum"]))
            vi[pre + "_sum"] = vi[y]
            x = relu(pre + "_r2", pre + "_sum")
            h, w, cin = oh, ow, cout
    nodes.append(Node("gap", "GlobalAveragePool", [x], ["gap_out"]))
    vi["gap_out"] = (batch, 512, 1, 1)
    nodes.append(Node("flatten", "Flatten", ["gap_out"], ["flat"], {"axis": 1}))
    vi["flat"] = (batch, 512)
    inits["fc_w"] = (rng.standard_normal((512, classes)) * np.sqrt(1.0 / 512)).astype(np.float32)
    inits["fc_b"] = (rng.standard_normal(classes) * 0.01).astype(np.float32)
    nodes.append(Node("fc", "Gemm", ["flat", "fc_w", "fc_b"], ["logits"], {"tbn_quantize": 0}))
    vi["logits"] = (batch, classes)
    vi["input"] = (batch, 3, 224, 224)
    return Spec(nodes, inits, {k: "float32" for k in inits}, {"input": (batch, 3, 224, 224)},
                {"logits": (batch, classes)}, vi)


def resnet_input(batch=32, seed=5):
    return np.random.default_rng(seed + 1000).standard_normal((batch, 3, 224, 224)).astype(np.float32)


# ---- building the device graph -------------------------------------------------------

def build_graph(spec, _tbn):
    g = _tbn.ModelGraph()
    for name, shape in spec.inputs.items():
        g.add_input(name, list(shape))
    for name, shape in spec.outputs.items():
        g.add_output(name, list(shape))
    for name, shape in spec.value_info.items():
        g.set_value_info(name, list(shape))
    for name, arr in spec.inits.items():
        g.add_initializer(name, arr, spec.init_dtypes[name])
    for n in spec.nodes:
        g.add_node(n.name, n.op, n.inputs, n.outputs, n.attrs)
    return g


def spec_from_onnx(m):
    """Spec of a model decoded by onnx_proto.decode_model (initializers as
    stored: float32, or int64 for shapes)."""
    nodes = [Node(n["name"], n["op_type"], list(n["inputs"]), list(n["outputs"]), dict(n["attributes"]))
             for n in m["nodes"]]
    inits = dict(m["inits"])
    dtypes = {k: str(v.dtype) for k, v in inits.items()}
    return Spec(nodes, inits, dtypes, {k: m["value_info"][k] for k in m["inputs"]},
                {k: m["value_info"][k] for k in m["outputs"]}, dict(m["value_info"]))


# ---- the CPU reference executor ------------------------------------------------------

def _conv_attrs(attrs):
    s = attrs.get("strides", [1, 1])
    p = attrs.get("pads", [0, 0, 0, 0])
    d = attrs.get("dilations", [1, 1])
    return (s[0], s[1]), (p[0], p[1]), (d[0], d[1])


class _Grouped:
    """The oracle's conv2d_f64 / conv2d_f32 applied group by group: group g
    convolves input channels [g*C/G, (g+1)*C/G) with output channels
    [g*M/G, (g+1)*M/G) of the [M, C/G, kh, kw] weights (the definition of a
    grouped convolution); every other oracle function passes through."""

    def __init__(self, orc, groups):
        self._orc, self._g = orc, groups

    def __getattr__(self, name):
        fn = getattr(self._orc, name)
        if self._g == 1 or name not in ("conv2d_f64", "conv2d_f32"):
            return fn

        def grouped(x, w, bias=None, stride=(1, 1), pad=(0, 0), dil=(1, 1)):
            cg, mg = x.shape[1] // self._g, w.shape[0] // self._g
            outs = [fn(np.ascontiguousarray(x[:, g * cg:(g + 1) * cg]), np.ascontiguousarray(w[g * mg:(g + 1) * mg]),
                       None if bias is None else np.ascontiguousarray(bias[g * mg:(g + 1) * mg]), stride, pad, dil)
                    for g in range(self._g)]
            return np.concatenate(outs, axis=1)
        return grouped


def gemm_already_binary(B):
    """The quantized Gemm's "already binary" test (model.hpp:765-786): the
    flattened B is sampled at i = 0, step, 2*step, ... with step =
    max(1, size // 1000), and every sample must be exactly -1, 1, 0, 0.999
    or -0.999 (fp32 equality, so -0.0 passes as 0)."""
    flat = np.asarray(B, np.float32).reshape(-1)
    step = max(1, flat.size // 1000)
    ok = set(np.float32([-1.0, 1.0, 0.0, 0.999, -0.999]).tolist())
    return all(float(v) in ok for v in flat[::step])


def run_oracle(spec, feeds, quant, orc, record=None, arithmetic="f32", overrides=None):
    """Executes the graph on the CPU (float64 products, fp32 values between
    nodes) with the reference Session's branch structure.  Returns
    {output name: array}; `record`, if a dict, receives every value.

    arithmetic="tbn": the quantized layers in the reference's own arithmetic
    (model.hpp:414-564,763-870; conv2d.cpp:195-316), bit for bit: ternarized
    activations, exact integer products, float(C) and the bias / scale /
    alpha / beta steps in float32 (tests/tbn_ref.py), and residual Adds in
    float32.  `overrides` maps value names to arrays used instead of
    computing the nodes that produce them (to continue from a device value)."""
    import tbn_ref

    tbn = arithmetic == "tbn"
    overrides = overrides or {}
    env = {k: np.asarray(v) for k, v in spec.inits.items()}
    env.update({k: np.asarray(v, np.float32) for k, v in feeds.items()})
    orc_base = orc
    for n in spec.nodes:
        orc = orc_base
        a = n.attrs
        quant_here = quant and a.get("tbn_quantize", 1) != 0
        if n.outputs[0] in overrides:
            env[n.outputs[0]] = np.asarray(overrides[n.outputs[0]], np.float32)
            continue
        if tbn and n.op == "Conv" and int(a.get("group", 1)) == 1:
            dt = spec.init_dtypes.get(n.inputs[1], "float32")
            if dt in ("binary", "ternary") or quant_here:
                x, W = env[n.inputs[0]], env[n.inputs[1]]
                b = env[n.inputs[2]].astype(np.float32) if len(n.inputs) > 2 else None
                stride, pad, dil = _conv_attrs(a)
                scale = None
                if dt == "binary":
                    sign = np.where(W == 1, 1, -1)
                elif dt == "ternary":
                    sign = np.where(W < 0, -1, 1)  # conv2d_ternary (conv2d.cpp:195-217)
                else:
                    s = orc.channel_mean_abs(W)
                    already = orc.already_binary(W, s)
                    sign = np.where(W >= 0 if already else W > 0, 1, -1)
                    scale = s if already else None
                C = tbn_ref.tbn_conv_int(orc, x, sign, stride, pad, dil)
                y = C.astype(np.float32)
                if b is not None:
                    y = y + b[None, :, None, None]
                if scale is not None:
                    y = y * np.asarray(scale, np.float32)[None, :, None, None]
                env[n.outputs[0]] = y.astype(np.float32)
                continue
        if tbn and n.op == "Gemm" and quant_here:
            A, B = env[n.inputs[0]], env[n.inputs[1]]
            if B.dtype == np.float32 and not a.get("transA", 0) and not a.get("transB", 0):
                already = gemm_already_binary(B)
                sign = np.where(B >= 0 if already else B > 0, 1, -1)
                C = env[n.inputs[2]] if len(n.inputs) > 2 else None
                env[n.outputs[0]] = tbn_ref.tbn_gemm_session(orc, A, sign, a.get("alpha", 1.0), C,
                                                             a.get("beta", 1.0))
                continue
        if tbn and n.op == "Add":
            xa, xb = env[n.inputs[0]].astype(np.float32), env[n.inputs[1]].astype(np.float32)
            if xa.ndim == 4 and xb.ndim in (1, 3):
                xb = xb.reshape(1, -1, 1, 1)
            env[n.outputs[0]] = (xa + xb).astype(np.float32)
            continue
        if n.op == "Conv":
            x = env[n.inputs[0]]
            wname = n.inputs[1]
            W = env[wname]
            b = env[n.inputs[2]].astype(np.float64) if len(n.inputs) > 2 else None
            stride, pad, dil = _conv_attrs(a)
            groups = int(a.get("group", 1))
            orc = _Grouped(orc_base, groups)
            dt = spec.init_dtypes.get(wname, "float32")
            if dt == "binary":
                y = orc.conv2d_f64(x, np.where(W == 1, 1.0, -1.0).astype(np.float32), None, stride, pad, dil)
                y = y + (0 if b is None else b[None, :, None, None])
            elif dt == "ternary":
                y = orc.conv2d_f64(x, W.astype(np.float32), None, stride, pad, dil)
                y = y + (0 if b is None else b[None, :, None, None])
            elif quant_here:
                s = orc.channel_mean_abs(W)
                if orc.already_binary(W, s):
                    # model.hpp:414-559: signs w >= 0, (conv + b) * s
                    sign = np.where(W >= 0, 1.0, -1.0).astype(np.float32)
                    y = orc.conv2d_f64(x, sign, None, stride, pad, dil)
                    if b is not None:
                        y = y + b[None, :, None, None]
                    y = y * s.astype(np.float64)[None, :, None, None]
                else:
                    # model.hpp:560-564: quantize_to_binary (w > 0), conv2d_binary, no scale
                    sign = np.where(W > 0, 1.0, -1.0).astype(np.float32)
                    y = orc.conv2d_f64(x, sign, None, stride, pad, dil)
                    if b is not None:
                        y = y + b[None, :, None, None]
            else:
                y = orc.conv2d_f64(x, W, None if b is None else b.astype(np.float32), stride, pad, dil)
        elif n.op in ("Gemm", "MatMul"):
            A = env[n.inputs[0]].astype(np.float64)
            B = env[n.inputs[1]]
            alpha = a.get("alpha", 1.0) if n.op == "Gemm" else 1.0
            beta = a.get("beta", 1.0) if n.op == "Gemm" else 0.0
            tA, tB = bool(a.get("transA", 0)), bool(a.get("transB", 0))
            C = env[n.inputs[2]] if (n.op == "Gemm" and len(n.inputs) > 2) else None
            if quant_here and n.op == "Gemm" and B.dtype == np.float32 and not tA and not tB:
                already = gemm_already_binary(B)
                sign = np.where(B >= 0 if already else B > 0, 1.0, -1.0)
                y = A @ sign
            else:
                y = (A.T if tA else A) @ (B.T if tB else B).astype(np.float64)
            y = y * np.float64(np.float32(alpha))
            if C is not None and beta != 0.0:
                y = y + np.float64(np.float32(beta)) * C.astype(np.float64)
        elif n.op == "Relu":
            x = env[n.inputs[0]]
            if quant and ("conv2d_1" in n.inputs[0] or "conv2_out" in n.inputs[0]):
                y = np.where(x > 0.5, 1.0, np.where(x < -0.5, -1.0, 0.0))
            else:
                y = np.maximum(x, 0)
        elif n.op == "MaxPool":
            k = a.get("kernel_shape", [2, 2])
            s = a.get("strides", k)
            p = a.get("pads", [0, 0, 0, 0])
            y = orc.maxpool2d(env[n.inputs[0]], tuple(k), tuple(s), (p[0], p[1]), ceil_mode=bool(a.get("ceil_mode", 0)))
        elif n.op in ("AveragePool", "AvgPool"):
            # model.hpp:632-682: no ceil_mode, count_include_pad read
            k = a.get("kernel_shape", [2, 2])
            s = a.get("strides", k)
            p = a.get("pads", [0, 0, 0, 0])
            y = orc.avgpool2d(env[n.inputs[0]], tuple(k), tuple(s), (p[0], p[1]),
                              count_include_pad=bool(a.get("count_include_pad", 0)))
        elif n.op in ("GlobalAveragePool", "GlobalAvgPool"):
            x = env[n.inputs[0]]
            y = orc.global_avgpool2d(x).reshape(x.shape[0], x.shape[1], 1, 1)
        elif n.op == "GlobalMaxPool":
            x = env[n.inputs[0]]
            y = orc.global_maxpool2d(x).reshape(x.shape[0], x.shape[1], 1, 1)
        elif n.op == "Flatten":
            x = env[n.inputs[0]]
            ax = a.get("axis", 1)
            y = x.reshape(int(np.prod(x.shape[:ax])), -1)
        elif n.op == "BatchNormalization":
            # ONNX inference form: (x - mean) / sqrt(var + eps) * scale + B over dim 1
            x = env[n.inputs[0]].astype(np.float64)
            sc, bb, mu, var = (env[k].astype(np.float64) for k in n.inputs[1:5])
            shp = (1, -1) + (1,) * (x.ndim - 2)
            eps = np.float64(np.float32(a.get("epsilon", 1e-5)))
            y = (x - mu.reshape(shp)) / np.sqrt(var.reshape(shp) + eps) * sc.reshape(shp) + bb.reshape(shp)
        elif n.op == "Reshape":
            # model.hpp:1039-1090: the shape input, one -1 inferred
            y = env[n.inputs[0]].reshape([int(d) for d in env[n.inputs[1]].reshape(-1)])
        elif n.op == "Cast":
            y = env[n.inputs[0]]  # model.hpp:1272-1287: values pass through as fp32
        elif n.op in ("Greater", "Less", "Sub"):
            # model.hpp:1176-1300: the right operand is read at i % its size
            x = env[n.inputs[0]].astype(np.float32)
            r = np.resize(env[n.inputs[1]].astype(np.float32).reshape(-1), x.size).reshape(x.shape)
            y = x > r if n.op == "Greater" else (x < r if n.op == "Less" else x - r)
        elif n.op == "Add":
            xa, xb = env[n.inputs[0]].astype(np.float64), env[n.inputs[1]].astype(np.float64)
            if xa.ndim == 4 and xb.ndim in (1, 3):
                xb = xb.reshape(1, -1, 1, 1)
            y = xa + xb
        else:
            raise NotImplementedError(n.op)
        # values cross node boundaries as fp32, as on the device
        env[n.outputs[0]] = np.asarray(y).astype(np.float32)
    if record is not None:
        record.update(env)
    return {k: env[k] for k in spec.outputs}
