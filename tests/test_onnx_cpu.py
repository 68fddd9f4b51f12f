"""The C++ ONNX reader (fast-arm-tbcnn_amd/runtime/onnx.cpp, the reference's
tbn-runtime/src/onnx_integration/onnx_parser.cpp:67-366) on the CPU.

Checks, for the reference's own model files (tests/golden/onnx, copied
unchanged from tests/models/simple/onnx and tests/train/mnist):
  * everything the reader returns equals what the independent Python codec
    (onnx_proto.py) decodes from the same bytes, bit for bit;
  * facts the reference's generator scripts fix (shapes, exact +-1 / ternary
    weight values, zero biases, the LeNet and MNIST-TBN layer structure);
  * simple_cnn.onnx's external tensors tile simple_cnn.onnx.data exactly,
    so none of them is left zero (the reference loads them as zeros).
Synthetic models then cover encodings those files do not use, and the
error paths.  No GPU is touched: Model(path) builds its Session lazily.
"""
import os

import numpy as np
import pytest

import onnx_proto as op

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "onnx")
MODELS = ["simple_matmul", "simple_conv", "simple_mlp", "binary_weights", "ternary_weights", "simple_cnn",
          "mnist_tbn"]
INVALID_MODEL, NOT_IMPLEMENTED = -4, -3


def path_of(name):
    return os.path.join(GOLDEN, name + ".onnx")


def parse_file(tbn, path):
    p = tbn.OnnxParser()
    p.parse_from_file(path)
    return p


def assert_graph_equals(g, ref):
    assert g.inputs == ref["inputs"]
    assert g.outputs == ref["outputs"]
    assert g.value_info == ref["value_info"]
    assert sorted(g.initializer_names()) == sorted(ref["inits"])
    for name, arr in ref["inits"].items():
        got = g.initializer(name)
        assert got.dtype == arr.dtype and got.shape == arr.shape, name
        assert got.tobytes() == arr.tobytes(), name
    nodes = g.nodes()
    assert len(nodes) == len(ref["nodes"])
    for got, want in zip(nodes, ref["nodes"]):
        for k in ("name", "op_type", "inputs", "outputs"):
            assert got[k] == want[k], (want["name"], k)
        assert got["attributes"].keys() == want["attributes"].keys(), want["name"]
        for k, v in want["attributes"].items():
            gv = got["attributes"][k]
            if isinstance(v, np.ndarray):
                assert gv.tobytes() == v.tobytes() and gv.shape == v.shape
            else:
                assert gv == v, (want["name"], k)


@pytest.mark.parametrize("name", MODELS)
def test_reference_model_decodes_like_the_checker(tbn, name):
    p = parse_file(tbn, path_of(name))
    ref = op.load(path_of(name))
    assert (p.get_producer_name(), p.get_producer_version()) == ref["producer"]
    assert p.ir_version() == ref["ir_version"]
    assert p.opset_version() == ref["opsets"][""]
    assert p.warnings() == []
    assert_graph_equals(p.get_graph(), ref)


def test_simple_models_match_their_generator(tbn):
    """tests/models/simple/generate_models.py:20-236 of the reference."""
    shapes = {"simple_matmul": ({"W": (4, 8), "B": (8,)}, [1, 4], [1, 8], ["MatMul", "Add"]),
              "simple_mlp": ({"W1": (16, 32), "B1": (32,), "W2": (32, 10), "B2": (10,)}, [1, 16], [1, 10],
                             ["MatMul", "Add", "Relu", "MatMul", "Add"]),
              "simple_conv": ({"conv_weight": (16, 3, 3, 3), "conv_bias": (16,)}, [1, 3, 32, 32], [1, 16, 30, 30],
                              ["Conv"]),
              "binary_weights": ({"W": (8, 4), "B": (4,)}, [1, 8], [1, 4], ["MatMul", "Add"]),
              "ternary_weights": ({"W": (8, 4), "B": (4,)}, [1, 8], [1, 4], ["MatMul", "Add"])}
    for name, (inits, xs, ys, ops) in shapes.items():
        g = parse_file(tbn, path_of(name)).get_graph()
        assert g.value_info["X"] == xs and g.value_info["Y"] == ys
        assert [n["op_type"] for n in g.nodes()] == ops
        for k, s in inits.items():
            a = g.initializer(k)
            assert a.shape == s and a.dtype == np.float32
            if k.startswith("B") or k == "conv_bias":
                assert not a.any()  # np.zeros in the generator
    assert set(np.unique(parse_file(tbn, path_of("binary_weights")).get_graph().initializer("W"))) <= {-1.0, 1.0}
    t = parse_file(tbn, path_of("ternary_weights")).get_graph().initializer("W")
    assert set(np.unique(t)) <= {-1.0, 0.0, 1.0} and len(np.unique(t)) >= 2
    conv = parse_file(tbn, path_of("simple_conv")).get_graph().nodes()[0]["attributes"]
    assert conv == {"kernel_shape": [3, 3], "pads": [0, 0, 0, 0], "strides": [1, 1]}


def test_simple_cnn_external_data_tiles_the_data_file(tbn):
    """Every external initializer of simple_cnn.onnx is found in
    simple_cnn.onnx.data, and together they cover the file without overlap
    (tests/models/cnn/create_cnn_model.py: LeNet 1->6->16, 256->120->84->10)."""
    g = parse_file(tbn, path_of("simple_cnn")).get_graph()
    blob = open(os.path.join(GOLDEN, "simple_cnn.onnx.data"), "rb").read()
    shapes = {"conv1.weight": (6, 1, 5, 5), "conv2.weight": (16, 6, 5, 5), "fc1.weight": (120, 256),
              "fc2.weight": (84, 120), "fc3.weight": (10, 84), "fc1.bias": (120,), "fc2.bias": (84,)}
    spans = []
    for name, shape in shapes.items():
        a = g.initializer(name)
        assert a.shape == shape and a.dtype == np.float32
        assert np.abs(a).max() > 0, name  # the reference leaves these zero
        off = blob.find(a.tobytes())
        assert off >= 0, name
        spans.append((off, off + a.nbytes))
    spans.sort()
    assert spans[0][0] == 0 and spans[-1][1] == len(blob)
    assert all(a[1] == b[0] for a, b in zip(spans, spans[1:]))
    assert g.initializer("val_5").tolist() == [-1, 256]
    assert [n["op_type"] for n in g.nodes()] == ["Conv", "Relu", "MaxPool", "Conv", "Relu", "MaxPool", "Reshape",
                                                 "Gemm", "Relu", "Gemm", "Relu", "Gemm"]


def test_mnist_tbn_matches_its_training_script(tbn):
    """tests/train/mnist/train_tbn_mnist.py:196-240: conv 1->16 5x5 p2, conv
    16->32 5x5 p2 with a +-0.5 ternary activation, pools 2 and 3, fc 512->10
    exported as sign(w) * mean|w| per output row."""
    g = parse_file(tbn, path_of("mnist_tbn")).get_graph()
    assert g.initializer("conv1_w").shape == (16, 1, 5, 5) and g.initializer("conv2_w").shape == (32, 16, 5, 5)
    fc = g.initializer("fc_w")
    assert fc.shape == (10, 512)
    assert np.all(np.abs(fc) == np.abs(fc[:, :1]))  # one magnitude per row
    assert float(g.initializer("val_1")) == 0.5 and float(g.initializer("val_2")) == -0.5
    assert g.initializer("val_1").shape == ()
    nodes = {n["op_type"] + str(i): n for i, n in enumerate(g.nodes())}
    assert nodes["MaxPool9"]["attributes"]["kernel_shape"] == [3, 3]
    assert nodes["Conv3"]["attributes"]["pads"] == [2, 2, 2, 2]
    assert nodes["Gemm11"]["attributes"]["transB"] == 1


def test_load_model_and_model_wrappers(tbn):
    m = tbn.load_onnx_model(path_of("simple_cnn"))
    assert (m.producer_name(), m.producer_version()) == ("pytorch", "2.11.0")
    assert m.get_input_shape("input") == [1, 1, 28, 28] and m.get_output_shape("output") == [1, 10]
    m.validate()
    model = tbn.Model(path_of("mnist_tbn"))
    assert model.input_names() == ["input"] and model.output_names() == ["output"]
    assert model.input_shape("input").dims == [1, 1, 28, 28]
    assert model.producer() == ("pytorch", "2.11.0")
    model2 = tbn.load_model(path_of("simple_mlp"), 64, 64, 128, 32, 32)
    assert model2.input_names() == ["X"]


def test_buffer_parse_needs_a_base_dir_for_external_data(tbn):
    data = open(path_of("simple_cnn"), "rb").read()
    p = tbn.OnnxParser()
    with pytest.raises(tbn.TBNError) as e:
        p.parse_from_buffer(data)
    assert e.value.code == INVALID_MODEL and "base directory" in str(e.value)
    p.parse_from_buffer(data, GOLDEN)
    assert_graph_equals(p.get_graph(), op.load(path_of("simple_cnn")))
    p.parse_from_buffer(open(path_of("simple_mlp"), "rb").read())  # no external data: no base dir needed
    assert p.get_graph().num_nodes() == 5


# ---- synthetic encodings ---------------------------------------------------------------

def _roundtrip(tbn, model_bytes, base_dir=""):
    p = tbn.OnnxParser()
    p.parse_from_buffer(model_bytes, base_dir)
    return p


def test_tensor_encodings_round_trip(tbn, tmp_path):
    rng = np.random.default_rng(3)
    f32 = rng.standard_normal((3, 5)).astype(np.float32)
    f32[0, :3] = [-0.0, np.inf, np.float32(1e-45)]
    arrays = {
        "raw": (f32, "raw"), "typed": (f32, "typed"), "unpacked": (f32[:2], "unpacked"),
        "i64": (np.array([-1, 256, -(2 ** 40), 2 ** 62], np.int64), "typed"),
        "i64u": (np.array([[-7], [9]], np.int64), "unpacked"),
        "i32": (np.array([-5, 2 ** 31 - 1, -(2 ** 31)], np.int32), "typed"),
        "i8": (np.array([-128, -1, 0, 127], np.int8), "typed"),
        "u8": (np.array([0, 1, 255], np.uint8), "unpacked"),
        "i16": (np.array([-32768, 5], np.int16), "typed"),
        "u16": (np.array([65535, 1], np.uint16), "typed"),
        "f16": (np.array([1.5, -2.0, 65504.0], np.float16), "typed"),
        "b": (np.array([True, False, True]), "typed"),
        "u32": (np.array([4294967295, 3], np.uint32), "typed"),
        "u64": (np.array([2 ** 64 - 1, 0], np.uint64), "typed"),
        "scalar": (np.array(2.5, np.float32), "typed"),
        "empty": (np.zeros((0, 4), np.float32), "raw"),
        "i8raw": (np.array([-3, 4], np.int8), "raw"),
    }
    inits = [op.encode_tensor(k, a, mode) for k, (a, mode) in arrays.items()]
    blob = rng.standard_normal(64).astype(np.float32)
    (tmp_path / "w.bin").write_bytes(b"\x00" * 12 + blob.tobytes())
    (tmp_path / "sub").mkdir()
    (tmp_path / "sub" / "w2.bin").write_bytes(blob[:6].tobytes())
    inits.append(op.encode_tensor("ext", blob.reshape(8, 8), "external", ("w.bin", 12, 256)))
    inits.append(op.encode_tensor("ext_nolen", blob[:6].reshape(2, 3), "external", ("sub/w2.bin", 0, None)))
    model = op.encode_model([op.encode_node("Relu", ["x"], ["y"])], inits, [op.encode_value_info("x", [2, 3])],
                            [op.encode_value_info("y", [2, 3])])
    g = _roundtrip(tbn, model, str(tmp_path)).get_graph()
    ref = op.decode_model(model, str(tmp_path))
    for k, (a, _) in arrays.items():
        got = g.initializer(k)
        assert got.shape == a.shape and got.tobytes() == a.tobytes(), k
        assert ref["inits"][k].tobytes() == a.tobytes(), k  # the checker agrees
    assert g.initializer("ext").tobytes() == blob.tobytes()
    assert g.initializer("ext_nolen").tobytes() == blob[:6].tobytes()
    assert g.initializer_dtype("b") == "bool" and g.initializer_dtype("i8") == "int8"


def test_graph_fields(tbn):
    w = np.ones((4, 2), np.float32)
    nodes = [
        op.encode_node("MatMul", ["x", "w"], ["t"]),  # unnamed: "MatMul_t"
        op.encode_node("Relu", ["t"], ["y"], name="act"),
        op.encode_node("Custom", ["y"], ["z"], name="c",
                       attrs={"i": -3, "f": 0.25, "s": "abc", "ints": [1, -2, 3], "floats": [0.5, -1.5],
                              "strings": ["p", "q"], "t": np.array([[1, 2]], np.int64)}),
        op.encode_node("Old", ["z"], ["u"], name="o", attrs={"i": 7, "ints": [4, 5], "s": "x"}, typed=False),
    ]
    model = op.encode_model(
        nodes, [op.encode_tensor("w", w)],
        [op.encode_value_info("x", [3, 4], symbolic=(0,)), op.encode_value_info("w", [4, 2])],
        [op.encode_value_info("u", [3, 2])], [op.encode_value_info("t", [5, 2], symbolic=(0,))],
        producer=("me", "0.1"), opset=13, ir_version=7)
    p = _roundtrip(tbn, model)
    g = p.get_graph()
    assert p.get_producer_name() == "me" and p.ir_version() == 7 and p.opset_version() == 13
    assert p.opset_version("com.other") == -1
    assert g.inputs == ["x"]  # "w" names an initializer: a constant, not an input
    assert g.value_info["x"] == [1, 4] and g.value_info["t"] == [1, 2]  # symbolic dims read as 1
    n = g.nodes()
    assert [d["name"] for d in n] == ["MatMul_t", "act", "c", "o"]
    a = n[2]["attributes"]
    assert a["i"] == -3 and a["f"] == 0.25 and a["s"] == "abc" and a["ints"] == [1, -2, 3]
    assert a["floats"] == [0.5, -1.5] and a["strings"] == ["p", "q"]
    assert a["t"].tolist() == [[1, 2]] and a["t"].dtype == np.int64
    assert n[3]["attributes"] == {"i": 7, "ints": [4, 5], "s": "x"}
    assert_graph_equals(g, op.decode_model(model))


def test_skipped_attribute_types_are_reported(tbn):
    graph_attr = op.f_bytes(1, "body") + op.f_bytes(6, op.f_bytes(2, "sub")) + op.f_varint(20, 5)
    node = op.encode_node("If", ["c"], ["y"], name="if") + op.f_bytes(5, graph_attr)
    model = op.encode_model([node], [], [op.encode_value_info("c", [1])], [op.encode_value_info("y", [1])])
    p = _roundtrip(tbn, model)
    assert p.get_graph().nodes()[0]["attributes"] == {}
    assert len(p.warnings()) == 1 and "body" in p.warnings()[0]


# ---- errors ------------------------------------------------------------------------------

def _raises(tbn, code, model_bytes, base_dir="", match=None):
    with pytest.raises(tbn.TBNError) as e:
        _roundtrip(tbn, model_bytes, base_dir)
    assert e.value.code == code, str(e.value)
    if match:
        assert match in str(e.value), str(e.value)


def _model_with(init):
    return op.encode_model([op.encode_node("Relu", ["x"], ["y"])], [init], [op.encode_value_info("x", [2])],
                           [op.encode_value_info("y", [2])])


def test_malformed_and_unsupported_models_raise(tbn, tmp_path):
    good = open(path_of("simple_mlp"), "rb").read()
    for cut in (1, 7, len(good) // 2, len(good) - 1):
        _raises(tbn, INVALID_MODEL, good[:cut])
    _raises(tbn, INVALID_MODEL, op.key(1, 3) + good)  # group wire type
    _raises(tbn, INVALID_MODEL, b"\xff" * 11)  # varint over 10 bytes
    _raises(tbn, INVALID_MODEL, op.f_varint(1, 8), match="no graph")
    _raises(tbn, INVALID_MODEL, op.f_bytes(7, op.f_varint(1, 5)))  # GraphProto.node as a varint
    a = np.arange(4, dtype=np.float32)
    bad_raw = op.f_packed_varints(1, [4]) + op.f_varint(2, 1) + op.f_bytes(8, "w") + op.f_bytes(9, a.tobytes()[:12])
    _raises(tbn, INVALID_MODEL, _model_with(bad_raw), match="raw_data")
    no_data = op.f_packed_varints(1, [4]) + op.f_varint(2, 1) + op.f_bytes(8, "w")
    _raises(tbn, INVALID_MODEL, _model_with(no_data), match="float_data")
    few = op.f_packed_varints(1, [4]) + op.f_varint(2, 7) + op.f_bytes(8, "w") + op.f_packed_varints(7, [1, 2])
    _raises(tbn, INVALID_MODEL, _model_with(few), match="int64_data")
    dbl = op.f_packed_varints(1, [1]) + op.f_varint(2, 11) + op.f_bytes(8, "d") + op.f_bytes(9, b"\0" * 8)
    _raises(tbn, NOT_IMPLEMENTED, _model_with(dbl), match="data type 11")
    neg = op.f_packed_varints(1, [-2]) + op.f_varint(2, 1) + op.f_bytes(8, "w")
    _raises(tbn, INVALID_MODEL, _model_with(neg), match="negative")
    (tmp_path / "d.bin").write_bytes(a.tobytes())
    for loc, off, ln, match in [("../d.bin", 0, 16, "relative"), ("/etc/passwd", 0, 16, "relative"),
                                ("sub/../../d.bin", 0, 16, "relative"), ("d.bin", 0, 12, "bytes"),
                                ("d.bin", 8, 16, "past the end"), ("d.bin", 20, None, "past the end"),
                                ("missing.bin", 0, 16, "cannot open")]:
        _raises(tbn, INVALID_MODEL, _model_with(op.encode_tensor("w", a, "external", (loc, off, ln))),
                str(tmp_path), match)
    bad_off = op.encode_tensor("w", a, "external", ("d.bin", "1x", 16))
    _raises(tbn, INVALID_MODEL, _model_with(bad_off), str(tmp_path), match="offset")
    p = tbn.OnnxParser()
    with pytest.raises(tbn.TBNError) as e:
        p.parse_from_file(os.path.join(GOLDEN, "no_such_model.onnx"))
    assert e.value.code == INVALID_MODEL
    with pytest.raises(tbn.TBNError) as e:
        tbn.load_model(os.path.join(GOLDEN, "no_such_model.onnx"))
    assert e.value.code == INVALID_MODEL


def test_sizes_are_checked_before_allocation(tbn, tmp_path):
    """A shape claiming ~4 TB with a few bytes of data is rejected from its
    data size, before any allocation, on every data path."""
    huge = [1 << 20, 1 << 20]
    typed = op.f_packed_varints(1, huge) + op.f_varint(2, 1) + op.f_bytes(8, "w") + op.f_bytes(4, b"\0" * 8)
    _raises(tbn, INVALID_MODEL, _model_with(typed), match="float_data")
    raw = op.f_packed_varints(1, huge) + op.f_varint(2, 1) + op.f_bytes(8, "w") + op.f_bytes(9, b"\0" * 8)
    _raises(tbn, INVALID_MODEL, _model_with(raw), match="raw_data")
    (tmp_path / "d.bin").write_bytes(b"\0" * 64)
    ext = op.f_packed_varints(1, huge) + op.f_varint(2, 1) + op.f_bytes(8, "w")
    ext += op.f_bytes(13, op.f_bytes(1, "location") + op.f_bytes(2, "d.bin")) + op.f_varint(14, 1)
    _raises(tbn, INVALID_MODEL, _model_with(ext), str(tmp_path), match="external data holds")


def test_mutated_reference_models_parse_or_raise(tbn):
    """Random byte edits of the reference model files (seeded): every parse
    either succeeds or raises TBNError; nothing else escapes and nothing
    crashes.  (The same mutator ran 60,000 times under AddressSanitizer and
    UndefinedBehaviorSanitizer on the host build without a report.)"""
    rng = np.random.default_rng(2024)
    seeds = [open(path_of(n), "rb").read() for n in ("simple_cnn", "simple_mlp", "mnist_tbn", "simple_conv")]
    parsed = failed = 0
    for _ in range(1500):
        b = bytearray(seeds[rng.integers(len(seeds))])
        for _ in range(int(rng.integers(1, 6))):
            pos = int(rng.integers(len(b)))
            kind = int(rng.integers(4))
            if kind == 0:
                b[pos] ^= 1 << int(rng.integers(8))
            elif kind == 1:
                b[pos] = int(rng.integers(256))
            elif kind == 2:
                del b[pos:]
            else:
                b.insert(pos, int(rng.integers(256)))
            if not b:
                break
        p = tbn.OnnxParser()
        try:
            p.parse_from_buffer(bytes(b), GOLDEN)
            p.get_graph()
            parsed += 1
        except tbn.TBNError:
            failed += 1
    assert parsed + failed == 1500 and parsed > 0 and failed > 0
