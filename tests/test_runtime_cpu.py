"""Host-side checks of the C++ runtime (_tbn module over libtbn.so) and of the
CPU reference executor used by the Session tests.  No kernel runs here."""
import numpy as np
import pytest

import models
import refmath as rm


def test_module_loads_and_reports_version(tbn):
    assert tbn.get_version() == "0.1.0"
    assert tbn.current_stream() == 0


def test_host_tensor_round_trip(tbn):
    for arr, dt in [(np.arange(12, dtype=np.float32).reshape(3, 4), "float32"),
                    (np.array([[1, 0], [0, 1]], np.uint8), "binary"),
                    (np.array([-1, 0, 1], np.int8), "ternary"),
                    (np.array([3, -1], np.int64), "int64")]:
        t = tbn.Tensor(arr, dt)
        assert t.dtype == dt and t.device == "cpu" and t.shape == list(arr.shape)
        assert np.array_equal(t.numpy(), arr)
    t = tbn.Tensor(np.ones((2, 6), np.float32))
    assert t.reshaped([3, 4]).shape == [3, 4]
    with pytest.raises(tbn.TBNError) as e:
        t.reshaped([5])
    assert e.value.code == -7


def test_graph_validation_errors(tbn):
    spec = models.lenet(seed=1)
    m = tbn.TBNModel(models.build_graph(spec, tbn))
    m.validate()
    assert m.inputs() == ["input"] and m.outputs() == ["output"]
    g = tbn.ModelGraph()
    with pytest.raises(tbn.TBNError) as e:
        tbn.TBNModel(g).validate()
    assert e.value.code == -4  # INVALID_MODEL: no inputs
    g = models.build_graph(spec, tbn)
    g.add_node("dangling", "Relu", ["missing"], ["output2"], {})
    with pytest.raises(tbn.TBNError) as e:
        tbn.TBNModel(g).validate()
    assert e.value.code == -4 and "missing" in str(e.value)


def test_session_input_checks_before_device_use(tbn):
    spec = models.lenet(seed=1)
    s = tbn.TBNModel(models.build_graph(spec, tbn)).create_session()
    with pytest.raises(tbn.TBNError) as e:
        s.set_input("input", np.zeros((1, 1, 28, 27), np.float32))
    assert e.value.code == -7
    with pytest.raises(tbn.TBNError) as e:
        s.set_input("nope", np.zeros((1, 1, 28, 28), np.float32))
    assert e.value.code == -1
    with pytest.raises(tbn.TBNError) as e:
        s.run()
    assert e.value.code == -1
    assert s.planned_launches() == 0


def _device_present():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.mark.skipif(_device_present(), reason="checks the error path of a host without a HIP device")
def test_device_operator_without_gpu_raises_device_not_supported(tbn):
    with pytest.raises(tbn.TBNError) as e:
        tbn.relu(np.ones(4, np.float32))
    assert e.value.code == -8


# ---- the CPU reference executor (pins tests/models.run_oracle) -------------------------

def _np_lenet(spec, x, quant):
    """LeNet through independent numpy formulations (refmath) only."""
    i = spec.inits
    def qconv(x, w, b):
        if not quant:
            return rm.f64_conv(x, w, b)
        flat = w.reshape(w.shape[0], -1)
        s = np.array([rm.seq_sum_f32(np.abs(r)) / np.float32(r.size) for r in flat], np.float32)
        sign = np.where(w >= 0, 1.0, -1.0)
        return ((rm.f64_conv(x, sign) + b[None, :, None, None]) * s[None, :, None, None])
    y = qconv(x, i["w1"], i["b1"]).astype(np.float32)
    y = rm.np_maxpool(np.maximum(y, 0), (2, 2), (2, 2))
    y = qconv(y, i["w2"], i["b2"]).astype(np.float32)
    y = rm.np_maxpool(np.maximum(y, 0), (2, 2), (2, 2)).reshape(1, -1)
    B = np.where(i["wf"] > 0, 1.0, -1.0) if quant else i["wf"].astype(np.float64)
    return y.astype(np.float64) @ B + i["bf"]


@pytest.mark.parametrize("quant", [True, False])
def test_run_oracle_lenet_matches_numpy(orc, quant):
    spec = models.lenet(seed=1, prebinarized=True)
    x = models.lenet_input(1)
    got = models.run_oracle(spec, {"input": x}, quant, orc)["output"]
    want = _np_lenet(spec, x, quant)
    rm.assert_within_tolerance(got, want, 256, 10.0, rel=1e-6)


def test_run_oracle_detects_prebinarized_weights(orc):
    spec = models.lenet(seed=1, prebinarized=True)
    w = spec.inits["w1"]
    assert orc.already_binary(w, orc.channel_mean_abs(w))
    raw = models.lenet(seed=1, prebinarized=False).inits["w1"]
    assert not orc.already_binary(raw, orc.channel_mean_abs(raw))


def test_resnet18_graph_shapes():
    spec = models.resnet18(batch=2)
    convs = [n for n in spec.nodes if n.op == "Conv"]
    assert len(convs) == 1 + 16 + 3
    assert sum(1 for n in convs if n.attrs.get("tbn_quantize", 1) == 0) == 1
    assert spec.value_info["pool_out"] == (2, 64, 56, 56)
    assert spec.value_info["l4b1_r2_out"] == (2, 512, 7, 7)
    assert spec.outputs == {"logits": (2, 1000)}


def test_gemm_engine_host_checks(tbn):
    """The GeMM engine API's argument checks (GeMM/05-final/GeMM.hpp:24-37,
    GeMM.cpp:29-150, test_final.cpp:76-133) throw before any device work."""
    t = tbn.TilingParams.default_128x128()
    assert (t.mblk, t.nblk, t.kblk, t.mmk, t.nmk) == (64, 64, 128, 32, 32)
    t.validate(128, 128, 128)
    for args, msg in [((128, 64, 128), "n must be multiple of 128"), ((48, 128, 128), "m must be multiple of mmk"),
                      ((128, 128, 40), "k must be multiple of nmk")]:
        with pytest.raises(ValueError, match=msg):
            t.validate(*args)
    with pytest.raises(ValueError, match="kblk must be multiple of 128"):
        tbn.TilingParams(64, 64, 64, 32, 32).validate(128, 128, 128)
    bad = np.zeros(8 * 64, np.int8); bad[0] = 2
    with pytest.raises(ValueError, match="values must be -1, 0, or \\+1"):
        tbn.TernaryMatrix.pack(bad, 8, 64)
    with pytest.raises(ValueError, match="values must be -1 or \\+1"):
        tbn.BinaryMatrix.pack(np.zeros(64 * 8, np.int8), 64, 8)
    with pytest.raises(ValueError, match="rows must be multiple of 8"):
        tbn.TernaryMatrix.pack(np.zeros(100, np.int8), 10, 10)
    with pytest.raises(ValueError, match="cols must be multiple of 64"):
        tbn.TernaryMatrix.pack_from_float(np.zeros(8 * 32, np.float32), 8, 32)
    assert tbn.TernaryMatrix().empty() and tbn.BinaryMatrix().empty()
    assert tbn.TernaryMatrix().rows == 0 and tbn.BinaryMatrix().cols == 0
