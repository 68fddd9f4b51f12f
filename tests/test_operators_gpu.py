"""The C++ operator entry points (tbn::qlinear_matmul_binary / _ternary /
_binary_float, conv2d_binary / _with_scales, quantize_to_binary, maxpool2d,
global_avgpool2d, gemm) through the _tbn module, against the oracle.

Each runs with host tensors (the result comes back on the host, as the
reference's operators return host tensors) and with HIP tensors (the result
stays on the device), at BASELINE.json's config-2 GEMM shape (1024^3) and
config-4 conv shape (64x64x14x14 -> 128, 3x3, pad 1), plus the config-3
ternary shape (256x4096x4096).  Reference routing:
tbn-runtime/src/operators/quantized_gemm_neon.cpp:380-538 (B dtype decides:
BINARY -> blocked path, FLOAT32 with values in {-1, 0, 1} -> the _float path
where w >= 0 reads as +1), tbn-runtime/src/operators/conv2d.cpp:220-369.
Float outputs are held to the north_star tolerance against float64; integer
and byte outputs compare bit for bit."""
import numpy as np
import pytest

import refmath as rm

pytestmark = pytest.mark.gpu

ERR_INVALID_ARGUMENT = -1
ERR_INVALID_SHAPE = -7


def _dev(tbn, a, dtype=""):
    return tbn.Tensor(np.ascontiguousarray(a), dtype, "hip")


def _out(t, want_device):
    assert t.device == ("hip" if want_device else "cpu")
    return t.numpy()


@pytest.fixture(scope="module")
def cfg2():
    rng = np.random.default_rng(2)
    A = rng.standard_normal((1024, 1024)).astype(np.float32)
    Bb = (rng.random((1024, 1024)) < 0.5).astype(np.uint8)
    sign = np.where(Bb == 1, 1.0, -1.0)
    return A, Bb, A.astype(np.float64) @ sign


@pytest.mark.parametrize("on_device", [False, True], ids=["host", "hip"])
def test_qlinear_matmul_binary_binary_b(dev, tbn, cfg2, on_device):
    A, Bb, ref = cfg2
    a, b = (_dev(tbn, A), _dev(tbn, Bb, "binary")) if on_device else (A, tbn.Tensor(Bb, "binary"))
    got = _out(tbn.qlinear_matmul_binary(a, b, 0.75), on_device)
    rm.assert_within_tolerance(got, ref * 0.75, 1024, np.abs(A).max() * 0.75)


@pytest.mark.parametrize("on_device", [False, True], ids=["host", "hip"])
def test_qlinear_matmul_binary_float32_pm1_b(dev, tbn, cfg2, on_device):
    """FLOAT32 B holding -1/+1 (and 0, which reads as +1) takes the _float route."""
    A, Bb, ref = cfg2
    Bf = np.where(Bb == 1, 1.0, -1.0).astype(np.float32)
    zeros = np.zeros_like(Bf, bool)
    zeros[::7, ::5] = True
    zeros &= Bb == 1  # zeros only where the sign is +1, so the reference stays `ref`
    Bf[zeros] = 0.0
    b = _dev(tbn, Bf) if on_device else Bf
    a = _dev(tbn, A) if on_device else A
    got = _out(tbn.qlinear_matmul_binary(a, b, 1.5), on_device)
    rm.assert_within_tolerance(got, ref * 1.5, 1024, np.abs(A).max() * 1.5)
    got_f = _out(tbn.qlinear_matmul_binary_float(a, b, 1.5), on_device)
    assert np.array_equal(got_f, got)


def test_qlinear_matmul_binary_float_zero_is_plus_one(dev, tbn, orc):
    """Known answer: B = [[0, -1], [1, 0]] reads as [[+1, -1], [+1, +1]]."""
    A = np.array([[1.0, -2.0], [3.0, -4.0]], np.float32)
    B = np.array([[0.0, -1.0], [1.0, 0.0]], np.float32)
    got = tbn.qlinear_matmul_binary(A, B, 0.5).numpy()
    np.testing.assert_array_equal(got, np.float32([[-0.5, -1.5], [-0.5, -3.5]]))


def test_qlinear_matmul_binary_rejects(tbn):
    """Argument errors carry the reference's ErrorCode (errors.hpp:10-22).  A
    FLOAT32 B with values outside {-1, 0, 1} is rejected here; the reference
    would read its bytes as BINARY bytes (quantized_gemm_neon.cpp:418-421,
    200-205), a result no caller can use."""
    A = np.ones((4, 8), np.float32)
    with pytest.raises(tbn.TBNError) as e:
        tbn.qlinear_matmul_binary(A, np.full((8, 3), 0.5, np.float32))
    assert e.value.code == ERR_INVALID_ARGUMENT
    with pytest.raises(tbn.TBNError) as e:
        tbn.qlinear_matmul_binary(A, tbn.Tensor(np.ones((7, 3), np.uint8), "binary"))
    assert e.value.code == ERR_INVALID_SHAPE
    with pytest.raises(tbn.TBNError) as e:
        tbn.qlinear_matmul_binary(A, np.ones((8, 3), np.int32))
    assert e.value.code == ERR_INVALID_ARGUMENT
    with pytest.raises(tbn.TBNError) as e:
        tbn.qlinear_matmul_ternary(A, tbn.Tensor(np.ones((8, 3), np.uint8), "binary"))
    assert e.value.code == ERR_INVALID_ARGUMENT


@pytest.mark.parametrize("on_device", [False, True], ids=["host", "hip"])
def test_qlinear_matmul_ternary_cfg3(dev, tbn, on_device):
    """Config 3: M=256, N=K=4096, weights -1/0/+1 with p = 0.3/0.4/0.3; the
    ternary 0 stays 0 (true float x ternary, test_quantized_operators.cpp:151-155)."""
    rng = np.random.default_rng(3)
    A = rng.standard_normal((256, 4096)).astype(np.float32)
    T = rng.choice(np.int8([-1, 0, 1]), size=(4096, 4096), p=[0.3, 0.4, 0.3])
    ref = A.astype(np.float64) @ T.astype(np.float64) * 0.5
    a, t = (_dev(tbn, A), _dev(tbn, T, "ternary")) if on_device else (A, tbn.Tensor(T, "ternary"))
    got = _out(tbn.qlinear_matmul_ternary(a, t, 0.5), on_device)
    rm.assert_within_tolerance(got, ref, 4096, np.abs(A).max() * 0.5)


def test_qlinear_matmul_ternary_known_answer(dev, tbn):
    # test_quantized_operators.cpp:121-155: A [[1,2],[3,4]], T [[1,-1],[0,1]], scale 0.5
    A = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    T = np.array([[1, -1], [0, 1]], np.int8)
    got = tbn.qlinear_matmul_ternary(A, tbn.Tensor(T, "ternary"), 0.5).numpy()
    assert got.reshape(-1).tolist() == [0.5, 0.5, 1.5, 0.5]


@pytest.fixture(scope="module")
def cfg4(orc):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((64, 64, 14, 14)).astype(np.float32)
    Wb = (rng.random((128, 64, 3, 3)) < 0.5).astype(np.uint8)
    b = (rng.standard_normal(128) * 0.01).astype(np.float32)
    s = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    acc = orc.conv2d_f64(x, np.where(Wb == 1, 1.0, -1.0).astype(np.float32), None, (1, 1), (1, 1))
    return x, Wb, b, s, acc


@pytest.mark.parametrize("on_device", [False, True], ids=["host", "hip"])
def test_conv2d_binary_cfg4(dev, tbn, cfg4, on_device):
    x, Wb, b, s, acc = cfg4
    xi = _dev(tbn, x) if on_device else x
    wi = _dev(tbn, Wb, "binary") if on_device else tbn.Tensor(Wb, "binary")
    bi = _dev(tbn, b) if on_device else b
    got = _out(tbn.conv2d_binary(xi, wi, bi, pad=[1, 1]), on_device)
    rm.assert_within_tolerance(got, acc + b[None, :, None, None], 576, np.abs(x).max())


@pytest.mark.parametrize("on_device", [False, True], ids=["host", "hip"])
def test_conv2d_binary_with_scales_cfg4(dev, tbn, cfg4, on_device):
    """conv2d.cpp:319-369: per-channel scale first, then bias."""
    x, Wb, b, s, acc = cfg4
    xi = _dev(tbn, x) if on_device else x
    wi = _dev(tbn, Wb, "binary") if on_device else tbn.Tensor(Wb, "binary")
    bi = _dev(tbn, b) if on_device else b
    got = _out(tbn.conv2d_binary_with_scales(xi, wi, bi, s.tolist(), pad=[1, 1]), on_device)
    ref = acc * s.astype(np.float64)[None, :, None, None] + b[None, :, None, None]
    rm.assert_within_tolerance(got, ref, 576, np.abs(x).max() * 1.5)


def test_conv2d_binary_rejects(tbn):
    x = np.ones((1, 3, 8, 8), np.float32)
    with pytest.raises(tbn.TBNError) as e:
        tbn.conv2d_binary(x, tbn.Tensor(np.ones((4, 2, 3, 3), np.uint8), "binary"))
    assert e.value.code == ERR_INVALID_SHAPE
    with pytest.raises(tbn.TBNError) as e:
        tbn.conv2d_binary_with_scales(x, tbn.Tensor(np.ones((4, 3, 3, 3), np.uint8), "binary"), None, [1.0] * 3)
    assert e.value.code in (ERR_INVALID_ARGUMENT, ERR_INVALID_SHAPE)


SPECIAL = np.array([0.0, -0.0, np.nan, np.inf, -np.inf, 1e-45, -1e-45, 0.1, -0.1, 3.0, -3.0], np.float32)


@pytest.mark.parametrize("on_device", [False, True], ids=["host", "hip"])
@pytest.mark.parametrize("thr", [0.0, 0.1])
def test_quantize_to_binary(dev, tbn, orc, on_device, thr):
    rng = np.random.default_rng(5)
    w = np.concatenate([SPECIAL, rng.standard_normal(128 * 64 * 9).astype(np.float32)]).reshape(-1, 1)
    wi = _dev(tbn, w) if on_device else w
    q = tbn.quantize_to_binary(wi, thr)
    assert q.dtype == "binary" and q.shape == [w.shape[0], 1]
    assert np.array_equal(_out(q, on_device).reshape(-1), orc.quantize_to_binary_f32(w.reshape(-1), thr))
    w8 = np.array([-128, -1, 0, 1, 127], np.int8)
    q8 = tbn.quantize_to_binary(_dev(tbn, w8, "int8") if on_device else w8)
    assert _out(q8, on_device).tolist() == [0, 0, 0, 1, 1]


@pytest.mark.parametrize("on_device", [False, True], ids=["host", "hip"])
def test_maxpool2d_and_global_avgpool(dev, tbn, orc, on_device):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((2, 64, 56, 56)).astype(np.float32)
    x[0, 0, ::3, ::4] = -0.0
    x[1, 2, 1::5, ::2] = np.nan
    xi = _dev(tbn, x) if on_device else x
    got = _out(tbn.maxpool2d(xi, [3, 3], [2, 2], [1, 1]), on_device)
    ref = orc.maxpool2d(x, (3, 3), (2, 2), (1, 1))
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    got2 = _out(tbn.maxpool2d(xi, [2, 2], [2, 2], [0, 0], True), on_device)
    assert np.array_equal(got2.view(np.uint32), orc.maxpool2d(x, (2, 2), (2, 2), (0, 0), ceil_mode=True).view(np.uint32))
    g = rng.standard_normal((32, 512, 7, 7)).astype(np.float32)
    gi = _dev(tbn, g) if on_device else g
    got3 = _out(tbn.global_avgpool2d(gi), on_device)
    assert np.array_equal(got3.reshape(32, 512), orc.global_avgpool2d(g).reshape(32, 512))


@pytest.mark.parametrize("on_device", [False, True], ids=["host", "hip"])
@pytest.mark.parametrize("tA,tB", [(False, False), (True, False), (False, True)])
def test_gemm_fp32(dev, tbn, on_device, tA, tB):
    """gemm.cpp:349-360: alpha*op(A)@op(B) + beta*C with a 1-D C bias."""
    rng = np.random.default_rng(7)
    M, K, N = 32, 512, 1000
    A = rng.standard_normal((K, M) if tA else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if tB else (K, N)).astype(np.float32)
    C = rng.standard_normal(N).astype(np.float32)
    ref = 0.5 * ((A.T if tA else A).astype(np.float64) @ (B.T if tB else B).astype(np.float64)) + 2.0 * C
    args = [_dev(tbn, v) for v in (A, B, C)] if on_device else [A, B, C]
    got = _out(tbn.gemm(*args, alpha=0.5, beta=2.0, transA=tA, transB=tB), on_device)
    rm.assert_within_tolerance(got, ref, K, np.abs(A).max() * np.abs(B).max())


@pytest.mark.parametrize("on_device", [False, True])
def test_avgpool2d_and_global_maxpool2d(dev, tbn, orc, on_device):
    """tbn::avgpool2d / tbn::global_maxpool2d (pooling.cpp:83-181), bitwise."""
    rng = np.random.default_rng(8)
    x = rng.standard_normal((2, 8, 15, 13)).astype(np.float32)
    a = _dev(tbn, x) if on_device else x
    y = _out(tbn.avgpool2d(a, [3, 3], [2, 2], [1, 1], False, True), on_device)
    assert np.array_equal(y, orc.avgpool2d(x, (3, 3), (2, 2), (1, 1), count_include_pad=True))
    g = _out(tbn.global_maxpool2d(a), on_device)
    assert np.array_equal(g.reshape(2, 8), orc.global_maxpool2d(x))
