"""Pooling / elementwise operators on the GPU vs the oracle.  Max, ReLU, the
window-order AvgPool and the sequential-sum GlobalAvgPool round exactly as
the reference does, so these compare bit for bit."""
import numpy as np
import pytest
import torch

import refmath as rm
import tbn_hip
from gpu_util import P, empty, host, to_dev

pytestmark = pytest.mark.gpu


def gpu_maxpool(x, k, s, p=(0, 0), ceil_mode=False):
    N, C, H, W = x.shape
    import ctypes
    hw = (ctypes.c_int64 * 2)()
    args = [N, C, H, W, k[0], k[1], s[0], s[1], p[0], p[1], 1, 1, int(ceil_mode)]
    tbn_hip.call("tbn_hip_maxpool2d", None, *args, None, hw, None)
    y = empty((N, C, hw[0], hw[1]), torch.float32)
    tbn_hip.call("tbn_hip_maxpool2d", P(to_dev(x)), *args, P(y), hw, None)
    return host(y)


@pytest.mark.parametrize("k,s,p,ceil_mode", [((2, 2), (2, 2), (0, 0), False), ((3, 3), (2, 2), (1, 1), False),
                                             ((3, 3), (2, 2), (0, 0), True), ((2, 3), (1, 2), (1, 1), False)])
def test_maxpool_bit_exact(dev, orc, k, s, p, ceil_mode):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((2, 3, 9, 8)).astype(np.float32)
    x[0, 0, 0, 0] = np.nan  # ignored by the running max, as in the reference
    assert np.array_equal(gpu_maxpool(x, k, s, p, ceil_mode), orc.maxpool2d(x, k, s, p, ceil_mode=ceil_mode))


def test_maxpool_known_answer_and_resnet_shape(dev, orc):
    x = (np.arange(32) % 10).astype(np.float32).reshape(1, 2, 4, 4)
    assert gpu_maxpool(x, (2, 2), (2, 2)).reshape(-1)[:2].tolist() == [5.0, 7.0]
    rng = np.random.default_rng(2)
    x = rng.standard_normal((2, 64, 112, 112)).astype(np.float32)
    assert np.array_equal(gpu_maxpool(x, (3, 3), (2, 2), (1, 1)), orc.maxpool2d(x, (3, 3), (2, 2), (1, 1)))


@pytest.mark.parametrize("shape,ceil_mode", [((2, 3, 9, 7), False), ((1, 2, 8, 8), True), ((1, 2, 200, 300), False),
                                              ((2, 2, 5, 130), True)])
def test_maxpool_3x3_stride2_bitwise(dev, orc, shape, ceil_mode):
    """The specialised 3x3 / stride 2 / pad 1 path (row maxima shared by
    neighbouring output rows): bit-identical to the reference's first-wins
    running max, including which zero sign survives, NaN taps, infinities,
    odd widths, ceil mode and planes wider than 64 outputs / taller than 64."""
    rng = np.random.default_rng(shape[3])
    x = rng.standard_normal(shape).astype(np.float32)
    x[..., ::3, 1::4] = 0.0
    x[..., 1::3, ::4] = -0.0
    x[..., 2::5, 2::3] = np.nan
    x[0, 0, 0, :3] = np.inf
    x[0, -1, -1, -3:] = -np.inf
    x[-1, -1, :, :] = np.nan
    got = gpu_maxpool(x, (3, 3), (2, 2), (1, 1), ceil_mode)
    ref = orc.maxpool2d(x, (3, 3), (2, 2), (1, 1), ceil_mode=ceil_mode)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("shape", [(1, 2, 4, 4), (32, 512, 7, 7), (3, 5, 1, 1)])
def test_global_avgpool_bit_exact(dev, orc, shape):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(shape).astype(np.float32)
    y = empty(shape[:2], torch.float32)
    tbn_hip.call("tbn_hip_global_avgpool2d", P(to_dev(x)), *shape, P(y), None)
    assert np.array_equal(host(y), orc.global_avgpool2d(x))


def gpu_avgpool(x, k, s, p=(0, 0), ceil_mode=False, include_pad=False):
    N, C, H, W = x.shape
    import ctypes
    hw = (ctypes.c_int64 * 2)()
    args = [N, C, H, W, k[0], k[1], s[0], s[1], p[0], p[1], 1, 1, int(ceil_mode), int(include_pad)]
    tbn_hip.call("tbn_hip_avgpool2d", None, *args, None, hw, None)
    y = empty((N, C, hw[0], hw[1]), torch.float32)
    tbn_hip.call("tbn_hip_avgpool2d", P(to_dev(x)), *args, P(y), hw, None)
    return host(y)


@pytest.mark.parametrize("k,s,p,ceil_mode,inc", [((2, 2), (2, 2), (0, 0), False, False),
                                                 ((3, 3), (2, 2), (1, 1), False, False),
                                                 ((3, 3), (2, 2), (1, 1), False, True),
                                                 ((3, 3), (2, 2), (0, 0), True, False),
                                                 ((3, 3), (2, 2), (0, 0), True, True),
                                                 ((2, 3), (1, 2), (1, 1), False, True),
                                                 ((7, 7), (1, 1), (0, 0), False, False)])
def test_avgpool_bit_exact(dev, orc, k, s, p, ceil_mode, inc):
    """tbn::avgpool2d (pooling.cpp:83-148): same window order, same count, so
    the sums and divisions round identically."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 3, 9, 8)).astype(np.float32)
    x[1, 2, 4, 4] = np.inf
    got = gpu_avgpool(x, k, s, p, ceil_mode, inc)
    ref = orc.avgpool2d(x, k, s, p, ceil_mode=ceil_mode, count_include_pad=inc)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    xk = (np.arange(32) % 10).astype(np.float32).reshape(1, 2, 4, 4)
    assert gpu_avgpool(xk, (2, 2), (2, 2))[0, 0].reshape(-1).tolist() == [2.5, 4.5, 5.5, 2.5]


@pytest.mark.parametrize("shape", [(1, 2, 4, 4), (32, 512, 7, 7), (3, 5, 1, 1), (2, 70, 13, 11)])
def test_global_maxpool_bit_exact(dev, orc, shape):
    """tbn::global_maxpool2d (pooling.cpp:151-181): NaN ignored, -inf for an
    all-NaN plane, the first of equal -0 / +0 kept."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal(shape).astype(np.float32)
    x[0, 0].flat[0] = np.nan
    if shape[1] > 1:
        x[0, 1] = 0.0
        x[0, 1].flat[0] = -0.0
    if shape[0] > 1:
        x[-1, -1] = np.nan
    y = empty(shape[:2], torch.float32)
    tbn_hip.call("tbn_hip_global_maxpool2d", P(to_dev(x)), *shape, P(y), None)
    ref = orc.global_maxpool2d(x)
    assert np.array_equal(host(y).view(np.uint32), ref.view(np.uint32))


def test_add_broadcasts_and_relu(dev):
    rng = np.random.default_rng(4)
    a = rng.standard_normal((2, 6, 5, 5)).astype(np.float32)
    same = rng.standard_normal(a.shape).astype(np.float32)
    ch = rng.standard_normal(6).astype(np.float32)
    y = empty(a.shape, torch.float32)
    tbn_hip.call("tbn_hip_add", P(to_dev(a)), P(to_dev(same)), 1, a.size, 1, 1, 0, P(y), None)
    assert np.array_equal(host(y), a + same)
    tbn_hip.call("tbn_hip_add", P(to_dev(a)), P(to_dev(same)), 1, a.size, 1, 1, tbn_hip.EPI_RELU, P(y), None)
    assert np.array_equal(host(y), np.maximum(a + same, 0))
    tbn_hip.call("tbn_hip_add", P(to_dev(a)), P(to_dev(ch)), 2, 6, 25, 1, 0, P(y), None)
    assert np.array_equal(host(y), a + ch[None, :, None, None])
    m2 = rng.standard_normal((7, 10)).astype(np.float32)
    b1 = rng.standard_normal(10).astype(np.float32)
    y2 = empty((7, 10), torch.float32)
    tbn_hip.call("tbn_hip_add", P(to_dev(m2)), P(to_dev(b1)), 7, 10, 1, 1, 0, P(y2), None)
    assert np.array_equal(host(y2), m2 + b1)


def test_relu(dev):
    x = np.array([-1.0, 0.0, -0.0, 2.5, np.nan, -np.inf, np.inf], np.float32)
    y = empty(x.size, torch.float32)
    tbn_hip.call("tbn_hip_relu", P(to_dev(x)), x.size, P(y), None)
    out = host(y)
    assert out.tolist() == [0.0, 0.0, 0.0, 2.5, 0.0, 0.0, np.inf]
    assert not np.signbit(out[2])
