"""Grouped / depthwise convolution and BatchNormalization on the CPU: the
oracle executor's definitions (tests/models.py: the oracle's conv applied
group by group; ONNX BatchNormalization in float64) against torch's own CPU
routines in float64, an independent implementation of the same textbook
operations; and the host-side argument checks of the new C-ABI entry points.
The reference has neither operation (conv2d.cpp:372-393 throws for
groups > 1; BatchNorm folding is planned only, ADR/README.md:51)."""
import ctypes

import numpy as np
import pytest
import torch

import models
import tbn_hip


@pytest.mark.parametrize("n,c,h,w,m,g,k,stride,pad,dil", [
    (2, 8, 9, 11, 8, 8, 3, 1, 1, 1),     # depthwise
    (1, 6, 10, 7, 12, 6, 3, 2, 1, 1),    # depthwise, channel multiplier 2, stride 2
    (2, 4, 12, 12, 4, 4, 5, 1, 4, 2),    # depthwise, dilation 2
    (3, 16, 8, 8, 24, 4, 3, 1, 1, 1),    # 4 groups of 4 -> 6
    (2, 64, 6, 5, 32, 2, 1, 1, 0, 1),    # 2 groups, pointwise
])
def test_oracle_grouped_conv_matches_torch(orc, n, c, h, w, m, g, k, stride, pad, dil):
    rng = np.random.default_rng(n * 1000 + c * 10 + g)
    x = rng.standard_normal((n, c, h, w)).astype(np.float32)
    wt = rng.standard_normal((m, c // g, k, k)).astype(np.float32)
    b = rng.standard_normal(m).astype(np.float32)
    conv = models._Grouped(orc, g).conv2d_f64
    got = conv(x, wt, b, (stride, stride), (pad, pad), (dil, dil))
    want = torch.nn.functional.conv2d(torch.from_numpy(x).double(), torch.from_numpy(wt).double(),
                                      torch.from_numpy(b).double(), stride=stride, padding=pad, dilation=dil,
                                      groups=g).numpy()
    assert got.shape == want.shape
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_oracle_batchnorm_matches_torch(orc):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((3, 5, 4, 6)).astype(np.float32)
    sc, bb, mu = (rng.standard_normal(5).astype(np.float32) for _ in range(3))
    var = rng.random(5).astype(np.float32) + 0.1
    spec = models.Spec(
        nodes=[models.Node("bn", "BatchNormalization", ["x", "s", "b", "m", "v"], ["y"], {"epsilon": 1e-3})],
        inits={"s": sc, "b": bb, "m": mu, "v": var}, init_dtypes={k: "float32" for k in "sbmv"},
        inputs={"x": list(x.shape)}, outputs={"y": list(x.shape)}, value_info={"y": list(x.shape)})
    got = models.run_oracle(spec, {"x": x}, False, orc)["y"]
    want = torch.nn.functional.batch_norm(torch.from_numpy(x).double(), torch.from_numpy(mu).double(),
                                          torch.from_numpy(var).double(), torch.from_numpy(sc).double(),
                                          torch.from_numpy(bb).double(), training=False,
                                          eps=float(np.float32(1e-3))).numpy()
    np.testing.assert_allclose(got, want.astype(np.float32), rtol=1e-6, atol=1e-6)


def test_new_entry_points_check_arguments_before_device_use():
    lib = tbn_hip.lib()
    d = tbn_hip.conv_desc(1, 6, 8, 8, 9, 3, 3)  # 9 outputs over 6 channels: not a multiple
    assert lib.tbn_hip_conv2d_depthwise(None, ctypes.byref(d), None, None, 1.0, None, None, 0, None,
                                        None) == tbn_hip.INVALID_SHAPE
    d = tbn_hip.conv_desc(1, 6, 8, 8, 12, 3, 3)
    assert lib.tbn_hip_conv2d_depthwise(None, ctypes.byref(d), None, None, 1.0, None, None,
                                        tbn_hip.EPI_MAXPOOL2X2, None, None) == tbn_hip.INVALID_ARGUMENT
    d = tbn_hip.conv_desc(1, 6, 2, 2, 6, 5, 5)  # empty output
    assert lib.tbn_hip_conv2d_depthwise(None, ctypes.byref(d), None, None, 1.0, None, None, 0, None,
                                        None) == tbn_hip.INVALID_SHAPE
    d = tbn_hip.conv_desc(0, 6, 8, 8, 6, 3, 3)  # empty batch: nothing to do
    assert lib.tbn_hip_conv2d_depthwise(None, ctypes.byref(d), None, None, 1.0, None, None, 0, None, None) == 0
    assert lib.tbn_hip_copy_channels(None, 2, 8, 6, 4, 16, None, 4, 0, None) == tbn_hip.INVALID_SHAPE
    assert lib.tbn_hip_copy_channels(None, 2, 8, 0, 4, 16, None, 4, 1, None) == tbn_hip.INVALID_SHAPE
    assert lib.tbn_hip_copy_channels(None, 0, 8, 0, 4, 16, None, 4, 0, None) == 0
    assert lib.tbn_hip_channel_affine(None, 1, 4, 9, None, None, tbn_hip.EPI_BIAS_THEN_SCALE, None,
                                      None) == tbn_hip.INVALID_ARGUMENT
    assert lib.tbn_hip_channel_affine(None, 1, 0, 9, None, None, 0, None, None) == tbn_hip.INVALID_SHAPE
