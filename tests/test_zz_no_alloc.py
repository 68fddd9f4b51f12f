"""The no-allocation conv entry point (tbn_hip_conv2d_f32_quantized_noalloc,
no counterpart in the reference) against tbn_hip_conv2d_f32_quantized, whose
arguments and results it shares: same kernels, so bit-identical outputs, on
consecutive calls whose scratch needs shrink and grow again (the buffer keeps
the previous call's contents), on the narrow-input path that needs no
scratch, and with the oversize rejection."""
import numpy as np
import pytest
import torch

import refmath as rm
import tbn_hip
from gpu_util import P, empty, host, to_dev

pytestmark = pytest.mark.gpu


def _case(N, C, H, W, M, k, pad, flags, residual, seed, ternary=False):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    K = C * k * k
    K_pad, N_pad = tbn_hip.padded_dims(K, M)
    if ternary:
        t = rng.choice(np.int8([-1, 0, 1]), size=(M, K), p=[0.3, 0.4, 0.3])
        packed = empty(N_pad * K_pad // 4, torch.uint8)
        tbn_hip.call("tbn_hip_pack_ternary", P(to_dev(t)), K, M, tbn_hip.LAYOUT_NK, K_pad, N_pad, P(packed), None)
        wref = t.astype(np.float32).reshape(M, C, k, k)
    else:
        wb = (rng.random((M, K)) < 0.5).astype(np.uint8)
        packed = empty(N_pad * K_pad // 8, torch.uint8)
        tbn_hip.call("tbn_hip_pack_binary", P(to_dev(wb)), K, M, tbn_hip.LAYOUT_NK, K_pad, N_pad, P(packed), None)
        wref = np.where(wb == 1, 1.0, -1.0).astype(np.float32).reshape(M, C, k, k)
    scale = rng.uniform(0.5, 1.5, M).astype(np.float32)
    bias = (rng.standard_normal(M) * 0.01).astype(np.float32)
    d = tbn_hip.conv_desc(N, C, H, W, M, k, k, 1, 1, pad, pad)
    OH, OW = tbn_hip.conv_out_hw(d)
    oshape = (N, M, OH // 2, OW // 2) if flags & tbn_hip.EPI_MAXPOOL2X2 else (N, M, OH, OW)
    res = rng.standard_normal((N, M, OH, OW)).astype(np.float32) if residual else None
    return dict(x=x, dx=to_dev(x), d=d, packed=packed, K_pad=K_pad, N_pad=N_pad, ds=to_dev(scale),
                db=to_dev(bias), dres=None if res is None else to_dev(res), flags=flags, oshape=oshape,
                kind=tbn_hip.WEIGHTS_TERNARY if ternary else tbn_hip.WEIGHTS_BINARY, K=K, wref=wref, scale=scale,
                bias=bias, res=res, pad=pad)


def _run(c, entry):
    y = empty(c["oshape"], torch.float32)
    y.fill_(np.nan)
    tbn_hip.call(entry, c["kind"], P(c["dx"]), c["d"], P(c["packed"]), c["K_pad"], c["N_pad"], P(c["ds"]), 1.0,
                 P(c["db"]), P(c["dres"]), c["flags"], P(y), None)
    return host(y)


def _check_vs_oracle(c, y):
    acc = rm.f64_conv(c["x"], c["wref"], None, (1, 1), (c["pad"], c["pad"]))
    s = c["scale"].astype(np.float64)[None, :, None, None]
    b = c["bias"].astype(np.float64)[None, :, None, None]
    ref = (acc + b) * s if c["flags"] & tbn_hip.EPI_BIAS_THEN_SCALE else acc * s + b
    if c["res"] is not None:
        ref = ref + c["res"]
    if c["flags"] & tbn_hip.EPI_RELU:
        ref = np.maximum(ref, 0.0)
    if c["flags"] & tbn_hip.EPI_MAXPOOL2X2:
        n, m, oh, ow = ref.shape
        ref = ref[:, :, :oh // 2 * 2, :ow // 2 * 2].reshape(n, m, oh // 2, 2, ow // 2, 2).max(axis=(3, 5))
    rm.assert_within_tolerance(y, ref, c["K"], np.abs(c["x"]).max() * 1.5 + (0 if c["res"] is None else 1))


def test_noalloc_conv_matches_allocating_entry_point(dev):
    R, BS = tbn_hip.EPI_RELU, tbn_hip.EPI_BIAS_THEN_SCALE
    big = _case(4, 512, 7, 7, 512, 3, 1, R | BS, True, 1)               # split K: weights + partial sums
    small = _case(8, 64, 14, 14, 128, 3, 1, R, False, 2)                # config-4 layer: weights only
    ternary = _case(2, 256, 7, 7, 96, 3, 1, R, False, 3, ternary=True)  # 2-bit weights, split K
    pooled = _case(3, 96, 12, 10, 64, 3, 1, tbn_hip.EPI_MAXPOOL2X2, False, 4)
    narrow = _case(1, 6, 12, 12, 16, 5, 0, R | tbn_hip.EPI_MAXPOOL2X2, False, 5)  # C < 16: no scratch used
    for c in (big, small, big, ternary, pooled, small, narrow):
        want = _run(c, "tbn_hip_conv2d_f32_quantized")
        got = _run(c, "tbn_hip_conv2d_f32_quantized_noalloc")
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), c["d"]
    for c in (big, small, ternary, pooled, narrow):
        _check_vs_oracle(c, _run(c, "tbn_hip_conv2d_f32_quantized_noalloc"))


def test_noalloc_conv_rejects_oversize_scratch(dev):
    # 256 images x 512 x 7 x 7 with 2 K splits forced (the batch alone would
    # run its chunk groups in one block, with no partial sums): 51 MB of
    # partial sums > 16 MiB
    d = tbn_hip.conv_desc(256, 512, 7, 7, 512, 3, 3, 1, 1, 1, 1)
    x = empty((256, 512, 7, 7), torch.float32)
    y = empty((256, 512, 7, 7), torch.float32)
    K_pad, N_pad = tbn_hip.padded_dims(512 * 9, 512)
    packed = empty(N_pad * K_pad // 8, torch.uint8)
    with tbn_hip.tuning(tbn_hip.TUNE_CONV_SPLITS, 2):
        rc = tbn_hip.lib().tbn_hip_conv2d_f32_quantized_noalloc(tbn_hip.WEIGHTS_BINARY, P(x), d, P(packed), K_pad,
                                                                N_pad, None, 1.0, None, None, 0, P(y), None)
        msg = tbn_hip.last_error()  # before the control's reset clears it
    assert rc == tbn_hip.INVALID_SHAPE
    assert "scratch" in msg
