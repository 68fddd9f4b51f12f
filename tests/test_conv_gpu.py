"""Implicit-GEMM Conv2D on the GPU vs the oracle (north_star subsystem 3).

Reference semantics (mode F32): the reference's fp32 conv2d (conv2d.cpp:78-192)
applied to the dequantized weights s[m]*sign(w), i.e. y = s*acc + b
(conv2d_binary_with_scales order, conv2d.cpp:319-369), then ReLU / MaxPool.
Tolerance: rel-L2 <= 1e-5, max-abs <= 1e-4*sqrt(K)*max|x|*max|s|."""
import re

import numpy as np
import pytest
import torch

import refmath as rm
import tbn_hip
from gpu_util import P, empty, host, to_dev

pytestmark = pytest.mark.gpu


def pack_conv_weights(w_sign_bytes, M, K):
    K_pad, N_pad = tbn_hip.padded_dims(K, M)
    packed = empty(N_pad * K_pad // 8, torch.uint8)
    tbn_hip.call("tbn_hip_pack_binary", P(to_dev(w_sign_bytes)), K, M, tbn_hip.LAYOUT_NK, K_pad, N_pad,
                 P(packed), None)
    return packed, K_pad, N_pad


def conv_ref(x, wsign, scale, alpha, bias, stride, pad, dil, flags):
    acc = rm.f64_conv(x, wsign, None, stride, pad, dil)
    mult = (np.float32(alpha) * scale.astype(np.float32)).astype(np.float64)[None, :, None, None]
    b = bias.astype(np.float64)[None, :, None, None]
    y = (acc + b) * mult if flags & tbn_hip.EPI_BIAS_THEN_SCALE else acc * mult + b
    if flags & tbn_hip.EPI_RELU:
        y = np.maximum(y, 0.0)
    if flags & tbn_hip.EPI_MAXPOOL2X2:
        N, M, OH, OW = y.shape
        y = y[:, :, :OH // 2 * 2, :OW // 2 * 2].reshape(N, M, OH // 2, 2, OW // 2, 2).max(axis=(3, 5))
    return y


CASES = [
    # N, C, H, W, M, kh, kw, stride, pad, dil, flags
    (64, 64, 14, 14, 128, 3, 3, (1, 1), (1, 1), (1, 1), tbn_hip.EPI_RELU),        # config 4
    (1, 1, 28, 28, 6, 5, 5, (1, 1), (0, 0), (1, 1), tbn_hip.EPI_RELU | tbn_hip.EPI_MAXPOOL2X2),  # LeNet conv1
    (1, 6, 12, 12, 16, 5, 5, (1, 1), (0, 0), (1, 1), tbn_hip.EPI_RELU | tbn_hip.EPI_MAXPOOL2X2),  # LeNet conv2
    (4, 64, 56, 56, 128, 3, 3, (2, 2), (1, 1), (1, 1), tbn_hip.EPI_RELU),          # ResNet downsample
    (4, 64, 56, 56, 128, 1, 1, (2, 2), (0, 0), (1, 1), 0),                          # 1x1 projection
    (2, 128, 28, 28, 128, 3, 3, (1, 1), (1, 1), (1, 1), tbn_hip.EPI_BIAS_THEN_SCALE),
    (2, 5, 13, 11, 40, 3, 2, (2, 1), (1, 0), (2, 2), tbn_hip.EPI_RELU),            # odd everything
    (3, 7, 9, 9, 70, 3, 3, (1, 1), (1, 1), (1, 1), tbn_hip.EPI_MAXPOOL2X2),        # odd output, floor pool
    # K split over blocks (deep layers): 8 chunks -> 2 splits, 16 chunks -> 4
    (3, 256, 7, 7, 96, 3, 3, (1, 1), (1, 1), (1, 1), tbn_hip.EPI_RELU),
    (2, 512, 7, 7, 72, 3, 3, (1, 1), (1, 1), (1, 1), tbn_hip.EPI_BIAS_THEN_SCALE),
    (2, 300, 9, 8, 40, 3, 3, (2, 2), (1, 1), (1, 1), 0),                            # ragged last split
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[:7])))
def test_conv_binary(dev, orc, case):
    N, C, H, W, M, kh, kw, stride, pad, dil, flags = case
    rng = np.random.default_rng(N * 131 + C * 7 + M)
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    wbytes = (rng.random((M, C, kh, kw)) < 0.5).astype(np.uint8)
    wsign = np.where(wbytes == 1, 1.0, -1.0).astype(np.float32)
    scale = rng.uniform(0.5, 1.5, M).astype(np.float32)
    bias = (rng.standard_normal(M) * 0.01).astype(np.float32)
    K = C * kh * kw
    packed, K_pad, N_pad = pack_conv_weights(wbytes, M, K)
    d = tbn_hip.conv_desc(N, C, H, W, M, kh, kw, *stride, *pad, *dil)
    OH, OW = tbn_hip.conv_out_hw(d)
    oshape = (N, M, OH // 2, OW // 2) if flags & tbn_hip.EPI_MAXPOOL2X2 else (N, M, OH, OW)
    y = empty(oshape, torch.float32)
    y.fill_(np.nan)
    tbn_hip.call("tbn_hip_conv2d_f32_binary", P(to_dev(x)), d, P(packed), K_pad, N_pad, P(to_dev(scale)), 1.0,
                 P(to_dev(bias)), flags, P(y), None)
    ref = conv_ref(x, wsign, scale, 1.0, bias, stride, pad, dil, flags)
    rm.assert_within_tolerance(host(y), ref, K, np.abs(x).max() * 1.5)
    if case[0] == 64:
        # fp32 reference operator on dequantized weights (conv2d.cpp:78-192) is within the same bound
        y32 = orc.conv2d_f32(x[:2], wsign * scale[:, None, None, None], bias, stride, pad, dil)
        rm.assert_within_tolerance(host(y)[:2], np.maximum(y32, 0), K, np.abs(x).max() * 1.5)


def test_conv_ternary(dev, orc):
    rng = np.random.default_rng(77)
    N, C, H, W, M, kh, kw = 2, 16, 10, 10, 48, 3, 3
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    t = rng.choice(np.array([-1, 0, 1], np.int8), size=(M, C, kh, kw), p=[0.3, 0.4, 0.3])
    scale = rng.uniform(0.5, 1.5, M).astype(np.float32)
    bias = (rng.standard_normal(M) * 0.01).astype(np.float32)
    K = C * kh * kw
    K_pad = (K + 31) // 32 * 32
    packed = empty(M * K_pad // 4, torch.uint8)
    tbn_hip.call("tbn_hip_pack_ternary", P(to_dev(t)), K, M, tbn_hip.LAYOUT_NK, K_pad, M, P(packed), None)
    d = tbn_hip.conv_desc(N, C, H, W, M, kh, kw, 1, 1, 1, 1)
    y = empty((N, M, H, W), torch.float32)
    tbn_hip.call("tbn_hip_conv2d_f32_ternary", P(to_dev(x)), d, P(packed), K_pad, M, P(to_dev(scale)), 1.0,
                 P(to_dev(bias)), tbn_hip.EPI_RELU, P(y), None)
    ref = conv_ref(x, t.astype(np.float32), scale, 1.0, bias, (1, 1), (1, 1), (1, 1), tbn_hip.EPI_RELU)
    rm.assert_within_tolerance(host(y), ref, K, np.abs(x).max() * 1.5)


@pytest.mark.parametrize("case", [(2, 3, 64, 64, 64, 7, 7, 2, 3, 0), (1, 1, 28, 28, 6, 5, 5, 1, 0, 4),
                                  (2, 8, 9, 9, 40, 3, 3, 1, 1, 1),
                                  # the stem kernel: partial tiles, M < 64, ReLU
                                  (3, 3, 70, 50, 64, 7, 7, 2, 3, 1), (1, 3, 33, 37, 40, 7, 7, 2, 3, 0),
                                  (2, 3, 224, 224, 64, 7, 7, 2, 3, 1)])
def test_conv_f32(dev, orc, case):
    """fp32 layers (ResNet stem 7x7/2, LeNet with quantization off)."""
    N, C, H, W, M, kh, kw, s, p, flags = case
    rng = np.random.default_rng(M + C)
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    w = (rng.standard_normal((M, C, kh, kw)) * np.sqrt(2.0 / (C * kh * kw))).astype(np.float32)
    b = (rng.standard_normal(M) * 0.01).astype(np.float32)
    d = tbn_hip.conv_desc(N, C, H, W, M, kh, kw, s, s, p, p)
    OH, OW = tbn_hip.conv_out_hw(d)
    pool = flags & tbn_hip.EPI_MAXPOOL2X2
    y = empty((N, M, OH // 2, OW // 2) if pool else (N, M, OH, OW), torch.float32)
    tbn_hip.call("tbn_hip_conv2d_f32", P(to_dev(x)), d, P(to_dev(w)), P(to_dev(b)), flags, P(y), None)
    ref = orc.conv2d_f64(x, w, b, (s, s), (p, p))
    if flags & tbn_hip.EPI_RELU:
        ref = np.maximum(ref, 0.0)
    if pool:
        ref = ref[:, :, :OH // 2 * 2, :OW // 2 * 2].reshape(N, M, OH // 2, 2, OW // 2, 2).max(axis=(3, 5))
    rm.assert_within_tolerance(host(y), ref, C * kh * kw, np.abs(x).max() * np.abs(w).max())


def _np_conv_layout_bits(wbytes, M_alloc):
    """Closed form of the conv weight layout: one 4-byte word per
    (step = (c // 32) * kh*kw + r*kw + s, output channel m), words ordered
    [step][m], bit c % 32 of the word set iff the weight is -1."""
    M, C, kh, kw = wbytes.shape
    chunks = (C + 31) // 32
    full = np.zeros((M_alloc, chunks, 32, kh * kw), np.uint8)  # [m, chunk, c%32, tap]
    t = (wbytes != 1).reshape(M, C, kh * kw)
    padded = np.zeros((M, chunks * 32, kh * kw), np.uint8)
    padded[:, :C] = t
    full[:M] = padded.reshape(M, chunks, 32, kh * kw)
    neg = full.transpose(0, 1, 3, 2).reshape(M_alloc, -1)  # [m, chunk, tap, c%32]
    words = np.packbits(neg, axis=1, bitorder="little").reshape(M_alloc, -1, 4)  # [m, step, 4 bytes]
    return words.transpose(1, 0, 2).reshape(-1)


@pytest.mark.parametrize("case", [(2, 16, 9, 9, 40, 3, 3, (1, 1), (1, 1), (1, 1), tbn_hip.EPI_RELU),
                                  (3, 40, 10, 7, 33, 3, 3, (2, 2), (1, 1), (1, 1), tbn_hip.EPI_MAXPOOL2X2),
                                  (2, 64, 8, 8, 200, 1, 1, (1, 1), (0, 0), (1, 1), 0),
                                  (1, 32, 12, 12, 16, 3, 3, (1, 1), (2, 2), (2, 2), tbn_hip.EPI_BIAS_THEN_SCALE),
                                  (2, 96, 19, 23, 72, 5, 5, (1, 2), (2, 2), (1, 1), tbn_hip.EPI_RELU)])
def test_conv_prepacked_entry_point(dev, orc, case):
    """Pre-packed conv-layout weights: tbn_hip_pack_conv_weights matches the
    closed form bit for bit, and tbn_hip_conv2d_f32_prepacked equals
    tbn_hip_conv2d_f32_binary bitwise (same kernel) and the float64 oracle
    within tolerance."""
    import ctypes
    N, C, H, W, M, kh, kw, stride, pad, dil, flags = case
    rng = np.random.default_rng(C * 1000 + M)
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    wbytes = (rng.random((M, C, kh, kw)) < 0.5).astype(np.uint8)
    scale = rng.uniform(0.5, 1.5, M).astype(np.float32)
    bias = (rng.standard_normal(M) * 0.01).astype(np.float32)
    K = C * kh * kw
    packed, K_pad, N_pad = pack_conv_weights(wbytes, M, K)
    d = tbn_hip.conv_desc(N, C, H, W, M, kh, kw, *stride, *pad, *dil)
    wb = ctypes.c_int64()
    tbn_hip.call("tbn_hip_conv_weights_bytes", tbn_hip.WEIGHTS_BINARY, d, ctypes.byref(wb))
    M_alloc = (M + 7) // 8 * 8
    assert wb.value == M_alloc * ((C + 31) // 32) * kh * kw * 32 // 8
    cw = empty(wb.value, torch.uint8)
    tbn_hip.call("tbn_hip_pack_conv_weights", tbn_hip.WEIGHTS_BINARY, P(packed), K_pad, N_pad, d, P(cw), None)
    assert np.array_equal(host(cw), _np_conv_layout_bits(wbytes, M_alloc))
    OH, OW = tbn_hip.conv_out_hw(d)
    oshape = (N, M, OH // 2, OW // 2) if flags & tbn_hip.EPI_MAXPOOL2X2 else (N, M, OH, OW)
    dx, ds, db = to_dev(x), to_dev(scale), to_dev(bias)
    y1 = empty(oshape, torch.float32)
    y2 = empty(oshape, torch.float32)
    y1.fill_(np.nan)
    tbn_hip.call("tbn_hip_conv2d_f32_prepacked", tbn_hip.WEIGHTS_BINARY, P(dx), d, P(cw), P(ds), 1.0, P(db), None,
                 flags, P(y1), None)
    tbn_hip.call("tbn_hip_conv2d_f32_binary", P(dx), d, P(packed), K_pad, N_pad, P(ds), 1.0, P(db), flags, P(y2), None)
    assert np.array_equal(host(y1), host(y2))
    wsign = np.where(wbytes == 1, 1.0, -1.0).astype(np.float32)
    ref = conv_ref(x, wsign, scale, 1.0, bias, stride, pad, dil, flags)
    rm.assert_within_tolerance(host(y1), ref, K, np.abs(x).max() * 1.5)


def test_conv_patch_residual_epilogue(dev, orc):
    """Residual add fused after scale/bias and before ReLU (the Session's Conv + Add + Relu)."""
    rng = np.random.default_rng(5)
    N, C, H, W, M = 2, 32, 10, 10, 32
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    res = rng.standard_normal((N, M, H, W)).astype(np.float32)
    wbytes = (rng.random((M, C, 3, 3)) < 0.5).astype(np.uint8)
    scale = rng.uniform(0.5, 1.5, M).astype(np.float32)
    bias = (rng.standard_normal(M) * 0.01).astype(np.float32)
    K = C * 9
    packed, K_pad, N_pad = pack_conv_weights(wbytes, M, K)
    d = tbn_hip.conv_desc(N, C, H, W, M, 3, 3, 1, 1, 1, 1)
    y = empty((N, M, H, W), torch.float32)
    flags = tbn_hip.EPI_RELU | tbn_hip.EPI_BIAS_THEN_SCALE
    tbn_hip.call("tbn_hip_conv2d_f32_quantized", tbn_hip.WEIGHTS_BINARY, P(to_dev(x)), d, P(packed), K_pad, N_pad,
                 P(to_dev(scale)), 1.0, P(to_dev(bias)), P(to_dev(res)), flags, P(y), None)
    wsign = np.where(wbytes == 1, 1.0, -1.0).astype(np.float32)
    ref = conv_ref(x, wsign, scale, 1.0, bias, (1, 1), (1, 1), (1, 1), tbn_hip.EPI_BIAS_THEN_SCALE)
    ref = np.maximum(ref + res, 0.0)
    rm.assert_within_tolerance(host(y), ref, K, np.abs(x).max() * 1.5)


@pytest.mark.parametrize("case", [(3, 40, 10, 7, 33, 3, 3, (1, 1), (1, 1), (1, 1), tbn_hip.EPI_RELU),
                                  (2, 40, 11, 9, 70, 3, 3, (1, 1), (1, 1), (1, 1), tbn_hip.EPI_MAXPOOL2X2),
                                  (2, 64, 8, 8, 200, 1, 1, (2, 2), (0, 0), (1, 1), 0)])
def test_conv_patch_writes_only_its_output(dev, orc, case):
    """Masked lanes (rows past M, pixels past the image, pooled-away lanes)
    store nothing: a guard region after the output keeps its sentinel, and
    every output element is written (NaN fill replaced)."""
    import ctypes
    N, C, H, W, M, kh, kw, stride, pad, dil, flags = case
    rng = np.random.default_rng(M)
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    wbytes = (rng.random((M, C, kh, kw)) < 0.5).astype(np.uint8)
    scale = rng.uniform(0.5, 1.5, M).astype(np.float32)
    packed, K_pad, N_pad = pack_conv_weights(wbytes, M, C * kh * kw)
    d = tbn_hip.conv_desc(N, C, H, W, M, kh, kw, *stride, *pad, *dil)
    OH, OW = tbn_hip.conv_out_hw(d)
    oshape = (N, M, OH // 2, OW // 2) if flags & tbn_hip.EPI_MAXPOOL2X2 else (N, M, OH, OW)
    n_out = int(np.prod(oshape))
    guard = 1 << 16
    buf = empty(n_out + guard, torch.float32)
    buf.fill_(np.nan)
    buf[n_out:].fill_(-12345.0)
    tbn_hip.call("tbn_hip_conv2d_f32_binary", P(to_dev(x)), d, P(packed), K_pad, N_pad, P(to_dev(scale)), 1.0, None,
                 flags, P(buf), None)
    out = host(buf)
    assert np.all(out[n_out:] == -12345.0)
    assert not np.isnan(out[:n_out]).any()


@pytest.mark.parametrize("case", [
    # N, C, H, W, M, kh, kw, stride, pad, dil, flags
    (3, 5, 13, 11, 24, 3, 3, (2, 1), (2, 1), (1, 2), tbn_hip.EPI_RELU | tbn_hip.EPI_MAXPOOL2X2),
    (2, 15, 8, 8, 40, 3, 3, (1, 1), (1, 1), (1, 1), tbn_hip.EPI_BIAS_THEN_SCALE | tbn_hip.EPI_RELU),
    (5, 1, 28, 28, 6, 5, 5, (1, 1), (2, 2), (1, 1), tbn_hip.EPI_RELU | tbn_hip.EPI_MAXPOOL2X2),
    (2, 3, 7, 9, 130, 1, 1, (1, 1), (0, 0), (1, 1), 0),  # 1x1: many channels per block
])
@pytest.mark.parametrize("weights", ["binary", "ternary", "f32"])
def test_conv_small_layers(dev, orc, case, weights):
    """Small layers (C < 16, a padded image of <= 8192 floats, <= 16384
    outputs per image) take the one-output-per-thread LDS kernel: padding,
    stride, dilation, fused pool, the scale/bias orders, a residual where the
    entry point takes one; each image's result is bit-identical to the same
    image run alone (the path depends on one image's shape only)."""
    N, C, H, W, M, kh, kw, stride, pad, dil, flags = case
    rng = np.random.default_rng(N * 7 + C * 3 + M)
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    K = C * kh * kw
    scale = rng.uniform(0.5, 1.5, M).astype(np.float32)
    bias = (rng.standard_normal(M) * 0.1).astype(np.float32)
    d = tbn_hip.conv_desc(N, C, H, W, M, kh, kw, *stride, *pad, *dil)
    OH, OW = tbn_hip.conv_out_hw(d)
    pool = bool(flags & tbn_hip.EPI_MAXPOOL2X2)
    oshape = (N, M, OH // 2, OW // 2) if pool else (N, M, OH, OW)
    res = None if pool or weights == "f32" else rng.standard_normal((N, M, OH, OW)).astype(np.float32)
    if weights == "f32":
        wf = (rng.standard_normal((M, C, kh, kw)) * 0.3).astype(np.float32)
        dw = to_dev(wf)
        flags &= ~tbn_hip.EPI_BIAS_THEN_SCALE

        def run(xs, n):
            y = empty((n,) + oshape[1:], torch.float32)
            dn = tbn_hip.conv_desc(n, C, H, W, M, kh, kw, *stride, *pad, *dil)
            tbn_hip.call("tbn_hip_conv2d_f32", P(to_dev(xs)), dn, P(dw), P(to_dev(bias)), flags, P(y), None)
            return host(y)
        acc = rm.f64_conv(x, wf, None, stride, pad, dil)
        ref = acc + bias.astype(np.float64)[None, :, None, None]
        xmax = np.abs(x).max() * np.abs(wf).max()
    else:
        K_pad = (K + 31) // 32 * 32
        if weights == "binary":
            wbytes = (rng.random((M, C, kh, kw)) < 0.5).astype(np.uint8)
            wv = np.where(wbytes == 1, 1.0, -1.0).astype(np.float32)
            packed, K_pad, N_pad = pack_conv_weights(wbytes, M, K)
            kind = tbn_hip.WEIGHTS_BINARY
        else:
            t = rng.choice(np.array([-1, 0, 1], np.int8), size=(M, C, kh, kw), p=[0.3, 0.4, 0.3])
            wv = t.astype(np.float32)
            N_pad = M
            packed = empty(M * K_pad // 4, torch.uint8)
            tbn_hip.call("tbn_hip_pack_ternary", P(to_dev(t)), K, M, tbn_hip.LAYOUT_NK, K_pad, M, P(packed), None)
            kind = tbn_hip.WEIGHTS_TERNARY
        ds, db = to_dev(scale), to_dev(bias)

        def run(xs, n, rs=None):
            y = empty((n,) + oshape[1:], torch.float32)
            dn = tbn_hip.conv_desc(n, C, H, W, M, kh, kw, *stride, *pad, *dil)
            tbn_hip.call("tbn_hip_conv2d_f32_quantized", kind, P(to_dev(xs)), dn, P(packed), K_pad, N_pad, P(ds), 0.75,
                         P(db), None if rs is None else P(to_dev(rs)), flags, P(y), None)
            return host(y)
        acc = rm.f64_conv(x, wv, None, stride, pad, dil)
        mult = (np.float32(0.75) * scale).astype(np.float64)[None, :, None, None]
        b = bias.astype(np.float64)[None, :, None, None]
        ref = (acc + b) * mult if flags & tbn_hip.EPI_BIAS_THEN_SCALE else acc * mult + b
        if res is not None:
            ref = ref + res
        xmax = np.abs(x).max() * 1.5
    if flags & tbn_hip.EPI_RELU:
        ref = np.maximum(ref, 0.0)
    if pool:
        ref = ref[:, :, :OH // 2 * 2, :OW // 2 * 2].reshape(N, M, OH // 2, 2, OW // 2, 2).max(axis=(3, 5))
    out = run(x, N) if res is None else run(x, N, res)
    assert out.shape == oshape
    rm.assert_within_tolerance(out, ref, K, xmax)
    one = run(x[1:2].copy(), 1) if res is None else run(x[1:2].copy(), 1, res[1:2].copy())
    assert np.array_equal(one.view(np.uint32), out[1:2].view(np.uint32))


@pytest.mark.parametrize("case", [(2, 224, 224, 64), (1, 65, 47, 40), (3, 30, 34, 64), (1, 9, 9, 8),
                                  (1, 40, 46, 64)])
def test_conv_f32_stem_maxpool3x3s2_fused(dev, orc, case):
    """The stem conv with ReLU and the 3x3/2 pad-1 max pool fused
    (TBN_EPI_MAXPOOL3X3S2; the pool of model.hpp:577-629) equals the stem
    conv with ReLU followed by the oracle's maxpool2d bit for bit: after the
    ReLU every value is +0 or more and none is NaN, so the order the maximum
    is taken in does not matter.  The input holds NaN, +-inf and -0.0; pooled
    widths divisible by 4 take the 16-byte store path, the others 4-byte
    stores; partial tiles at the bottom and right, M < 64."""
    N, H, W, M = case
    rng = np.random.default_rng(H * W + M)
    x = rng.standard_normal((N, 3, H, W)).astype(np.float32)
    flat = x.reshape(-1)
    flat[rng.choice(flat.size, 6, replace=False)] = [np.nan, np.inf, -np.inf, -0.0, np.nan, 0.0]
    w = (rng.standard_normal((M, 3, 7, 7)) * 0.1).astype(np.float32)
    b = (rng.standard_normal(M) * 0.05).astype(np.float32)
    d = tbn_hip.conv_desc(N, 3, H, W, M, 7, 7, 2, 2, 3, 3)
    OH, OW = tbn_hip.conv_out_hw(d)
    PH, PW = (OH - 1) // 2 + 1, (OW - 1) // 2 + 1
    dx, dw, db = to_dev(x), to_dev(w), to_dev(b)
    conv = empty((N, M, OH, OW), torch.float32)
    tbn_hip.call("tbn_hip_conv2d_f32", P(dx), d, P(dw), P(db), tbn_hip.EPI_RELU, P(conv), None)
    y = empty((N, M, PH, PW), torch.float32)
    y.fill_(np.nan)  # every output is written
    tbn_hip.call("tbn_hip_conv2d_f32", P(dx), d, P(dw), P(db), tbn_hip.EPI_RELU | tbn_hip.EPI_MAXPOOL3X3S2, P(y),
                 None)
    ref = orc.maxpool2d(host(conv), (3, 3), (2, 2), (1, 1))
    assert ref.shape == (N, M, PH, PW)
    got = host(y)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_conv_f32_stem_inf_stays_local(dev, orc):
    """An infinite input pixel reaches only the outputs whose 7x7 window
    holds it: the stem kernel's padded tap columns (kw = 7 of 8) and padded
    k rows carry zero weights and zero inputs, never inf * 0."""
    N, C, H, W, M = 1, 3, 40, 40, 64
    rng = np.random.default_rng(9)
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    w = (rng.standard_normal((M, C, 7, 7)) * 0.1).astype(np.float32)
    b = np.zeros(M, np.float32)
    ih, iw = 21, 18
    x[0, 1, ih, iw] = np.inf
    d = tbn_hip.conv_desc(N, C, H, W, M, 7, 7, 2, 2, 3, 3)
    OH, OW = tbn_hip.conv_out_hw(d)
    y = empty((N, M, OH, OW), torch.float32)
    tbn_hip.call("tbn_hip_conv2d_f32", P(to_dev(x)), d, P(to_dev(w)), P(to_dev(b)), 0, P(y), None)
    out = host(y)
    oh = np.arange(OH)[:, None]
    ow = np.arange(OW)[None, :]
    touched = (np.abs(2 * oh - 3 + 3 - ih) <= 3) & (np.abs(2 * ow - 3 + 3 - iw) <= 3)
    assert np.all(np.isfinite(out[:, :, ~touched]))
    assert not np.any(np.isfinite(out[:, :, touched]))
    x0 = x.copy()
    x0[0, 1, ih, iw] = 0.0
    ref = orc.conv2d_f64(x0, w, b, (2, 2), (3, 3))
    rm.assert_within_tolerance(np.where(touched, 0.0, out), np.where(touched, 0.0, ref), C * 49,
                               np.abs(x0).max() * np.abs(w).max())


def test_conv_patch_split_k_residual_and_ternary(dev, orc):
    """Split-K with the residual epilogue (binary) and with ternary weights:
    the reduce applies scale, bias, residual and ReLU after adding the splits."""
    rng = np.random.default_rng(11)
    N, C, H, W, M = 2, 512, 7, 7, 64
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    res = rng.standard_normal((N, M, H, W)).astype(np.float32)
    wbytes = (rng.random((M, C, 3, 3)) < 0.5).astype(np.uint8)
    scale = rng.uniform(0.5, 1.5, M).astype(np.float32)
    bias = (rng.standard_normal(M) * 0.01).astype(np.float32)
    K = C * 9
    packed, K_pad, N_pad = pack_conv_weights(wbytes, M, K)
    d = tbn_hip.conv_desc(N, C, H, W, M, 3, 3, 1, 1, 1, 1)
    y = empty((N, M, H, W), torch.float32)
    tbn_hip.call("tbn_hip_conv2d_f32_quantized", tbn_hip.WEIGHTS_BINARY, P(to_dev(x)), d, P(packed), K_pad, N_pad,
                 P(to_dev(scale)), 1.0, P(to_dev(bias)), P(to_dev(res)), tbn_hip.EPI_RELU, P(y), None)
    wsign = np.where(wbytes == 1, 1.0, -1.0).astype(np.float32)
    ref = conv_ref(x, wsign, scale, 1.0, bias, (1, 1), (1, 1), (1, 1), 0)
    rm.assert_within_tolerance(host(y), np.maximum(ref + res, 0.0), K, np.abs(x).max() * 1.5)
    # ternary weights through the same split path
    t = rng.integers(-1, 2, (M, C * 9)).astype(np.int8)
    K_pad = (K + 31) // 32 * 32
    tp = empty(M * K_pad // 4, torch.uint8)
    tbn_hip.call("tbn_hip_pack_ternary", P(to_dev(t)), K, M, tbn_hip.LAYOUT_NK, K_pad, M, P(tp), None)
    y2 = empty((N, M, H, W), torch.float32)
    tbn_hip.call("tbn_hip_conv2d_f32_ternary", P(to_dev(x)), d, P(tp), K_pad, M, P(to_dev(scale)), 1.0,
                 P(to_dev(bias)), 0, P(y2), None)
    ref2 = conv_ref(x, t.reshape(M, C, 3, 3).astype(np.float32), scale, 1.0, bias, (1, 1), (1, 1), (1, 1), 0)
    rm.assert_within_tolerance(host(y2), ref2, K, np.abs(x).max() * 1.5)


@pytest.mark.parametrize("case", [(2, 64, 14, 14, 128, 3, 3, (1, 1), (1, 1), (1, 1), tbn_hip.EPI_RELU),
                                  (3, 96, 12, 10, 64, 3, 3, (1, 1), (1, 1), (1, 1), tbn_hip.EPI_MAXPOOL2X2),
                                  (2, 256, 7, 7, 96, 3, 3, (1, 1), (1, 1), (1, 1), tbn_hip.EPI_BIAS_THEN_SCALE),
                                  (2, 64, 15, 13, 64, 1, 1, (2, 2), (0, 0), (1, 1), 0),
                                  # stacked tiles: runs across image boundaries (7x9 images
                                  # smaller than a tile), dilation with the full zero band,
                                  # no padding, a 5x5 kernel, a 1x1 kernel, many chunks
                                  (5, 64, 7, 9, 64, 3, 3, (1, 1), (1, 1), (1, 1), tbn_hip.EPI_RELU),
                                  (2, 32, 9, 11, 128, 3, 3, (1, 1), (2, 2), (2, 2), 0),
                                  (3, 32, 10, 10, 64, 3, 3, (1, 1), (0, 0), (1, 1), tbn_hip.EPI_RELU),
                                  (2, 32, 11, 12, 64, 5, 5, (1, 1), (2, 1), (1, 1), 0),
                                  (3, 96, 6, 13, 128, 1, 1, (1, 1), (0, 0), (1, 1), tbn_hip.EPI_RELU),
                                  (2, 256, 14, 14, 128, 3, 3, (1, 1), (1, 1), (1, 1), tbn_hip.EPI_BIAS_THEN_SCALE)])
def test_conv_patch_every_tile_gives_the_same_bits(dev, orc, case):
    """Each tile of the menu (forced with the conv-tile control: linear, 2-D
    and stacked tiles, with two LDS buffers or one) sums every output in the
    same order, so all feasible tiles give
    bit-identical outputs; one of them is checked against the float64 oracle."""
    N, C, H, W, M, kh, kw, stride, pad, dil, flags = case
    rng = np.random.default_rng(C * 17 + M)
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    wbytes = (rng.random((M, C, kh, kw)) < 0.5).astype(np.uint8)
    scale = rng.uniform(0.5, 1.5, M).astype(np.float32)
    bias = (rng.standard_normal(M) * 0.01).astype(np.float32)
    K = C * kh * kw
    packed, K_pad, N_pad = pack_conv_weights(wbytes, M, K)
    d = tbn_hip.conv_desc(N, C, H, W, M, kh, kw, *stride, *pad, *dil)
    OH, OW = tbn_hip.conv_out_hw(d)
    oshape = (N, M, OH // 2, OW // 2) if flags & tbn_hip.EPI_MAXPOOL2X2 else (N, M, OH, OW)
    import ctypes
    wb = ctypes.c_int64()
    tbn_hip.call("tbn_hip_conv_weights_bytes", tbn_hip.WEIGHTS_BINARY, d, ctypes.byref(wb))
    cw = empty(wb.value, torch.uint8)
    tbn_hip.call("tbn_hip_pack_conv_weights", tbn_hip.WEIGHTS_BINARY, P(packed), K_pad, N_pad, d, P(cw), None)
    dx, ds, db = to_dev(x), to_dev(scale), to_dev(bias)
    outs = {}
    for tile in range(128):
        with tbn_hip.tuning(tbn_hip.TUNE_CONV_TILE, tile):
            y = empty(oshape, torch.float32)
            y.fill_(np.nan)
            # the pre-packed entry point runs only the patch kernel (no fallback)
            rc = tbn_hip.lib().tbn_hip_conv2d_f32_prepacked(tbn_hip.WEIGHTS_BINARY, P(dx), d, P(cw), P(ds), 1.0,
                                                            P(db), None, flags, P(y), None)
            if rc == tbn_hip.INVALID_SHAPE:
                continue  # this tile cannot hold the geometry
            assert rc == 0, tbn_hip.last_error()
            outs[tile] = host(y)
    assert len(outs) >= 2, sorted(outs)
    assert any(32 <= t < 64 or t >= 96 for t in outs) and any(t < 32 or 64 <= t < 96 for t in outs), sorted(outs)
    stacked = stride == (1, 1) and C % 32 == 0 and M % 64 == 0 and not flags & tbn_hip.EPI_MAXPOOL2X2
    assert any(64 <= t < 128 for t in outs) == stacked, sorted(outs)
    first = next(iter(outs.values()))
    for tile, y in outs.items():
        assert np.array_equal(y, first), f"tile {tile} differs"
    wsign = np.where(wbytes == 1, 1.0, -1.0).astype(np.float32)
    ref = conv_ref(x, wsign, scale, 1.0, bias, stride, pad, dil, flags)
    rm.assert_within_tolerance(first, ref, K, np.abs(x).max() * 1.5)


@pytest.mark.parametrize("case", [(32, 512, 7, 7, 512, False, True), (128, 256, 7, 7, 128, True, True),
                                  (128, 300, 7, 6, 96, False, False)], ids=["stage4", "ternary_res", "ragged"])
def test_conv_folded_groups_match_split_k(dev, case):
    """Deep layers sum their chunks in groups whose order the shape fixes.
    With enough images the groups run in one block (folded), with few they
    run split over blocks: every image gets the same bits at batch N as at
    batch 2, and the same bits as the forced split of the same batch."""
    import ctypes
    N, C, H, W, M, ternary, with_res = case
    rng = np.random.default_rng(C + M + H)
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    scale = rng.uniform(0.5, 1.5, M).astype(np.float32)
    bias = (rng.standard_normal(M) * 0.01).astype(np.float32)
    res = rng.standard_normal((N, M, H, W)).astype(np.float32) if with_res else None
    K = C * 9
    if ternary:
        kind = tbn_hip.WEIGHTS_TERNARY
        wt = rng.integers(-1, 2, (M, K)).astype(np.int8)
        K_pad, N_pad = (K + 31) // 32 * 32, M
        packed = empty(M * K_pad // 4, torch.uint8)
        tbn_hip.call("tbn_hip_pack_ternary", P(to_dev(wt)), K, M, tbn_hip.LAYOUT_NK, K_pad, M, P(packed), None)
        wref = wt.reshape(M, C, 3, 3).astype(np.float32)
    else:
        kind = tbn_hip.WEIGHTS_BINARY
        wbytes = (rng.random((M, C, 3, 3)) < 0.5).astype(np.uint8)
        packed, K_pad, N_pad = pack_conv_weights(wbytes, M, K)
        wref = np.where(wbytes == 1, 1.0, -1.0).astype(np.float32)

    def run(n):
        d = tbn_hip.conv_desc(n, C, H, W, M, 3, 3, 1, 1, 1, 1)
        wb = ctypes.c_int64()
        tbn_hip.call("tbn_hip_conv_weights_bytes", kind, d, ctypes.byref(wb))
        cw = empty(wb.value, torch.uint8)
        tbn_hip.call("tbn_hip_pack_conv_weights", kind, P(packed), K_pad, N_pad, d, P(cw), None)
        y = empty((n, M, H, W), torch.float32)
        y.fill_(np.nan)
        dr = to_dev(res[:n]) if with_res else None
        tbn_hip.call("tbn_hip_conv2d_f32_prepacked", kind, P(to_dev(x[:n])), d, P(cw), P(to_dev(scale)), 1.0,
                     P(to_dev(bias)), P(dr) if with_res else None, tbn_hip.EPI_RELU, P(y), None)
        name = ctypes.create_string_buffer(200)
        tbn_hip.call("tbn_hip_conv2d_kernel_name", kind, d, tbn_hip.EPI_RELU, int(with_res), name, 200)
        return host(y), name.value.decode()

    big, big_name = run(N)
    small, small_name = run(2)
    assert big_name.endswith(", true, false>"), big_name       # folded: one block runs every group
    assert small_name.endswith(", false, false>"), small_name  # split over blocks
    assert np.array_equal(big[:2], small)
    with tbn_hip.tuning(tbn_hip.TUNE_CONV_SPLITS, 2):
        forced, _ = run(N)
    if C // 32 * 9 // 2 >= 36 and M * H * W * 2 <= 1 << 16:  # the rule's own split is 2 here
        assert np.array_equal(big, forced)
        # every tile gives these bits, folded or split; two equal chunk groups
        # also run on tiles with two K groups of waves, one group each
        pair = re.compile(r"PatchCfg<\d+, \d+, \d+, \d+, \d+, 2>, (true|false), 9, \d, true, false>$")
        pairs = 0
        for tile in range(128):
            with tbn_hip.tuning(tbn_hip.TUNE_CONV_TILE, tile):
                try:
                    y_t, name_t = run(N)
                except tbn_hip.TbnError:
                    continue
            assert np.array_equal(y_t, big), (tile, name_t)
            pairs += bool(pair.search(name_t))
        assert pairs >= 1
    ref = conv_ref(x, wref, scale, 1.0, bias, (1, 1), (1, 1), (1, 1), 0)
    if with_res:
        ref = ref + res
    ref = np.maximum(ref, 0.0)
    rm.assert_within_tolerance(big, ref, K, np.abs(x).max() * 1.5)


def _prepacked_setup(case, seed):
    import ctypes
    N, C, H, W, M, kh, kw, stride, pad, dil, flags = case
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    wbytes = (rng.random((M, C, kh, kw)) < 0.5).astype(np.uint8)
    scale = rng.uniform(0.5, 1.5, M).astype(np.float32)
    bias = (rng.standard_normal(M) * 0.01).astype(np.float32)
    packed, K_pad, N_pad = pack_conv_weights(wbytes, M, C * kh * kw)
    d = tbn_hip.conv_desc(N, C, H, W, M, kh, kw, *stride, *pad, *dil)
    wb = ctypes.c_int64()
    tbn_hip.call("tbn_hip_conv_weights_bytes", tbn_hip.WEIGHTS_BINARY, d, ctypes.byref(wb))
    cw = empty(wb.value, torch.uint8)
    tbn_hip.call("tbn_hip_pack_conv_weights", tbn_hip.WEIGHTS_BINARY, P(packed), K_pad, N_pad, d, P(cw), None)
    OH, OW = tbn_hip.conv_out_hw(d)
    oshape = (N, M, OH // 2, OW // 2) if flags & tbn_hip.EPI_MAXPOOL2X2 else (N, M, OH, OW)
    ref = conv_ref(x, np.where(wbytes == 1, 1.0, -1.0).astype(np.float32), scale, 1.0, bias, stride, pad, dil, flags)
    return dict(x=to_dev(x), d=d, cw=cw, s=to_dev(scale), b=to_dev(bias), flags=flags, oshape=oshape, ref=ref,
                K=C * kh * kw, xmax=float(np.abs(x).max()))


def _run_prepacked(st, entry="tbn_hip_conv2d_f32_prepacked"):
    y = empty(st["oshape"], torch.float32)
    y.fill_(np.nan)
    tbn_hip.call(entry, tbn_hip.WEIGHTS_BINARY, P(st["x"]), st["d"], P(st["cw"]), P(st["s"]), 1.0, P(st["b"]),
                 None, st["flags"], P(y), None)
    return host(y)


@pytest.mark.parametrize("case", [CASES[0], (4, 64, 56, 56, 128, 3, 3, (1, 1), (1, 1), (1, 1), 0),
                                  (3, 256, 7, 7, 96, 3, 3, (1, 1), (1, 1), (1, 1), tbn_hip.EPI_RELU)],
                         ids=["cfg4", "56x56", "splitK"])
def test_conv_tune_keeps_the_bits(dev, case):
    """tbn_hip_conv2d_tune_prepacked times the tiles and caches one; calls
    before (static rule) and after (tuned tile) give the same bits."""
    st = _prepacked_setup(case, 21)
    before = _run_prepacked(st)
    _run_prepacked(st, "tbn_hip_conv2d_tune_prepacked")
    after = _run_prepacked(st)
    assert np.array_equal(before, after)
    rm.assert_within_tolerance(after, st["ref"], st["K"], st["xmax"] * 1.5)


def test_conv_forced_splits_skip_pooled_convs(dev):
    """A forced K-split count applies to unpooled convs only: a conv with the
    fused 2x2 pool keeps one split (same bits as unforced), an unpooled one
    splits and stays within tolerance."""
    pooled = _prepacked_setup((3, 96, 12, 10, 64, 3, 3, (1, 1), (1, 1), (1, 1),
                               tbn_hip.EPI_MAXPOOL2X2 | tbn_hip.EPI_RELU), 22)
    plain = _prepacked_setup((2, 128, 14, 14, 64, 3, 3, (1, 1), (1, 1), (1, 1), tbn_hip.EPI_RELU), 23)
    want_pooled = _run_prepacked(pooled)
    with tbn_hip.tuning(tbn_hip.TUNE_CONV_SPLITS, 2):
        got_pooled = _run_prepacked(pooled)
        got_plain = _run_prepacked(plain)
    assert np.array_equal(got_pooled, want_pooled)
    rm.assert_within_tolerance(got_pooled, pooled["ref"], pooled["K"], pooled["xmax"] * 1.5)
    rm.assert_within_tolerance(got_plain, plain["ref"], plain["K"], plain["xmax"] * 1.5)


PAIR_CASES = [
    # N, C, H, W, M, stride, ternary, flags, proj_flags, with_residual
    (4, 64, 56, 56, 128, 2, False, tbn_hip.EPI_RELU, 0, False),       # two chunks
    (4, 128, 28, 28, 256, 2, False, tbn_hip.EPI_RELU, 0, False),      # four chunks in turn
    (32, 256, 14, 14, 512, 2, False, tbn_hip.EPI_RELU, 0, False),     # chunk groups folded into one block
    (2, 72, 20, 18, 72, 2, True, tbn_hip.EPI_RELU, tbn_hip.EPI_BIAS_THEN_SCALE, True),  # ternary, ragged C / M
    (3, 96, 15, 13, 80, 1, False, tbn_hip.EPI_BIAS_THEN_SCALE, tbn_hip.EPI_RELU, True),  # stride 1
]


def _conv_layout(kind, rng, M, C, k):
    """Random binary / ternary weights [M, C, k, k] in the conv layout of a k x k desc, and their values."""
    import ctypes
    K = C * k * k
    if kind == tbn_hip.WEIGHTS_TERNARY:
        wt = rng.integers(-1, 2, (M, K)).astype(np.int8)
        K_pad, N_pad = (K + 31) // 32 * 32, M
        packed = empty(M * K_pad // 4, torch.uint8)
        tbn_hip.call("tbn_hip_pack_ternary", P(to_dev(wt)), K, M, tbn_hip.LAYOUT_NK, K_pad, M, P(packed), None)
        wref = wt.reshape(M, C, k, k).astype(np.float32)
    else:
        wbytes = (rng.random((M, C, k, k)) < 0.5).astype(np.uint8)
        packed, K_pad, N_pad = pack_conv_weights(wbytes, M, K)
        wref = np.where(wbytes == 1, 1.0, -1.0).astype(np.float32)

    def layout(d):
        wb = ctypes.c_int64()
        tbn_hip.call("tbn_hip_conv_weights_bytes", kind, d, ctypes.byref(wb))
        cw = empty(wb.value, torch.uint8)
        tbn_hip.call("tbn_hip_pack_conv_weights", kind, P(packed), K_pad, N_pad, d, P(cw), None)
        return cw
    return layout, wref


@pytest.mark.parametrize("case", PAIR_CASES, ids=["two_chunks", "chunks", "folded", "ternary", "stride1"])
def test_conv_pair_matches_separate_convs(dev, case):
    """A 3x3 pad-1 conv and the 1x1 projection of its input in one launch give
    the bits of the two separate calls, for the tuned tile and every tile that
    takes the pair; the pair's projection is also within tolerance of float64."""
    N, C, H, W, M, st, ternary, flags, pflags, with_res = case
    kind = tbn_hip.WEIGHTS_TERNARY if ternary else tbn_hip.WEIGHTS_BINARY
    rng = np.random.default_rng(N + C + M + st)
    x = to_dev(rng.standard_normal((N, C, H, W)).astype(np.float32))
    d3 = tbn_hip.conv_desc(N, C, H, W, M, 3, 3, st, st, 1, 1)
    d1 = tbn_hip.conv_desc(N, C, H, W, M, 1, 1, st, st, 0, 0)
    OH, OW = tbn_hip.conv_out_hw(d3)
    assert (OH, OW) == tbn_hip.conv_out_hw(d1)
    lay3, w3 = _conv_layout(kind, rng, M, C, 3)
    lay1, w1 = _conv_layout(kind, rng, M, C, 1)
    cw3, cw1 = lay3(d3), lay1(d1)
    s3 = to_dev(rng.uniform(0.5, 1.5, M).astype(np.float32))
    b3 = to_dev((rng.standard_normal(M) * 0.01).astype(np.float32))
    s1 = rng.uniform(0.5, 1.5, M).astype(np.float32)
    b1 = (rng.standard_normal(M) * 0.01).astype(np.float32)
    res = to_dev(rng.standard_normal((N, M, OH, OW)).astype(np.float32)) if with_res else None

    def separate():
        y, py = empty((N, M, OH, OW), torch.float32), empty((N, M, OH, OW), torch.float32)
        tbn_hip.call("tbn_hip_conv2d_f32_prepacked", kind, P(x), d3, P(cw3), P(s3), 1.0, P(b3), P(res), flags, P(y),
                     None)
        tbn_hip.call("tbn_hip_conv2d_f32_prepacked", kind, P(x), d1, P(cw1), P(to_dev(s1)), 0.5, P(to_dev(b1)), None,
                     pflags, P(py), None)
        return host(y), host(py)

    def pair(mode=0):
        y, py = empty((N, M, OH, OW), torch.float32), empty((N, M, OH, OW), torch.float32)
        y.fill_(np.nan)
        py.fill_(np.nan)
        tbn_hip.call("tbn_hip_conv2d_f32_prepacked_pair", kind, P(x), d3, P(cw3), P(s3), 1.0, P(b3), P(res), flags,
                     P(y), P(cw1), P(to_dev(s1)), 0.5, P(to_dev(b1)), pflags, P(py), mode, None)
        return host(y), host(py)

    tbn_hip.call("tbn_hip_conv2d_f32_prepacked_pair", kind, None, d3, None, None, 1.0, None, None, flags, None,
                 None, None, 0.5, None, pflags, None, 2, None)  # pairs: no pointer read
    want_y, want_p = separate()
    got_y, got_p = pair()
    assert np.array_equal(got_y, want_y) and np.array_equal(got_p, want_p)
    pair(mode=1)  # tuned
    got_y, got_p = pair()
    assert np.array_equal(got_y, want_y) and np.array_equal(got_p, want_p)
    ran = 0
    for tile in range(128):
        with tbn_hip.tuning(tbn_hip.TUNE_CONV_TILE, tile):
            try:
                got_y, got_p = pair()
            except tbn_hip.TbnError:
                continue
        assert np.array_equal(got_y, want_y) and np.array_equal(got_p, want_p), tile
        ran += 1
    assert ran >= 1
    ref = conv_ref(host(x), w1, s1, 0.5, b1, (st, st), (0, 0), (1, 1), pflags)
    rm.assert_within_tolerance(want_p, ref, C, float(np.abs(host(x)).max()) * 1.5)


def test_conv_pair_declines_split_and_other_shapes(dev):
    """Geometries that split K over blocks (few images of a deep layer) or
    have another kernel size or padding return TBN_NOT_IMPLEMENTED without
    work."""
    for d in (tbn_hip.conv_desc(2, 256, 14, 14, 512, 3, 3, 2, 2, 1, 1),   # K split at batch 2
              tbn_hip.conv_desc(2, 64, 16, 16, 64, 5, 5, 1, 1, 2, 2),     # 5x5
              tbn_hip.conv_desc(2, 64, 16, 16, 64, 3, 3, 1, 1, 0, 0)):    # pad 0
        with pytest.raises(tbn_hip.TbnError) as e:
            tbn_hip.call("tbn_hip_conv2d_f32_prepacked_pair", tbn_hip.WEIGHTS_BINARY, None, d, None, None, 1.0, None,
                         None, 0, None, None, None, 1.0, None, 0, None, 2, None)
        assert e.value.code == tbn_hip.NOT_IMPLEMENTED
