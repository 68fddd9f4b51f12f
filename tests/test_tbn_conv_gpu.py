"""TBN-mode convolution on the GPU (tbn_hip_conv2d_tbn_prepacked): the
reference Session's quantized conv arithmetic, bit-exact.

Reference: tbn-runtime/include/tbn/runtime/model.hpp:482-557 (im2col_
ternary_packed at +-0.1, the popcount product, + bias, * scale) and
conv2d_binary (conv2d.cpp:220-316: float(C) + bias).  The checker forms the
exact integer C from the oracle's im2col_ternary_packed (pinned on the
reference's golden vectors) and the float32 epilogue one rounding per
operation (tests/tbn_ref.py)."""
import ctypes

import numpy as np
import pytest
import torch

import tbn_hip
import tbn_ref
from gpu_util import P, empty, host, to_dev

pytestmark = pytest.mark.gpu

RELU, POOL, BTS = tbn_hip.EPI_RELU, tbn_hip.EPI_MAXPOOL2X2, tbn_hip.EPI_BIAS_THEN_SCALE

CASES = [
    # N, C, H, W, M, kh, kw, stride, pad, dil, flags, scale, residual
    (64, 64, 14, 14, 128, 3, 3, (1, 1), (1, 1), (1, 1), RELU, False, False),          # config 4
    (1, 1, 28, 28, 6, 5, 5, (1, 1), (0, 0), (1, 1), RELU | POOL, True, False),         # LeNet conv1
    (1, 6, 12, 12, 16, 5, 5, (1, 1), (0, 0), (1, 1), RELU | POOL | BTS, True, False),  # LeNet conv2
    (2, 64, 56, 56, 128, 3, 3, (2, 2), (1, 1), (1, 1), RELU, False, False),            # ResNet downsample
    (2, 64, 56, 56, 128, 1, 1, (2, 2), (0, 0), (1, 1), 0, True, False),                # 1x1 projection
    (2, 128, 28, 28, 128, 3, 3, (1, 1), (1, 1), (1, 1), RELU | BTS, True, True),       # residual block
    (3, 512, 7, 7, 96, 3, 3, (1, 1), (1, 1), (1, 1), RELU, True, True),                # 8 chunks
    (2, 300, 9, 8, 40, 3, 3, (2, 2), (1, 1), (1, 1), 0, False, False),                 # ragged last chunk
    (2, 5, 13, 11, 70, 3, 2, (2, 1), (1, 0), (2, 2), RELU, True, False),               # odd everything
    (3, 7, 9, 9, 70, 3, 3, (1, 1), (1, 1), (1, 1), RELU | POOL, False, False),         # odd output, floor pool
    (1, 32, 100, 100, 8, 3, 3, (1, 1), (1, 1), (1, 1), RELU, False, False),            # wide rows: column tiles
]


def threshold_input(rng, shape):
    """N(0, 0.2) with values on and next to the +-0.1 thresholds, NaN, +-inf,
    -0.0 and denormals mixed in."""
    x = (rng.standard_normal(shape) * 0.2).astype(np.float32)
    flat = x.reshape(-1)
    vals = np.array([0.1, -0.1, np.nextafter(np.float32(0.1), np.float32(1)),
                     np.nextafter(np.float32(-0.1), np.float32(-1)), np.nan, np.inf, -np.inf, -0.0, 0.0,
                     1e-38, -1e-45], np.float32)
    idx = rng.choice(flat.size, size=min(flat.size, 8 * vals.size), replace=False)
    flat[idx] = np.resize(vals, idx.size)
    return x


def pack_tbn_conv(binw, d):
    """binw [M, C, kh, kw] bytes (1 = +1) -> reference BinaryMatrix (NK) ->
    TBN conv layout, on the device."""
    M = binw.shape[0]
    K = binw[0].size
    K_pad, N_pad = tbn_hip.padded_dims(K, M)
    packed = empty(N_pad * K_pad // 8, torch.uint8)
    tbn_hip.call("tbn_hip_pack_binary", P(to_dev(binw.reshape(M, K))), K, M, tbn_hip.LAYOUT_NK, K_pad, N_pad,
                 P(packed), None)
    nbytes = ctypes.c_int64()
    tbn_hip.call("tbn_hip_tbn_conv_weights_bytes", ctypes.byref(d), ctypes.byref(nbytes))
    w4 = empty(nbytes.value, torch.uint8)
    tbn_hip.call("tbn_hip_pack_tbn_conv_weights", P(packed), K_pad, N_pad, ctypes.byref(d), P(w4), None)
    return w4


def run_tbn_conv(x, d, w4, scale, bias, residual, flags, out_shape):
    y = empty(out_shape, torch.float32)
    y.fill_(np.nan)
    nbytes = ctypes.c_int64()
    tbn_hip.call("tbn_hip_tbn_conv_scratch_bytes", ctypes.byref(d), ctypes.byref(nbytes))
    scratch = empty(max(nbytes.value, 16), torch.uint8)
    tbn_hip.call("tbn_hip_conv2d_tbn_prepacked", P(x), ctypes.byref(d), P(w4), P(scale), 1.0, P(bias), P(residual),
                 flags, tbn_ref.LO, tbn_ref.HI, P(scratch), P(y), None)
    out = host(y)
    # the same call on the library's stream workspace gives the same bits
    y.fill_(np.nan)
    tbn_hip.call("tbn_hip_conv2d_tbn_prepacked", P(x), ctypes.byref(d), P(w4), P(scale), 1.0, P(bias), P(residual),
                 flags, tbn_ref.LO, tbn_ref.HI, None, P(y), None)
    assert np.array_equal(host(y).view(np.uint32), out.view(np.uint32))
    return out


@pytest.mark.parametrize("variant", [1, 2], ids=["fused", "two_pass"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[:7])))
def test_tbn_conv_matches_oracle(dev, orc, case, variant):
    """Both kernel variants (the fused kernel staging ternarized patches in
    LDS, where a tile fits; the records pass then the barrier-free product)
    bit-exact against the oracle, with and without caller scratch."""
    with tbn_hip.tuning(tbn_hip.TUNE_TBN_CONV, variant):
        _check_case(orc, case)


def _check_case(orc, case):
    N, C, H, W, M, kh, kw, stride, pad, dil, flags, with_scale, with_res = case
    rng = np.random.default_rng(N * 131 + C * 7 + M + kh)
    x = threshold_input(rng, (N, C, H, W))
    binw = (rng.random((M, C, kh, kw)) < 0.5).astype(np.uint8)
    scale = rng.uniform(0.5, 1.5, M).astype(np.float32) if with_scale else None
    bias = (rng.standard_normal(M) * 3.0).astype(np.float32)
    d = tbn_hip.conv_desc(N, C, H, W, M, kh, kw, *stride, *pad, *dil)
    OH, OW = tbn_ref.conv_out_hw(H, W, kh, kw, stride, pad, dil)
    pool = bool(flags & POOL)
    out_shape = (N, M, OH // 2, OW // 2) if pool else (N, M, OH, OW)
    res = (rng.standard_normal((N, M, OH, OW)) * 4).astype(np.float32) if with_res else None

    Cint = tbn_ref.tbn_conv_int(orc, x, np.where(binw == 1, 1, -1), stride, pad, dil)
    ref = tbn_ref.tbn_conv_epilogue(Cint, scale, 1.0, bias, res, bool(flags & BTS), bool(flags & RELU), pool)

    w4 = pack_tbn_conv(binw, d)
    dx = to_dev(x)
    ds = None if scale is None else to_dev(scale)
    db, dr = to_dev(bias), None if res is None else to_dev(res)
    y1 = run_tbn_conv(dx, d, w4, ds, db, dr, flags, out_shape)
    y2 = run_tbn_conv(dx, d, w4, ds, db, dr, flags, out_shape)
    bad = np.argwhere(y1.view(np.uint32) != ref.view(np.uint32))
    if bad.size:
        name = ctypes.create_string_buffer(160)
        tbn_hip.call("tbn_hip_conv2d_tbn_kernel_name", ctypes.byref(d), flags, name, 160)
        where = [(tuple(int(v) for v in i), float(y1[tuple(i)]), float(ref[tuple(i)])) for i in bad[:12]]
        pytest.fail(f"{len(bad)} of {ref.size} differ ({name.value.decode()}): {where}")
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


def test_tbn_conv_no_bias_no_scale_is_float_of_integer(dev, orc):
    """Without scale and bias the output is float(C) itself: the integer
    product of conv2d_binary's qlinear_matmul_binary (scale 1)."""
    rng = np.random.default_rng(3)
    N, C, H, W, M = 4, 96, 10, 10, 64
    x = threshold_input(rng, (N, C, H, W))
    binw = (rng.random((M, C, 3, 3)) < 0.5).astype(np.uint8)
    d = tbn_hip.conv_desc(N, C, H, W, M, 3, 3, ph=1, pw=1)
    y = run_tbn_conv(to_dev(x), d, pack_tbn_conv(binw, d), None, None, None, 0, (N, M, H, W))
    Cint = tbn_ref.tbn_conv_int(orc, x, np.where(binw == 1, 1, -1), (1, 1), (1, 1), (1, 1))
    assert np.array_equal(y, Cint.astype(np.float32))
    assert np.abs(Cint).max() <= C * 9


def test_tbn_conv_error_codes(dev):
    d = tbn_hip.conv_desc(1, 8, 8, 8, 8, 3, 3, ph=1, pw=1)
    buf = empty(1 << 16, torch.uint8)
    y = empty((1, 8, 8, 8), torch.float32)
    x = empty((1, 8, 8, 8), torch.float32)
    cases = [
        (POOL, tbn_hip.NOT_IMPLEMENTED),               # the fused pool needs the fused ReLU
        (tbn_hip.EPI_MAXPOOL3X3S2, tbn_hip.INVALID_ARGUMENT),
    ]
    for flags, code in cases:
        with pytest.raises(tbn_hip.TbnError) as e:
            tbn_hip.call("tbn_hip_conv2d_tbn_prepacked", P(x), ctypes.byref(d), P(buf), None, 1.0, None, None, flags,
                         -0.1, 0.1, P(buf), P(y), None)
        assert e.value.code == code
    with pytest.raises(tbn_hip.TbnError) as e:  # residual with the fused pool
        tbn_hip.call("tbn_hip_conv2d_tbn_prepacked", P(x), ctypes.byref(d), P(buf), None, 1.0, None, P(y),
                     RELU | POOL, -0.1, 0.1, P(buf), P(y), None)
    assert e.value.code == tbn_hip.INVALID_ARGUMENT


TBN_PAIR_CASES = [
    # N, C, H, W, M, stride, flags, proj_flags, residual
    (4, 64, 56, 56, 128, 2, RELU, 0, False),        # ResNet stage 2's downsampling block
    (2, 128, 28, 28, 256, 2, RELU | BTS, BTS, True),  # two chunks, bias-then-scale, residual on the conv
    (3, 300, 9, 8, 40, 2, 0, RELU, False),          # ragged last chunk and M
    (2, 96, 15, 13, 80, 1, RELU, RELU, True),       # stride 1
]


@pytest.mark.parametrize("case", TBN_PAIR_CASES, ids=["stage2", "bts_res", "ragged", "stride1"])
def test_tbn_conv_pair_matches_separate_convs(dev, case):
    """A 3x3 pad-1 TBN conv and the 1x1 TBN projection of its input in one
    launch (tbn_hip_conv2d_tbn_prepacked_pair) give the bits of the two
    separate calls: every product and sum is an exact integer."""
    N, C, H, W, M, st, flags, pflags, with_res = case
    rng = np.random.default_rng(N + C + M + st)
    x = to_dev(threshold_input(rng, (N, C, H, W)))
    d3 = tbn_hip.conv_desc(N, C, H, W, M, 3, 3, st, st, 1, 1)
    d1 = tbn_hip.conv_desc(N, C, H, W, M, 1, 1, st, st, 0, 0)
    OH, OW = tbn_hip.conv_out_hw(d3)
    assert (OH, OW) == tbn_hip.conv_out_hw(d1)
    w3 = pack_tbn_conv((rng.random((M, C, 3, 3)) < 0.5).astype(np.uint8), d3)
    w1 = pack_tbn_conv((rng.random((M, C, 1, 1)) < 0.5).astype(np.uint8), d1)
    s3 = to_dev(rng.uniform(0.5, 1.5, M).astype(np.float32))
    b3 = to_dev(rng.standard_normal(M).astype(np.float32))
    s1 = to_dev(rng.uniform(0.5, 1.5, M).astype(np.float32))
    b1 = to_dev(rng.standard_normal(M).astype(np.float32))
    res = to_dev(rng.standard_normal((N, M, OH, OW)).astype(np.float32)) if with_res else None
    want_y = run_tbn_conv(x, d3, w3, s3, b3, res, flags, (N, M, OH, OW))
    want_p = run_tbn_conv(x, d1, w1, s1, b1, None, pflags, (N, M, OH, OW))
    tbn_hip.call("tbn_hip_conv2d_tbn_prepacked_pair", None, ctypes.byref(d3), None, None, 1.0, None, None, flags,
                 tbn_ref.LO, tbn_ref.HI, None, None, None, 1.0, None, pflags, None, 2, None)  # pairs: no pointer read
    y, py = empty((N, M, OH, OW), torch.float32), empty((N, M, OH, OW), torch.float32)
    y.fill_(np.nan)
    py.fill_(np.nan)
    tbn_hip.call("tbn_hip_conv2d_tbn_prepacked_pair", P(x), ctypes.byref(d3), P(w3), P(s3), 1.0, P(b3), P(res),
                 flags, tbn_ref.LO, tbn_ref.HI, P(y), P(w1), P(s1), 1.0, P(b1), pflags, P(py), 0, None)
    assert np.array_equal(host(y).view(np.uint32), want_y.view(np.uint32))
    assert np.array_equal(host(py).view(np.uint32), want_p.view(np.uint32))


def test_tbn_conv_pair_declines(dev):
    """Another kernel size or padding, and a geometry forced onto the two-pass
    kernels, return TBN_NOT_IMPLEMENTED without work; a pooled epilogue is an
    invalid request."""
    d = tbn_hip.conv_desc(2, 64, 16, 16, 64, 3, 3, 2, 2, 1, 1)
    for dd in (tbn_hip.conv_desc(2, 64, 16, 16, 64, 5, 5, 1, 1, 2, 2), tbn_hip.conv_desc(2, 64, 16, 16, 64, 3, 3, 1, 1, 0, 0)):
        with pytest.raises(tbn_hip.TbnError) as e:
            tbn_hip.call("tbn_hip_conv2d_tbn_prepacked_pair", None, ctypes.byref(dd), None, None, 1.0, None, None, 0,
                         tbn_ref.LO, tbn_ref.HI, None, None, None, 1.0, None, 0, None, 2, None)
        assert e.value.code == tbn_hip.NOT_IMPLEMENTED
    with tbn_hip.tuning(tbn_hip.TUNE_TBN_CONV, 2):
        with pytest.raises(tbn_hip.TbnError) as e:
            tbn_hip.call("tbn_hip_conv2d_tbn_prepacked_pair", None, ctypes.byref(d), None, None, 1.0, None, None, 0,
                         tbn_ref.LO, tbn_ref.HI, None, None, None, 1.0, None, 0, None, 2, None)
        assert e.value.code == tbn_hip.NOT_IMPLEMENTED
    with pytest.raises(tbn_hip.TbnError) as e:
        tbn_hip.call("tbn_hip_conv2d_tbn_prepacked_pair", None, ctypes.byref(d), None, None, 1.0, None, None,
                     RELU | POOL, tbn_ref.LO, tbn_ref.HI, None, None, None, 1.0, None, 0, None, 2, None)
    assert e.value.code == tbn_hip.INVALID_ARGUMENT
