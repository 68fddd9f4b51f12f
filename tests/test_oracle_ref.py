"""The oracle's fp32 operator restatements against the reference's own fp32
operators, compiled from the reference sources into oracle/_ref (see
oracle/Makefile `ref`).  Bit-exact: both sides run the same loop order with
separately rounded fp32 multiplies and adds.  Skipped where oracle/_ref was
not built (it needs the reference tree, which only the build host has)."""
import ctypes
import os
import pathlib

import numpy as np
import pytest

REF_LIB = pathlib.Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "libtbn_ref.so"

pytestmark = pytest.mark.skipif(not REF_LIB.exists(), reason="oracle/_ref not built (no reference tree here)")

I64 = ctypes.c_int64


@pytest.fixture(scope="module")
def ref():
    # the GeMM symbols of the quantized variants are unresolved: bind lazily
    return ctypes.CDLL(str(REF_LIB), mode=os.RTLD_LAZY)


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def ref_conv2d(ref, x, w, b, stride, pad, dil):
    N, C, H, W = x.shape
    M, _, kh, kw = w.shape
    OH = (H + 2 * pad[0] - dil[0] * (kh - 1) - 1) // stride[0] + 1
    OW = (W + 2 * pad[1] - dil[1] * (kw - 1) - 1) // stride[1] + 1
    y = np.empty((N, M, OH, OW), np.float32)
    rc = ref.ref_conv2d(_p(x), I64(N), I64(C), I64(H), I64(W), _p(w), I64(M), I64(kh), I64(kw), _p(b),
                        I64(stride[0]), I64(stride[1]), I64(pad[0]), I64(pad[1]), I64(dil[0]), I64(dil[1]), _p(y))
    assert rc == 0
    return y


@pytest.mark.parametrize("shape", [
    # (N, C, H, W, M, k, stride, pad, dil)
    (1, 1, 28, 28, 6, 5, 1, 0, 1),       # LeNet conv1
    (2, 6, 12, 12, 16, 5, 1, 0, 1),      # LeNet conv2
    (2, 3, 23, 23, 8, 7, 2, 3, 1),       # ResNet stem geometry
    (1, 8, 9, 11, 5, 3, 2, 1, 2),        # stride 2, dilation 2, ragged
    (3, 4, 6, 6, 7, 1, 1, 0, 1),         # 1x1
])
@pytest.mark.parametrize("with_bias", [True, False])
def test_conv2d_f32_matches_reference_bitwise(orc, ref, shape, with_bias):
    N, C, H, W, M, k, s, p, d = shape
    rng = np.random.default_rng(N * 1000 + C * 10 + M)
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    w = rng.standard_normal((M, C, k, k)).astype(np.float32)
    b = rng.standard_normal(M).astype(np.float32) if with_bias else None
    want = ref_conv2d(ref, x, w, b, (s, s), (p, p), (d, d))
    got = orc.conv2d_f32(x, w, b, (s, s), (p, p), (d, d))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("M,K,N,ta,tb,cmode", [
    (7, 130, 9, False, False, None), (64, 64, 64, False, False, "1d"), (33, 200, 65, True, False, "2d"),
    (5, 70, 130, False, True, "1d"), (1, 256, 10, False, False, "1d"), (70, 129, 3, True, True, None)])
def test_gemm_f32_blocked_matches_reference_bitwise(orc, ref, M, K, N, ta, tb, cmode):
    rng = np.random.default_rng(M * 7 + K + N)
    A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    C = None if cmode is None else rng.standard_normal(N if cmode == "1d" else (M, N)).astype(np.float32)
    alpha, beta = np.float32(0.75), np.float32(1.25)
    want = np.empty((M, N), np.float32)
    rc = ref.ref_gemm(_p(A), _p(B), _p(C), ctypes.c_int(int(cmode == "1d")), I64(M), I64(K), I64(N),
                      ctypes.c_float(alpha), ctypes.c_float(beta), ctypes.c_int(int(ta)), ctypes.c_int(int(tb)),
                      _p(want))
    assert rc == 0
    got = orc.gemm_f32_blocked(A, B, C, alpha, beta, ta, tb)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("k,s,p,ceil", [((2, 2), (2, 2), (0, 0), False), ((3, 3), (2, 2), (1, 1), False),
                                        ((3, 3), (2, 2), (0, 0), True), ((2, 3), (1, 2), (1, 0), False)])
def test_maxpool2d_matches_reference_bitwise(orc, ref, k, s, p, ceil):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 3, 13, 11)).astype(np.float32)
    hw = np.zeros(2, np.int64)
    assert ref.ref_maxpool2d(_p(x), I64(2), I64(3), I64(13), I64(11), I64(k[0]), I64(k[1]), I64(s[0]), I64(s[1]),
                             I64(p[0]), I64(p[1]), ctypes.c_int(int(ceil)), None, _p(hw)) == 0
    want = np.empty((2, 3, int(hw[0]), int(hw[1])), np.float32)
    assert ref.ref_maxpool2d(_p(x), I64(2), I64(3), I64(13), I64(11), I64(k[0]), I64(k[1]), I64(s[0]), I64(s[1]),
                             I64(p[0]), I64(p[1]), ctypes.c_int(int(ceil)), _p(want), _p(hw)) == 0
    got = orc.maxpool2d(x, k, s, p, ceil_mode=ceil)
    assert np.array_equal(got, want)


def test_global_avgpool_matches_reference_bitwise(orc, ref):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, 5, 7, 7)).astype(np.float32)
    want = np.empty((3, 5), np.float32)
    assert ref.ref_global_avgpool2d(_p(x), I64(3), I64(5), I64(7), I64(7), _p(want)) == 0
    got = orc.global_avgpool2d(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("k,s,p,ceil,inc", [((2, 2), (2, 2), (0, 0), False, False), ((3, 3), (2, 2), (1, 1), False, True),
                                            ((3, 3), (2, 2), (1, 1), True, False), ((3, 3), (2, 2), (0, 0), True, True),
                                            ((2, 3), (1, 2), (1, 0), False, True)])
def test_avgpool2d_matches_reference_bitwise(orc, ref, k, s, p, ceil, inc):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 3, 13, 11)).astype(np.float32)
    x[0, 1, 3, 4] = np.nan
    hw = np.zeros(2, np.int64)
    args = [I64(2), I64(3), I64(13), I64(11), I64(k[0]), I64(k[1]), I64(s[0]), I64(s[1]), I64(p[0]), I64(p[1]),
            ctypes.c_int(int(ceil)), ctypes.c_int(int(inc))]
    assert ref.ref_avgpool2d(_p(x), *args, None, _p(hw)) == 0
    want = np.empty((2, 3, int(hw[0]), int(hw[1])), np.float32)
    assert ref.ref_avgpool2d(_p(x), *args, _p(want), _p(hw)) == 0
    got = orc.avgpool2d(x, k, s, p, ceil_mode=ceil, count_include_pad=inc)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_global_maxpool_matches_reference_bitwise(orc, ref):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((3, 5, 7, 7)).astype(np.float32)
    x[0, 0, 2, 2] = np.nan
    x[1, 1] = 0.0
    x[1, 1, 0, 0] = -0.0
    x[2, 3] = np.nan
    want = np.empty((3, 5), np.float32)
    assert ref.ref_global_maxpool2d(_p(x), I64(3), I64(5), I64(7), I64(7), _p(want)) == 0
    got = orc.global_maxpool2d(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
