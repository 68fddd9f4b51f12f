"""Pins the CPU oracle (oracle/tbn_oracle.c) before it is trusted as the checker.

Each oracle function is checked against at least one of: the reference's own
golden vectors (tests/golden/gemm_golden.npz, from GeMM/05-final/
matrices_to_test.hpp and GeMM/03-blocked/matrices_64x64.hpp), known answers
from the reference's tests, or an independent numpy formulation
(tests/refmath.py) / float64 brute force.  CPU only.
"""
import pathlib

import numpy as np
import pytest

import refmath as rm

GOLDEN = pathlib.Path(__file__).with_name("golden") / "gemm_golden.npz"

# Tilings exercised by GeMM/05-final/test_final.cpp:23-70.
FINAL_TILINGS = [(128, 128, 128, 64, 64), (64, 64, 128, 32, 32), (32, 32, 128, 16, 16), (64, 64, 128, 32, 32)]


@pytest.fixture(scope="module")
def golden():
    return dict(np.load(GOLDEN))


# ---------------------------------------------------------------- TBN popcount GEMM

@pytest.mark.parametrize("tiling", FINAL_TILINGS)
def test_tbn_gemm_golden_128(orc, golden, tiling):
    A, B, C = golden["A128"], golden["B128"], golden["C128"]
    rc, pos, neg = orc.ternary_matrix_pack_from_float(A.astype(np.float32), 128, 128)
    assert rc == 0
    rc, bits = orc.binary_matrix_pack(B, 128, 128)
    assert rc == 0
    rc, out = orc.tbn_gemm(pos, neg, bits, 128, 128, 128, tiling)
    assert rc == 0
    assert np.array_equal(np.sign(out), C)  # the reference's own expectation (sign of C)
    assert np.array_equal(out, A.astype(np.int64) @ B.astype(np.int64))  # full int32 by brute force


def test_tbn_gemm_golden_64_padded(orc, golden):
    # 05-final needs n % 128 == 0, so the 64^3 set runs padded as the runtime pads it.
    A = np.zeros((64, 128), np.float32); A[:, :64] = golden["A64"]
    B = np.ones((128, 64), np.int8); B[:64] = golden["B64"]
    rc, pos, neg = orc.ternary_matrix_pack_from_float(A, 64, 128)
    rc2, bits = orc.binary_matrix_pack(B, 128, 64)
    assert rc == 0 and rc2 == 0
    rc, out = orc.tbn_gemm(pos, neg, bits, 64, 128, 64, (64, 64, 128, 32, 32))
    assert rc == 0
    assert np.array_equal(np.sign(out), golden["C64"])


def test_tbn_gemm_rejects_bad_tiling(orc, golden):
    # GeMM/05-final/test_final.cpp:105-118: kblk = 64 must throw.
    rc, pos, neg = orc.ternary_matrix_pack_from_float(golden["A128"].astype(np.float32), 128, 128)
    _, bits = orc.binary_matrix_pack(golden["B128"], 128, 128)
    rc, _ = orc.tbn_gemm(pos, neg, bits, 128, 128, 128, (64, 64, 64, 32, 32))
    assert rc == -1


def test_pack_rejects_bad_values_and_dims(orc):
    bad = np.ones(64 * 8, np.int8); bad[0] = 0  # test_final.cpp:86-94
    assert orc.binary_matrix_pack(bad, 64, 8)[0] == -1
    assert orc.binary_matrix_pack(np.ones(100, np.int8), 10, 10)[0] == -1
    rc, _, _ = orc.ternary_matrix_pack_from_float(np.zeros((10, 10), np.float32), 10, 10)
    assert rc == -1  # test_final.cpp:96-103


def test_qlinear_matmul_binary_tbn_known_answer(orc):
    # The reference's own operator on test_quantized_operators.cpp:165-179 inputs
    # ternarizes the activations: 1.4, -1.4, 1.4, -1.4 (survey probe of the
    # compiled reference); with the default tiling M=2 pads to 16 and throws.
    A = np.array([[1.0, -2.0], [3.0, -4.0]], np.float32)
    Bb = np.array([[1, 0], [0, 1]], np.uint8)
    rc, _ = orc.qlinear_matmul_binary_tbn(A, Bb, 0.7)
    assert rc == -1
    rc, out = orc.qlinear_matmul_binary_tbn(A, Bb, 0.7, (16, 16, 128, 16, 8))
    assert rc == 0
    np.testing.assert_allclose(out.reshape(-1), [1.4, -1.4, 1.4, -1.4], rtol=1e-6)


def test_qlinear_matmul_binary_tbn_random(orc):
    rng = np.random.default_rng(3)
    M, K, N = 96, 200, 40
    A = rng.standard_normal((M, K)).astype(np.float32) * 0.2
    Bb = (rng.random((K, N)) < 0.5).astype(np.uint8)
    rc, out = orc.qlinear_matmul_binary_tbn(A, Bb, 0.25, (128, 256, 256, 16, 8))
    assert rc == 0
    t = np.where(A < -0.1, -1, np.where(A > 0.1, 1, 0)).astype(np.int64)
    w = np.where(Bb == 1, 1, -1).astype(np.int64)
    np.testing.assert_array_equal(out, (t @ w).astype(np.float32) * np.float32(0.25))


def test_im2col_ternary_packed_matches_numpy(orc):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 3, 9, 7)).astype(np.float32) * 0.3
    for stride, pad, dil in [((1, 1), (0, 0), (1, 1)), ((2, 1), (1, 2), (1, 1)), ((1, 1), (1, 1), (2, 2))]:
        cols, OH, OW = rm.np_im2col(x, 3, 3, stride, pad, dil)
        m_pad, k_pad = (cols.shape[0] + 15) // 16 * 16, 128
        rc, pos, neg = orc.im2col_ternary_packed(x, 3, 3, stride, pad, dil, m_pad, k_pad)
        assert rc == 0
        full = np.zeros((m_pad, k_pad)); full[:cols.shape[0], :cols.shape[1]] = cols
        ep = np.packbits(full > 0.1, axis=1, bitorder="little").reshape(-1)
        en = np.packbits(full < -0.1, axis=1, bitorder="little").reshape(-1)
        assert np.array_equal(pos, ep) and np.array_equal(neg, en)


# ---------------------------------------------------------------- packing

@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("K,N", [(1, 1), (25, 6), (150, 16), (300, 13), (576, 128)])
def test_pack_binary_closed_form(orc, layout, K, N):
    rng = np.random.default_rng(K * 7 + N)
    binw = rng.integers(0, 3, size=K * N).astype(np.uint8)  # byte 2 is also -1
    K_pad, N_pad = (K + 127) // 128 * 128, (N + 7) // 8 * 8
    got = orc.pack_binary(binw, K, N, layout, K_pad, N_pad)
    assert np.array_equal(got, rm.np_pack_binary(binw, K, N, layout, K_pad, N_pad))


def test_binary_matrix_pack_closed_form(orc):
    rng = np.random.default_rng(5)
    data = np.where(rng.random((128, 24)) < 0.5, -1, 1).astype(np.int8)
    rc, bits = orc.binary_matrix_pack(data, 128, 24)
    assert rc == 0
    expect = np.packbits((data == -1).T, axis=1, bitorder="little").reshape(-1)
    assert np.array_equal(bits, expect)


def test_ternary_pack2_known_answer(orc):
    # [-1, 0, 1, 1, -1] -> a4 00 (survey probe of TernaryPackedWeights::set_weight)
    got = orc.ternary_pack2(np.array([-1, 0, 1, 1, -1], np.int8))
    assert got.tolist() == [0xA4, 0x00]


def test_ternary_pack2_roundtrip_and_reserved_code(orc):
    rng = np.random.default_rng(6)
    t = rng.integers(-1, 2, size=1001).astype(np.int8)
    packed = orc.ternary_pack2(t)
    assert np.array_equal(packed, rm.np_ternary_pack2(t))
    assert np.array_equal(orc.ternary_get2(packed, t.size), t)
    # code 11 is reserved and decodes to 0; out-of-range values encode as 0
    assert orc.ternary_get2(np.array([0b11100100], np.uint8), 4).tolist() == [-1, 0, 1, 0]
    assert orc.ternary_pack2(np.array([5, -7, 1, -1], np.int8)).tolist() == [0b00100101]


@pytest.mark.parametrize("layout", [0, 1])
def test_pack_ternary_gemm_layout(orc, layout):
    rng = np.random.default_rng(7 + layout)
    K, N = 70, 11
    t = rng.integers(-1, 2, size=K * N).astype(np.int8)
    K_pad, N_pad = 96, 16
    got = orc.pack_ternary(t, K, N, layout, K_pad, N_pad)
    assert np.array_equal(got, rm.np_pack_ternary(t, K, N, layout, K_pad, N_pad))


# ---------------------------------------------------------------- sign rules

SPECIAL = np.array([0.0, -0.0, np.nan, np.inf, -np.inf, 1e-45, -1e-45, 0.1, -0.1, 3.0, -2.0], np.float32)


def test_sign_rules_special_values(orc):
    # quantize_to_binary: w > thr (quantized_gemm_neon.cpp:553)
    assert orc.quantize_to_binary_f32(SPECIAL).tolist() == [0, 0, 0, 1, 0, 1, 0, 1, 0, 1, 0]
    assert orc.quantize_to_binary_f32(SPECIAL, 0.1).tolist() == [0, 0, 0, 1, 0, 0, 0, 0, 0, 1, 0]
    # Session extraction: w >= 0 (model.hpp:433)
    assert orc.sign_ge0_f32(SPECIAL).tolist() == [1, 1, 0, 1, 0, 1, 0, 1, 0, 1, 0]
    # quantize_to_ternary: < lo -> -1, > hi -> +1 (quantized_gemm_neon.cpp:584-590)
    assert orc.quantize_to_ternary_f32(SPECIAL).tolist() == [0, 0, 0, 1, -1, 0, 0, 0, 0, 1, -1]
    assert orc.quantize_to_binary_i8(np.array([-128, -1, 0, 1, 127], np.int8)).tolist() == [0, 0, 0, 1, 1]


def test_channel_mean_abs_sequential(orc):
    rng = np.random.default_rng(8)
    w = rng.standard_normal((16, 6, 5, 5)).astype(np.float32) * 0.1
    got = orc.channel_mean_abs(w)
    for c in range(16):
        assert got[c] == np.float32(rm.seq_sum_f32(np.abs(w[c])) / np.float32(150))


def test_already_binary_heuristic(orc):
    rng = np.random.default_rng(9)
    s = np.array([0.5, 2.0], np.float32)
    w = np.where(rng.random((2, 100)) < 0.5, -1.0, 1.0).astype(np.float32) * s[:, None]
    assert orc.already_binary(w, orc.channel_mean_abs(w))
    w2 = rng.standard_normal((2, 100)).astype(np.float32)
    assert not orc.already_binary(w2, orc.channel_mean_abs(w2))


# ---------------------------------------------------------------- mode F32 GEMM

def test_float_binary_known_answer(orc):
    # test_quantized_operators.cpp:165-179 inputs; true float x binary gives
    # 2.1, -2.1, 4.9, -4.9 (the file's own 0.7, -1.4, ... treats byte 0 as 0).
    A = np.array([[1.0, -2.0], [3.0, -4.0]], np.float32)
    Bb = np.array([[1, 0], [0, 1]], np.uint8)
    out = orc.qlinear_matmul_binary_naive(A, Bb, 0.7)
    np.testing.assert_allclose(out.reshape(-1), [2.1, -2.1, 4.9, -4.9], rtol=1e-6)
    packed = orc.pack_binary(Bb, 2, 2, 0, 128, 8)
    np.testing.assert_allclose(orc.gemm_f32_binary(A, packed, 128, 2, alpha=0.7).reshape(-1),
                               [2.1, -2.1, 4.9, -4.9], rtol=1e-6)


def test_float_ternary_known_answer(orc):
    # test_quantized_operators.cpp:124-155: [1,2;3,4] x [1,-1;0,1] x 0.5
    A = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    t = np.array([[1, -1], [0, 1]], np.int8)
    packed = orc.pack_ternary(t, 2, 2, 0, 32, 2)
    out = orc.gemm_f32_ternary(A, packed, 32, 2, alpha=0.5)
    np.testing.assert_allclose(out.reshape(-1), [0.5, 0.5, 1.5, 0.5], rtol=1e-7)


@pytest.mark.parametrize("M,K,N", [(1, 25, 6), (7, 300, 13), (33, 1000, 40)])
def test_gemm_binary_vs_float64(orc, M, K, N):
    rng = np.random.default_rng(M + K + N)
    A = rng.standard_normal((M, K)).astype(np.float32)
    binw = (rng.random((K, N)) < 0.5).astype(np.uint8)
    scale = rng.uniform(0.5, 1.5, N).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32) * 0.01
    K_pad, N_pad = (K + 127) // 128 * 128, (N + 7) // 8 * 8
    packed = orc.pack_binary(binw, K, N, 0, K_pad, N_pad)
    W = rm.np_unpack_binary(packed, K, N, K_pad)
    assert np.array_equal(W, np.where(binw.reshape(K, N) == 1, 1, -1))
    ref = rm.f64_gemm(A, W, scale, 0.9, bias, relu=True)
    o64 = orc.gemm_f64_binary(A, packed, K_pad, N, scale, 0.9, bias, True)
    np.testing.assert_allclose(o64, ref, rtol=1e-12, atol=1e-12)
    o32 = orc.gemm_f32_binary(A, packed, K_pad, N, scale, 0.9, bias, True)
    rm.assert_within_tolerance(o32, ref, K, np.abs(A).max() * 1.5)
    # sequential fp32 is the reference's qlinear_matmul_binary_naive loop
    naive = orc.qlinear_matmul_binary_naive(A, binw.reshape(K, N), 1.0)
    assert np.array_equal(orc.gemm_f32_binary(A, packed, K_pad, N), naive)


def test_gemm_ternary_vs_float64(orc):
    rng = np.random.default_rng(11)
    M, K, N = 9, 260, 17
    A = rng.standard_normal((M, K)).astype(np.float32)
    t = rng.choice([-1, 0, 1], size=(K, N), p=[0.3, 0.4, 0.3]).astype(np.int8)
    scale = rng.uniform(0.5, 1.5, N).astype(np.float32)
    packed = orc.pack_ternary(t, K, N, 0, 288, N)
    assert np.array_equal(rm.np_unpack_ternary(packed, K, N, 288), t)
    ref = rm.f64_gemm(A, t, scale)
    np.testing.assert_allclose(orc.gemm_f64_ternary(A, packed, 288, N, scale), ref, rtol=1e-12, atol=1e-12)
    rm.assert_within_tolerance(orc.gemm_f32_ternary(A, packed, 288, N, scale), ref, K, np.abs(A).max() * 1.5)


# ---------------------------------------------------------------- fp32 operators

@pytest.mark.parametrize("stride,pad,dil", [((1, 1), (0, 0), (1, 1)), ((1, 1), (1, 1), (1, 1)),
                                            ((2, 2), (3, 3), (1, 1)), ((2, 1), (0, 2), (2, 1))])
def test_conv2d_vs_numpy(orc, stride, pad, dil):
    rng = np.random.default_rng(12)
    x = rng.standard_normal((2, 3, 11, 10)).astype(np.float32)
    w = rng.standard_normal((5, 3, 3, 4)).astype(np.float32)
    b = rng.standard_normal(5).astype(np.float32)
    ref = rm.f64_conv(x, w, b, stride, pad, dil)
    np.testing.assert_allclose(orc.conv2d_f64(x, w, b, stride, pad, dil), ref, rtol=1e-12, atol=1e-12)
    rm.assert_within_tolerance(orc.conv2d_f32(x, w, b, stride, pad, dil), ref, 36, np.abs(x).max() * np.abs(w).max())


def test_maxpool_known_answer(orc):
    # tbn-runtime/tests/test_pooling.cpp:7-17,83-88: input i % 10 over [1,2,4,4]
    x = (np.arange(32) % 10).astype(np.float32).reshape(1, 2, 4, 4)
    y = orc.maxpool2d(x, (2, 2), (2, 2))
    assert y.shape == (1, 2, 2, 2)
    assert y.reshape(-1)[:2].tolist() == [5.0, 7.0]


@pytest.mark.parametrize("k,s,p,ceil_mode", [((2, 2), (2, 2), (0, 0), False), ((3, 3), (2, 2), (1, 1), False),
                                             ((3, 3), (2, 2), (0, 0), True), ((2, 3), (1, 2), (1, 1), False)])
def test_maxpool_vs_numpy(orc, k, s, p, ceil_mode):
    rng = np.random.default_rng(13)
    x = rng.standard_normal((2, 3, 9, 8)).astype(np.float32)
    assert np.array_equal(orc.maxpool2d(x, k, s, p, ceil_mode=ceil_mode), rm.np_maxpool(x, k, s, p, ceil_mode))


def test_global_avgpool(orc):
    rng = np.random.default_rng(14)
    x = rng.standard_normal((2, 3, 7, 7)).astype(np.float32)
    y = orc.global_avgpool2d(x)
    for n in range(2):
        for c in range(3):
            assert y[n, c] == np.float32(rm.seq_sum_f32(x[n, c]) / np.float32(49))
    # known answer from the pooling test input
    x2 = (np.arange(32) % 10).astype(np.float32).reshape(1, 2, 4, 4)
    np.testing.assert_allclose(orc.global_avgpool2d(x2).reshape(-1), [x2[0, 0].mean(), x2[0, 1].mean()], rtol=1e-7)


def test_avgpool_known_answer(orc):
    # the reference's pooling test input (tbn-runtime/tests/test_pooling.cpp:
    # 7-17,46-60), i % 10 over [1,2,4,4], 2x2/2: window means by hand
    x = (np.arange(32) % 10).astype(np.float32).reshape(1, 2, 4, 4)
    y = orc.avgpool2d(x, (2, 2), (2, 2))
    assert y.shape == (1, 2, 2, 2)
    assert y[0, 0].reshape(-1).tolist() == [2.5, 4.5, 5.5, 2.5]
    assert orc.global_maxpool2d(x).reshape(-1).tolist() == [9.0, 9.0]


def _np_avgpool(x, k, s, p, ceil_mode, include_pad):
    """Window sums over a NaN-padded copy: NaN marks taps outside the image.
    Integer-valued inputs keep every sum exact, so one rounding (the
    division) is left and the comparison is exact."""
    N, C, H, W = x.shape
    if ceil_mode:
        OH = (H + 2 * p[0] - k[0] + s[0] - 1) // s[0] + 1
        OW = (W + 2 * p[1] - k[1] + s[1] - 1) // s[1] + 1
    else:
        OH = (H + 2 * p[0] - k[0]) // s[0] + 1
        OW = (W + 2 * p[1] - k[1]) // s[1] + 1
    big = np.full((N, C, OH * s[0] + k[0] + p[0], OW * s[1] + k[1] + p[1]), np.nan)
    big[:, :, p[0]:p[0] + H, p[1]:p[1] + W] = x
    y = np.empty((N, C, OH, OW), np.float32)
    for oh in range(OH):
        for ow in range(OW):
            win = big[:, :, oh * s[0]:oh * s[0] + k[0], ow * s[1]:ow * s[1] + k[1]].reshape(N, C, -1)
            inside = ~np.isnan(win)
            total = np.where(inside, win, 0.0).sum(-1)
            count = np.full((N, C), k[0] * k[1]) if include_pad else inside.sum(-1)
            y[:, :, oh, ow] = np.where(count > 0, total.astype(np.float32) / np.maximum(count, 1).astype(np.float32), 0)
    return y


@pytest.mark.parametrize("k,s,p,ceil_mode,include_pad", [
    ((2, 2), (2, 2), (0, 0), False, False), ((3, 3), (2, 2), (1, 1), False, False),
    ((3, 3), (2, 2), (1, 1), False, True), ((3, 3), (2, 2), (0, 0), True, False),
    ((3, 3), (2, 2), (0, 0), True, True), ((2, 3), (1, 2), (1, 1), False, True)])
def test_avgpool_vs_numpy(orc, k, s, p, ceil_mode, include_pad):
    rng = np.random.default_rng(16)
    x = rng.integers(-50, 50, size=(2, 3, 9, 8)).astype(np.float32)
    got = orc.avgpool2d(x, k, s, p, ceil_mode=ceil_mode, count_include_pad=include_pad)
    assert np.array_equal(got, _np_avgpool(x, k, s, p, ceil_mode, include_pad))


def test_global_maxpool_special_values(orc):
    rng = np.random.default_rng(17)
    x = rng.standard_normal((2, 3, 5, 6)).astype(np.float32)
    x[0, 0, 1, 2] = np.nan
    x[1, 2] = np.nan  # an all-NaN plane keeps the -inf start
    y = orc.global_maxpool2d(x)
    want = np.nanmax(np.where(np.isnan(x), -np.inf, x).reshape(2, 3, -1), axis=-1).astype(np.float32)
    assert np.array_equal(y, want)
    assert y[1, 2] == -np.inf
    # equal -0 / +0: the first in memory order is kept
    z = np.zeros((1, 2, 1, 2), np.float32)
    z[0, 0, 0, 0] = -0.0
    z[0, 1, 0, 1] = -0.0
    zy = orc.global_maxpool2d(z)
    assert np.signbit(zy[0, 0]) and not np.signbit(zy[0, 1])


@pytest.mark.parametrize("transA,transB", [(False, False), (False, True), (True, False)])
def test_gemm_f32_blocked(orc, transA, transB):
    rng = np.random.default_rng(15)
    M, K, N = 70, 130, 90
    A = rng.standard_normal((K, M) if transA else (M, K)).astype(np.float32)
    B = rng.standard_normal((N, K) if transB else (K, N)).astype(np.float32)
    C1 = rng.standard_normal(N).astype(np.float32)
    out = orc.gemm_f32_blocked(A, B, C1, 0.5, 2.0, transA, transB)
    ref = 0.5 * ((A.T if transA else A).astype(np.float64) @ (B.T if transB else B).astype(np.float64)) + 2.0 * C1
    rm.assert_within_tolerance(out, ref, K, np.abs(A).max() * np.abs(B).max())
