"""Packing and quantization on the GPU: bit-exact against the oracle and the
closed forms (north_star subsystem 1)."""
import numpy as np
import pytest
import torch

import refmath as rm
import tbn_hip
from gpu_util import P, empty, host, to_dev

pytestmark = pytest.mark.gpu

SPECIAL = np.array([0.0, -0.0, np.nan, np.inf, -np.inf, 1e-45, -1e-45, 0.1, -0.1, 3.0, -2.0,
                    np.float32(0.1) + np.float32(1e-8)], np.float32)


def test_elementwise_quantizers_bit_exact(dev, orc):
    rng = np.random.default_rng(0)
    w = np.concatenate([SPECIAL, rng.standard_normal(100003).astype(np.float32) * 0.2])
    n = w.size
    dw = to_dev(w)
    out = empty(n, torch.uint8)
    for thr in (0.0, 0.1, -0.05):
        tbn_hip.call("tbn_hip_quantize_to_binary_f32", P(dw), n, thr, P(out), None)
        assert np.array_equal(host(out), orc.quantize_to_binary_f32(w, thr))
    tbn_hip.call("tbn_hip_sign_ge0_f32", P(dw), n, P(out), None)
    assert np.array_equal(host(out), orc.sign_ge0_f32(w))
    t = empty(n, torch.int8)
    tbn_hip.call("tbn_hip_quantize_to_ternary_f32", P(dw), n, -0.1, 0.1, P(t), None)
    assert np.array_equal(host(t), orc.quantize_to_ternary_f32(w, -0.1, 0.1))
    wi = rng.integers(-128, 128, size=5001).astype(np.int8)
    out_i = empty(wi.size, torch.uint8)
    tbn_hip.call("tbn_hip_quantize_to_binary_i8", P(to_dev(wi)), wi.size, P(out_i), None)
    assert np.array_equal(host(out_i), orc.quantize_to_binary_i8(wi))


@pytest.mark.parametrize("shape", [(6, 1, 5, 5), (16, 6, 5, 5), (512, 256, 3, 3), (130, 7, 3, 3), (100, 1, 1, 65)])
def test_channel_mean_abs_bit_exact(dev, orc, shape):
    rng = np.random.default_rng(1)
    w = rng.standard_normal(shape).astype(np.float32) * 0.1
    out = empty(shape[0], torch.float32)
    tbn_hip.call("tbn_hip_channel_mean_abs", P(to_dev(w)), shape[0], w.size // shape[0], P(out), None)
    assert np.array_equal(host(out), orc.channel_mean_abs(w))


@pytest.mark.parametrize("layout", [tbn_hip.LAYOUT_KN, tbn_hip.LAYOUT_NK])
@pytest.mark.parametrize("K,N", [(1, 1), (25, 6), (150, 16), (256, 10), (300, 13), (576, 128), (4096, 4096)])
def test_pack_binary_bit_exact(dev, orc, layout, K, N):
    rng = np.random.default_rng(K + N + layout)
    binw = rng.integers(0, 3, size=K * N).astype(np.uint8)
    K_pad, N_pad = tbn_hip.padded_dims(K, N)
    out = empty(N_pad * K_pad // 8, torch.uint8)
    out.fill_(0xAB)  # every byte must be written
    tbn_hip.call("tbn_hip_pack_binary", P(to_dev(binw)), K, N, layout, K_pad, N_pad, P(out), None)
    got = host(out)
    assert np.array_equal(got, rm.np_pack_binary(binw, K, N, layout, K_pad, N_pad))
    if K * N <= 200000:
        assert np.array_equal(got, orc.pack_binary(binw, K, N, layout, K_pad, N_pad))
    # the sign decode
    dec = empty(K * N, torch.int8)
    tbn_hip.call("tbn_hip_unpack_binary", P(out), K, N, layout, K_pad, P(dec), None)
    expect = np.where(binw == 1, 1, -1).astype(np.int8)
    assert np.array_equal(host(dec), expect)


@pytest.mark.parametrize("rule,thr", [(tbn_hip.SIGN_GT_THRESHOLD, 0.0), (tbn_hip.SIGN_GT_THRESHOLD, 0.1),
                                      (tbn_hip.SIGN_GE_ZERO, 0.0)])
@pytest.mark.parametrize("layout", [tbn_hip.LAYOUT_KN, tbn_hip.LAYOUT_NK])
def test_quantize_pack_binary_fused(dev, orc, rule, thr, layout):
    rng = np.random.default_rng(3)
    K, N = 300, 37
    w = rng.standard_normal(K * N).astype(np.float32) * 0.1
    w[:SPECIAL.size] = SPECIAL
    K_pad, N_pad = tbn_hip.padded_dims(K, N)
    out = empty(N_pad * K_pad // 8, torch.uint8)
    tbn_hip.call("tbn_hip_quantize_pack_binary_f32", P(to_dev(w)), K, N, layout, rule, thr, K_pad, N_pad,
                 P(out), None)
    binw = orc.quantize_to_binary_f32(w, thr) if rule == tbn_hip.SIGN_GT_THRESHOLD else orc.sign_ge0_f32(w)
    assert np.array_equal(host(out), orc.pack_binary(binw, K, N, layout, K_pad, N_pad))


@pytest.mark.parametrize("K,N", [(300, 37), (64, 8), (1024, 1000)])
@pytest.mark.parametrize("passes", [True, False])
def test_quantize_pack_binary_gemm_sampled(dev, orc, K, N, passes):
    """TBN_SIGN_GEMM_SAMPLED: the Session's Gemm test (model.hpp:773-781)
    decided on the device.  Sampled elements hold -1, 0, -0, +1, +-0.999 (the
    values the test accepts); an unsampled 0.5 does not matter; one sampled
    0.998 rejects the tensor, which then packs as w > 0."""
    rng = np.random.default_rng(K + N)
    w = np.where(rng.random(K * N) < 0.5, 1.0, -1.0).astype(np.float32)
    step = max(1, w.size // 1000)
    sampled = np.arange(0, w.size, step)
    w[sampled[:6]] = [0.0, -0.0, 0.999, -0.999, 1.0, -1.0]
    if step > 1:
        w[sampled[7] + 1] = 0.5   # between samples
    if not passes:
        w[sampled[-1]] = 0.998
    from models import gemm_already_binary
    assert gemm_already_binary(w.reshape(K, N)) == passes
    K_pad, N_pad = tbn_hip.padded_dims(K, N)
    out = empty(N_pad * K_pad // 8, torch.uint8)
    tbn_hip.call("tbn_hip_quantize_pack_binary_f32", P(to_dev(w)), K, N, tbn_hip.LAYOUT_KN,
                 tbn_hip.SIGN_GEMM_SAMPLED, 0.0, K_pad, N_pad, P(out), None)
    binw = orc.sign_ge0_f32(w) if passes else orc.quantize_to_binary_f32(w, 0.0)
    assert np.array_equal(host(out), orc.pack_binary(binw, K, N, tbn_hip.LAYOUT_KN, K_pad, N_pad))


@pytest.mark.parametrize("n", [1, 4, 5, 1001, 4096 * 4096])
def test_pack_ternary2_bit_exact(dev, orc, n):
    rng = np.random.default_rng(n)
    t = rng.integers(-1, 2, size=n).astype(np.int8)
    if n >= 4:
        t[:4] = [5, -7, 1, -1]  # out-of-range values encode as 0
    out = empty((n + 3) // 4, torch.uint8)
    tbn_hip.call("tbn_hip_pack_ternary2", P(to_dev(t)), n, P(out), None)
    got = host(out)
    assert np.array_equal(got, rm.np_ternary_pack2(t))
    if n <= 5000:
        assert np.array_equal(got, orc.ternary_pack2(t))
    dec = empty(n, torch.int8)
    tbn_hip.call("tbn_hip_unpack_ternary2", P(out), n, P(dec), None)
    assert np.array_equal(host(dec), np.clip(np.where(np.abs(t) > 1, 0, t), -1, 1))


def test_pack_ternary2_known_answer(dev):
    out = empty(2, torch.uint8)
    tbn_hip.call("tbn_hip_pack_ternary2", P(to_dev(np.array([-1, 0, 1, 1, -1], np.int8))), 5, P(out), None)
    assert host(out).tolist() == [0xA4, 0x00]
    codes = to_dev(np.array([0b11100100], np.uint8))
    dec = empty(4, torch.int8)
    tbn_hip.call("tbn_hip_unpack_ternary2", P(codes), 4, P(dec), None)
    assert host(dec).tolist() == [-1, 0, 1, 0]


@pytest.mark.parametrize("layout", [tbn_hip.LAYOUT_KN, tbn_hip.LAYOUT_NK])
@pytest.mark.parametrize("K,N", [(2, 2), (70, 11), (4096, 4096)])
def test_pack_ternary_gemm_layout(dev, orc, layout, K, N):
    rng = np.random.default_rng(K * N + layout)
    t = rng.choice([-1, 0, 1], size=K * N, p=[0.3, 0.4, 0.3]).astype(np.int8)
    K_pad, N_pad = (K + 31) // 32 * 32, N
    out = empty(N_pad * K_pad // 4, torch.uint8)
    tbn_hip.call("tbn_hip_pack_ternary", P(to_dev(t)), K, N, layout, K_pad, N_pad, P(out), None)
    got = host(out)
    assert np.array_equal(got, rm.np_pack_ternary(t, K, N, layout, K_pad, N_pad))
    if K * N < 100000:
        assert np.array_equal(got, orc.pack_ternary(t, K, N, layout, K_pad, N_pad))
    w = rng.standard_normal(K * N).astype(np.float32) * 0.2
    tbn_hip.call("tbn_hip_quantize_pack_ternary_f32", P(to_dev(w)), K, N, layout, -0.1, 0.1, K_pad, N_pad,
                 P(out), None)
    q = np.where(w < -0.1, -1, np.where(w > 0.1, 1, 0)).astype(np.int8)
    assert np.array_equal(host(out), rm.np_pack_ternary(q, K, N, layout, K_pad, N_pad))
