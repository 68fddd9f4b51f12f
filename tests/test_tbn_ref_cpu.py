"""CPU checks of the TBN-mode test reference (tests/tbn_ref.py) and of the
oracle executor's TBN arithmetic (tests/models.py run_oracle(arithmetic=
"tbn")): the decoded ternary im2col and the integer products against brute
force from the definition, the fused multiply-add against 64-bit-mantissa
long double arithmetic (exact for the cases drawn), and the executor on
LeNet against a direct loop restatement of the reference Session."""
import numpy as np
import pytest

import models
import tbn_ref


def t_of(v, lo=-0.1, hi=0.1):
    """The reference's ternarization (quantized_gemm_neon.cpp:93-113):
    v < lo -> -1, v > hi -> +1, else 0 (NaN -> 0)."""
    v = np.asarray(v, np.float32)
    return np.where(v < np.float32(lo), -1, np.where(v > np.float32(hi), 1, 0)).astype(np.int64)


def brute_tbn_conv(x, sign, stride, pad, dil):
    N, C, H, W = x.shape
    M, _, kh, kw = sign.shape
    OH, OW = tbn_ref.conv_out_hw(H, W, kh, kw, stride, pad, dil)
    out = np.zeros((N, M, OH, OW), np.int64)
    t = t_of(x)
    for n in range(N):
        for oh in range(OH):
            for ow in range(OW):
                for r in range(kh):
                    for s in range(kw):
                        ih = oh * stride[0] - pad[0] + r * dil[0]
                        iw = ow * stride[1] - pad[1] + s * dil[1]
                        if 0 <= ih < H and 0 <= iw < W:
                            out[n, :, oh, ow] += sign[:, :, r, s] @ t[n, :, ih, iw]
    return out


@pytest.mark.parametrize("shape,M,k,stride,pad,dil", [((1, 3, 5, 5), 4, 3, (1, 1), (1, 1), (1, 1)),
                                                      ((2, 2, 7, 6), 3, 3, (2, 1), (0, 1), (1, 2)),
                                                      ((1, 5, 6, 6), 2, 1, (2, 2), (0, 0), (1, 1))])
def test_tbn_conv_int_matches_definition(orc, shape, M, k, stride, pad, dil):
    rng = np.random.default_rng(sum(shape) + M)
    x = (rng.standard_normal(shape) * 0.2).astype(np.float32)
    x.reshape(-1)[::5] = np.float32(0.1)
    x.reshape(-1)[1::7] = np.float32(-0.1)
    x.reshape(-1)[2::11] = np.nan
    sign = np.where(rng.random((M, shape[1], k, k)) < 0.5, 1, -1)
    got = tbn_ref.tbn_conv_int(orc, x, sign, stride, pad, dil)
    assert np.array_equal(got, brute_tbn_conv(x, sign, stride, pad, dil))


def test_tbn_gemm_session_matches_definition(orc):
    rng = np.random.default_rng(4)
    A = (rng.standard_normal((5, 70)) * 0.2).astype(np.float32)
    A[0, :4] = [0.1, -0.1, np.nan, np.inf]
    sign = np.where(rng.random((70, 9)) < 0.5, 1, -1)
    C = t_of(A) @ sign
    assert np.array_equal(tbn_ref.tbn_gemm_session(orc, A, sign), C.astype(np.float32))
    cin = rng.standard_normal(9).astype(np.float32)
    got = tbn_ref.tbn_gemm_session(orc, A, sign, alpha=0.3, cin=cin, beta=-1.7)
    want = tbn_ref.fma32(np.float32(-1.7), cin[None, :], C.astype(np.float32) * np.float32(0.3))
    assert np.array_equal(got, want)


def test_fma32_single_rounding():
    # (1 + 2^-12)^2 - 1 = 2^-11 + 2^-24 exactly (fits float32); rounding the
    # product first gives 2^-11
    a = np.float32(1 + 2.0 ** -12)
    assert tbn_ref.fma32(a, a, np.float32(-1.0))[()] == np.float32(2.0 ** -11 + 2.0 ** -24)
    assert np.float32(a * a) - np.float32(1.0) == np.float32(2.0 ** -11)
    assert tbn_ref.fma32(np.float32(3), np.float32(0.5), np.float32(0.25))[()] == np.float32(1.75)


@pytest.mark.skipif(np.finfo(np.longdouble).nmant < 63, reason="needs x87 80-bit long double")
def test_fma32_matches_long_double():
    """a*b + c with |exponent gap| small enough that the sum is exact in a
    64-bit mantissa, so one rounding of the long double gives fma."""
    rng = np.random.default_rng(9)
    a = (rng.standard_normal(4000) * 3).astype(np.float32)
    b = (rng.standard_normal(4000) * 3).astype(np.float32)
    c = (rng.standard_normal(4000) * 3).astype(np.float32)
    exact = np.longdouble(a) * np.longdouble(b) + np.longdouble(c)
    gap_ok = np.abs(np.log2(np.abs(a.astype(np.float64) * b) + 1e-30) - np.log2(np.abs(c) + 1e-30)) < 12
    got = tbn_ref.fma32(a, b, c)
    want = exact.astype(np.float32)
    assert gap_ok.sum() > 3000
    assert np.array_equal(got[gap_ok], want[gap_ok])


def _pool2(v):
    N, M, H, W = v.shape
    return v[:, :, :H // 2 * 2, :W // 2 * 2].reshape(N, M, H // 2, 2, W // 2, 2).max(axis=(3, 5))


@pytest.mark.parametrize("prebinarized", [True, False])
def test_run_oracle_tbn_lenet_matches_direct_restatement(orc, prebinarized):
    """LeNet through run_oracle(arithmetic="tbn") equals the reference
    Session's steps written out directly: per conv, the exact ternarized
    integer conv, + bias, * mean|w| when the weights are already binary
    (signs w >= 0), else signs w > 0 and no scale; Relu; 2x2 pool; Flatten;
    the Gemm float(C) then + bias (alpha = beta = 1)."""
    spec = models.lenet(seed=1, prebinarized=prebinarized)
    x = models.lenet_input(1)
    got = models.run_oracle(spec, {"input": x}, True, orc, arithmetic="tbn")["output"]

    def conv(v, w, b):
        s = orc.channel_mean_abs(w)
        already = orc.already_binary(w, s)
        sign = np.where(w >= 0 if already else w > 0, 1, -1)
        y = brute_tbn_conv(v, sign, (1, 1), (0, 0), (1, 1)).astype(np.float32) + b[None, :, None, None]
        return (y * s[None, :, None, None]).astype(np.float32) if already else y.astype(np.float32)

    i = spec.inits
    assert orc.already_binary(i["w1"], orc.channel_mean_abs(i["w1"])) == prebinarized
    h = _pool2(np.maximum(conv(x, i["w1"], i["b1"]), 0))
    h = _pool2(np.maximum(conv(h, i["w2"], i["b2"]), 0)).reshape(1, -1)
    already = models.gemm_already_binary(i["wf"])
    sign = np.where(i["wf"] >= 0 if already else i["wf"] > 0, 1, -1)
    want = (t_of(h) @ sign).astype(np.float32) + i["bf"][None, :]
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))
