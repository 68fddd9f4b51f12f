"""float x binary / float x ternary GEMM on the GPU vs the oracle (north_star
subsystem 2).  Tolerance (north_star): rel-L2 <= 1e-5 and max-abs <=
1e-4*sqrt(K)*max|x| (x = activations times the largest column multiplier)
against the float64 oracle; the fp32 sequential oracle is checked the same way.
Full-size shapes (4096^3) are checked through size-independent properties:
exact row spot checks, column checksums and linearity."""
import ctypes

import numpy as np
import pytest
import torch

import refmath as rm
import gpu_util
import tbn_hip
from gpu_util import P, empty, host, to_dev

pytestmark = pytest.mark.gpu


def make_binary_problem(M, K, N, seed, lda=None):
    rng = np.random.default_rng(seed)
    lda = lda or K
    A = rng.standard_normal((M, lda)).astype(np.float32)
    binw = (rng.random((K, N)) < 0.5).astype(np.uint8)
    scale = rng.uniform(0.5, 1.5, N).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
    return A, binw, scale, bias


def gpu_pack_binary(binw, K, N):
    K_pad, N_pad = tbn_hip.padded_dims(K, N)
    packed = empty(N_pad * K_pad // 8, torch.uint8)
    tbn_hip.call("tbn_hip_pack_binary", P(to_dev(binw)), K, N, tbn_hip.LAYOUT_KN, K_pad, N_pad, P(packed), None)
    return packed, K_pad, N_pad


def run_gemm(kind, A, lda, M, N, K, packed, K_pad, N_pad, scale=None, alpha=1.0, bias=None, flags=0, ldc=None):
    ldc = ldc or N
    dA = A if isinstance(A, torch.Tensor) else to_dev(A)
    gpu_util._KEEP.append(dA)
    C = empty((M, ldc), torch.float32)
    C.fill_(np.nan)
    ds = None if scale is None else to_dev(scale)
    db = None if bias is None else to_dev(bias)
    tbn_hip.call(f"tbn_hip_gemm_f32_{kind}", P(dA), lda, M, N, K, P(packed), K_pad, N_pad, P(ds), alpha, P(db),
                 flags, P(C), ldc, None)
    return C


@pytest.mark.parametrize("M,K,N,lda", [(1, 25, 6, 25), (1, 256, 10, 256), (7, 300, 13, 301), (64, 64, 64, 64),
                                       (130, 257, 70, 260), (33, 1000, 129, 1000), (200, 576, 128, 576)])
def test_gemm_binary_small_shapes(dev, orc, M, K, N, lda):
    A, binw, scale, bias = make_binary_problem(M, K, N, seed=M * 1000 + K, lda=lda)
    packed, K_pad, N_pad = gpu_pack_binary(binw, K, N)
    Ak = np.ascontiguousarray(A[:, :K])
    hp = host(packed)
    for flags, alpha in [(0, 1.0), (tbn_hip.EPI_RELU, 0.7), (tbn_hip.EPI_BIAS_THEN_SCALE, 1.3)]:
        out = host(run_gemm("binary", A, lda, M, N, K, packed, K_pad, N_pad, scale, alpha, bias, flags))
        ref = orc.gemm_f64_binary(Ak, hp, K_pad, N, scale, alpha, bias, bool(flags & 1)) \
            if not flags & tbn_hip.EPI_BIAS_THEN_SCALE else \
            rm.f64_gemm(Ak, rm.np_unpack_binary(hp, K, N, K_pad), scale, alpha, bias, bias_then_scale=True)
        rm.assert_within_tolerance(out, ref, K, np.abs(A).max() * alpha * 1.5)
    # the sequential-fp32 reference loop (qlinear_matmul_binary_naive) is within the same bound
    out = host(run_gemm("binary", A, lda, M, N, K, packed, K_pad, N_pad))
    rm.assert_within_tolerance(out, orc.qlinear_matmul_binary_naive(Ak, binw, 1.0), K, np.abs(A).max())


def test_gemm_binary_no_scale_no_bias_and_ldc(dev, orc):
    M, K, N = 50, 128, 40
    A, binw, _, _ = make_binary_problem(M, K, N, seed=5)
    packed, K_pad, N_pad = gpu_pack_binary(binw, K, N)
    C = host(run_gemm("binary", A, K, M, N, K, packed, K_pad, N_pad, ldc=48))
    ref = orc.gemm_f64_binary(A, host(packed), K_pad, N)
    rm.assert_within_tolerance(C[:, :N], ref, K, np.abs(A).max())
    assert np.isnan(C[:, N:]).all()  # columns past N untouched


def test_gemm_binary_cfg2_1024(dev, orc):
    """Config 2: M=N=K=1024, A ~ N(0,1), W +-1 p=0.5, per-column scale U[0.5,1.5]."""
    M = N = K = 1024
    A, binw, scale, _ = make_binary_problem(M, K, N, seed=2)
    packed, K_pad, N_pad = gpu_pack_binary(binw, K, N)
    out = host(run_gemm("binary", A, K, M, N, K, packed, K_pad, N_pad, scale))
    ref = orc.gemm_f64_binary(A, host(packed), K_pad, N, scale)
    r, m = rm.assert_within_tolerance(out, ref, K, np.abs(A).max() * 1.5)
    assert r < 1e-6  # exact products, fp32 accumulation


def test_gemm_headline_4096_properties(dev, orc):
    """4096^3 float x binary: exact oracle rows, column checksum, linearity."""
    M = N = K = 4096
    rng = np.random.default_rng(42)
    A = rng.standard_normal((M, K)).astype(np.float32)
    binw = (rng.random((K, N)) < 0.5).astype(np.uint8)
    scale = rng.uniform(0.5, 1.5, N).astype(np.float32)
    packed, K_pad, N_pad = gpu_pack_binary(binw, K, N)
    dA = to_dev(A)
    C = run_gemm("binary", dA, K, M, N, K, packed, K_pad, N_pad, scale)
    hp = host(packed)
    rows = rng.choice(M, 24, replace=False)
    rows = np.concatenate([[0, M - 1], rows])
    Cr = host(C)[rows]
    ref_rows = orc.gemm_f64_binary(A[rows], hp, K_pad, N, scale)
    rm.assert_within_tolerance(Cr, ref_rows, K, np.abs(A).max() * 1.5)
    # column checksum: sum_m C[m, :] == (sum_m A[m, :]) W diag(s)
    colsum = host(C).astype(np.float64).sum(axis=0)
    asum = A.astype(np.float64).sum(axis=0)
    W = rm.np_unpack_binary(hp, K, N, K_pad).astype(np.float64)
    expect = (asum @ W) * scale.astype(np.float64)
    assert rm.rel_l2(colsum, expect) < 1e-5
    # linearity: C(A1 + A2) == C(A1) + C(A2) within fp32 accumulation error
    A2 = rng.standard_normal((M, K)).astype(np.float32)
    C2 = run_gemm("binary", to_dev(A2), K, M, N, K, packed, K_pad, N_pad, scale)
    C12 = run_gemm("binary", dA + to_dev(A2), K, M, N, K, packed, K_pad, N_pad, scale)
    lhs = host(C12).astype(np.float64)
    rhs = host(C).astype(np.float64) + host(C2)
    assert rm.rel_l2(lhs, rhs) < 1e-5


def _f64_dev_gemm(A, binw, scale, alpha=1.0, bias=None, cin=None, beta=0.0, relu=False, bias_then_scale=False):
    """float64 A @ W on the GPU (binw 1 -> +1, 0 -> -1, as tbn_hip_pack_binary reads it), then the epilogue."""
    dA = torch.as_tensor(A, dtype=torch.float64, device="cuda")
    dW = 2.0 * torch.as_tensor(binw, dtype=torch.float64, device="cuda") - 1.0
    acc = dA @ dW
    s = torch.as_tensor(scale, dtype=torch.float64, device="cuda") * alpha
    b = 0.0 if bias is None else torch.as_tensor(bias, dtype=torch.float64, device="cuda")
    out = (acc + b) * s if bias_then_scale else acc * s + b
    if cin is not None:
        out = out + beta * torch.as_tensor(cin, dtype=torch.float64, device="cuda")
    if relu:
        out = out.clamp_min(0.0)
    return out.cpu().numpy()


@pytest.mark.parametrize("M,K,N,lda", [(2048, 4096, 4096, 4096), (2000, 1000, 4000, 1004), (1500, 1064, 5000, 1064)])
def test_gemm_binary_wide_tiles(dev, orc, M, K, N, lda):
    """Shapes taken by the wide-tile kernel (128 x 512 block tiles): ragged M / N,
    a K tail (K % 32 != 0), padded rows (lda > K); every element checked against
    float64, sampled rows against the oracle, all epilogue variants."""
    A, binw, scale, bias = make_binary_problem(M, K, N, seed=M + K + N, lda=lda)
    packed, K_pad, N_pad = gpu_pack_binary(binw, K, N)
    Ak = np.ascontiguousarray(A[:, :K])
    dA = to_dev(A)
    xmax = np.abs(A).max() * 1.5
    for flags, alpha in [(0, 1.0), (tbn_hip.EPI_RELU, 0.7), (tbn_hip.EPI_BIAS_THEN_SCALE, 1.3)]:
        out = host(run_gemm("binary", dA, lda, M, N, K, packed, K_pad, N_pad, scale, alpha, bias, flags))
        ref = _f64_dev_gemm(Ak, binw, scale, alpha, bias, relu=bool(flags & tbn_hip.EPI_RELU),
                            bias_then_scale=bool(flags & tbn_hip.EPI_BIAS_THEN_SCALE))
        r, _ = rm.assert_within_tolerance(out, ref, K, xmax * alpha)
        assert r < 1e-6
    rows = np.array([0, 1, M // 2, M - 1])
    out = host(run_gemm("binary", dA, lda, M, N, K, packed, K_pad, N_pad, scale, 1.0, bias))
    ref = orc.gemm_f64_binary(Ak[rows], host(packed), K_pad, N, scale, 1.0, bias, False)
    rm.assert_within_tolerance(out[rows], ref, K, xmax)
    # GEMM with an fp32 addend (ONNX Gemm C): [M, N] and [N]
    rng = np.random.default_rng(7)
    cin = rng.standard_normal((M, N)).astype(np.float32)
    c1 = rng.standard_normal(N).astype(np.float32)
    for c, is1d in [(cin, 1), (c1, 1), (cin, 0)]:
        if is1d and c.ndim == 2:
            continue
        dc = to_dev(c)
        C = empty((M, N), torch.float32)
        tbn_hip.call("tbn_hip_gemm_f32_quantized", tbn_hip.WEIGHTS_BINARY, P(dA), lda, M, N, K, P(packed), K_pad,
                     N_pad, P(to_dev(scale)), 0.5, None, P(dc), is1d, 2.0, 0, P(C), N, None)
        ref = _f64_dev_gemm(Ak, binw, scale, 0.5, None, cin=c, beta=2.0)
        rm.assert_within_tolerance(host(C), ref, K, xmax)


def _f64_dev_ternary(A, t, scale, alpha=1.0, bias=None, relu=False, bias_then_scale=False, cin=None, beta=0.0):
    dA = torch.as_tensor(A, dtype=torch.float64, device="cuda")
    dT = torch.as_tensor(t, dtype=torch.float64, device="cuda")
    acc = dA @ dT
    s = torch.as_tensor(scale, dtype=torch.float64, device="cuda") * alpha
    b = 0.0 if bias is None else torch.as_tensor(bias, dtype=torch.float64, device="cuda")
    out = (acc + b) * s if bias_then_scale else acc * s + b
    if cin is not None:
        out = out + beta * torch.as_tensor(cin, dtype=torch.float64, device="cuda")
    if relu:
        out = out.clamp_min(0.0)
    return out.cpu().numpy()


@pytest.mark.parametrize("M,K,N", [(256, 4096, 4096), (384, 2600, 2600), (2048, 1024, 4096), (130, 1000, 700)])
def test_gemm_ternary_wide_and_split(dev, orc, M, K, N):
    """Ternary weights through the wide kernel: split-K for few tiles (the
    first two shapes), one pass for many (the third); the last shape stays on
    the small-tile engine.  Every element against float64, all epilogues."""
    rng = np.random.default_rng(M + K + N)
    A = rng.standard_normal((M, K)).astype(np.float32)
    t = rng.choice(np.array([-1, 0, 1], np.int8), size=(K, N), p=[0.3, 0.4, 0.3])
    scale = rng.uniform(0.5, 1.5, N).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
    K_pad = (K + 63) // 64 * 64
    packed = empty(N * K_pad // 4, torch.uint8)
    tbn_hip.call("tbn_hip_pack_ternary", P(to_dev(t)), K, N, tbn_hip.LAYOUT_KN, K_pad, N, P(packed), None)
    dA = to_dev(A)
    xmax = np.abs(A).max() * 1.5
    for flags, alpha in [(0, 1.0), (tbn_hip.EPI_RELU, 0.7), (tbn_hip.EPI_BIAS_THEN_SCALE, 1.3)]:
        out = host(run_gemm("ternary", dA, K, M, N, K, packed, K_pad, N, scale, alpha, bias, flags))
        ref = _f64_dev_ternary(A, t, scale, alpha, bias, relu=bool(flags & tbn_hip.EPI_RELU),
                               bias_then_scale=bool(flags & tbn_hip.EPI_BIAS_THEN_SCALE))
        r, _ = rm.assert_within_tolerance(out, ref, K, xmax * alpha)
        assert r < 1e-6
    rows = np.array([0, M // 3, M - 1])
    out = host(run_gemm("ternary", dA, K, M, N, K, packed, K_pad, N, scale, 0.5))
    ref = orc.gemm_f64_ternary(A[rows], host(packed), K_pad, N, scale, 0.5)
    rm.assert_within_tolerance(out[rows], ref, K, xmax)
    # deterministic: a second launch gives identical bits
    out2 = host(run_gemm("ternary", dA, K, M, N, K, packed, K_pad, N, scale, 0.5))
    assert np.array_equal(out.view(np.uint32), out2.view(np.uint32))


@pytest.mark.parametrize("M,K,N", [(640, 2000, 2048), (256, 4096, 4096), (512, 777, 4000)])
def test_gemm_binary_split_k(dev, orc, M, K, N):
    """Binary GEMMs with few wide tiles split K and reduce in a second pass:
    ragged M / N / K, the fp32 addend, bit-for-bit repeatable."""
    A, binw, scale, bias = make_binary_problem(M, K, N, seed=M * 3 + K)
    packed, K_pad, N_pad = gpu_pack_binary(binw, K, N)
    dA = to_dev(A)
    xmax = np.abs(A).max() * 1.5
    out = host(run_gemm("binary", dA, K, M, N, K, packed, K_pad, N_pad, scale, 0.9, bias, tbn_hip.EPI_RELU))
    ref = _f64_dev_gemm(A, binw, scale, 0.9, bias, relu=True)
    r, _ = rm.assert_within_tolerance(out, ref, K, xmax)
    assert r < 1e-6
    out2 = host(run_gemm("binary", dA, K, M, N, K, packed, K_pad, N_pad, scale, 0.9, bias, tbn_hip.EPI_RELU))
    assert np.array_equal(out.view(np.uint32), out2.view(np.uint32))
    cin = np.random.default_rng(1).standard_normal((M, N)).astype(np.float32)
    C = empty((M, N), torch.float32)
    tbn_hip.call("tbn_hip_gemm_f32_quantized", tbn_hip.WEIGHTS_BINARY, P(dA), K, M, N, K, P(packed), K_pad, N_pad,
                 P(to_dev(scale)), 1.0, None, P(to_dev(cin)), 0, -1.5, 0, P(C), N, None)
    ref = _f64_dev_gemm(A, binw, scale, 1.0, None, cin=cin, beta=-1.5)
    rm.assert_within_tolerance(host(C), ref, K, xmax)


def test_gemm_binary_wide_special_values(dev):
    """inf / nan rows through the wide kernel: +-inf per column sign, nan rows stay nan."""
    M, K, N = 2048, 512, 4096
    A, binw, scale, _ = make_binary_problem(M, K, N, seed=11)
    A[0, 5] = np.inf
    A[1, 7] = -np.inf
    A[2, 9] = np.nan
    packed, K_pad, N_pad = gpu_pack_binary(binw, K, N)
    out = host(run_gemm("binary", A, K, M, N, K, packed, K_pad, N_pad, scale))
    sign = 2.0 * binw - 1.0
    assert np.array_equal(out[0], np.where(sign[5] > 0, np.inf, -np.inf).astype(np.float32))
    assert np.array_equal(out[1], np.where(sign[7] > 0, -np.inf, np.inf).astype(np.float32))
    assert np.isnan(out[2]).all()
    ref = _f64_dev_gemm(A[3:], binw, scale)
    rm.assert_within_tolerance(out[3:], ref, K, np.abs(A[3:]).max() * 1.5)


@pytest.mark.parametrize("M,K,N", [(1, 2, 2), (9, 260, 17), (64, 512, 96)])
def test_gemm_ternary_small(dev, orc, M, K, N):
    rng = np.random.default_rng(M + K + N)
    A = rng.standard_normal((M, K)).astype(np.float32)
    t = rng.choice([-1, 0, 1], size=(K, N), p=[0.3, 0.4, 0.3]).astype(np.int8)
    scale = rng.uniform(0.5, 1.5, N).astype(np.float32)
    K_pad = (K + 31) // 32 * 32
    packed = empty(N * K_pad // 4, torch.uint8)
    tbn_hip.call("tbn_hip_pack_ternary", P(to_dev(t)), K, N, tbn_hip.LAYOUT_KN, K_pad, N, P(packed), None)
    out = host(run_gemm("ternary", A, K, M, N, K, packed, K_pad, N, scale, 0.5))
    ref = orc.gemm_f64_ternary(A, host(packed), K_pad, N, scale, 0.5)
    rm.assert_within_tolerance(out, ref, K, np.abs(A).max() * 0.75)


def test_gemm_ternary_known_answer(dev):
    # tbn-runtime/tests/test_quantized_operators.cpp:151-155
    A = np.array([[1.0, 2.0], [3.0, 4.0]], np.float32)
    t = np.array([[1, -1], [0, 1]], np.int8)
    packed = empty(2 * 32 // 4, torch.uint8)
    tbn_hip.call("tbn_hip_pack_ternary", P(to_dev(t)), 2, 2, tbn_hip.LAYOUT_KN, 32, 2, P(packed), None)
    out = host(run_gemm("ternary", A, 2, 2, 2, 2, packed, 32, 2, alpha=0.5))
    assert out.reshape(-1).tolist() == [0.5, 0.5, 1.5, 0.5]


def test_gemm_binary_known_answer(dev):
    # test_quantized_operators.cpp:165-179 inputs, true float x binary
    A = np.array([[1.0, -2.0], [3.0, -4.0]], np.float32)
    packed, K_pad, N_pad = gpu_pack_binary(np.array([[1, 0], [0, 1]], np.uint8), 2, 2)
    out = host(run_gemm("binary", A, 2, 2, 2, 2, packed, K_pad, N_pad, alpha=0.7))
    np.testing.assert_allclose(out.reshape(-1), [2.1, -2.1, 4.9, -4.9], rtol=1e-6)


def test_gemm_ternary_cfg3(dev, orc):
    """Config 3: M=256, N=K=4096, T in {-1,0,1} p={.3,.4,.3}, 2-bit packed, scale U[0.5,1.5]."""
    M, N, K = 256, 4096, 4096
    rng = np.random.default_rng(3)
    A = rng.standard_normal((M, K)).astype(np.float32)
    t = rng.choice(np.array([-1, 0, 1], np.int8), size=(K, N), p=[0.3, 0.4, 0.3])
    scale = rng.uniform(0.5, 1.5, N).astype(np.float32)
    packed = empty(N * K // 4, torch.uint8)
    tbn_hip.call("tbn_hip_pack_ternary", P(to_dev(t)), K, N, tbn_hip.LAYOUT_KN, K, N, P(packed), None)
    out = host(run_gemm("ternary", A, K, M, N, K, packed, K, N, scale))
    rows = np.arange(0, M, 4)
    ref = orc.gemm_f64_ternary(A[rows], host(packed), K, N, scale)
    rm.assert_within_tolerance(out[rows], ref, K, np.abs(A).max() * 1.5)


@pytest.mark.parametrize("M,K,N,lda", [(1, 256, 10, 256), (1000, 300, 7, 301), (33, 128, 64, 128), (5, 8000, 1, 8000)])
def test_gemm_small_heads(dev, M, K, N, lda):
    """Classifier heads (N <= 64, N*K <= 8192) take the LDS FMA kernel: one
    output per thread, row groups looped over the grid, lda > K, the 2-D
    addend and both scale/bias orders; a row's bits do not depend on the
    number of rows."""
    A, binw, scale, bias = make_binary_problem(M, K, N, seed=M + K + N, lda=lda)
    packed, K_pad, N_pad = gpu_pack_binary(binw, K, N)
    xmax = np.abs(A).max() * 1.5
    Ak = A[:, :K]
    for flags, alpha in [(tbn_hip.EPI_RELU, 0.8), (tbn_hip.EPI_BIAS_THEN_SCALE, 1.2)]:
        out = host(run_gemm("binary", A, lda, M, N, K, packed, K_pad, N_pad, scale, alpha, bias, flags))
        ref = _f64_dev_gemm(Ak, binw, scale, alpha, bias, relu=bool(flags & tbn_hip.EPI_RELU),
                            bias_then_scale=bool(flags & tbn_hip.EPI_BIAS_THEN_SCALE))
        rm.assert_within_tolerance(out, ref, K, xmax * alpha)
        last = host(run_gemm("binary", A[M - 1:].copy(), lda, 1, N, K, packed, K_pad, N_pad, scale, alpha, bias,
                             flags))
        assert np.array_equal(last.view(np.uint32), out[M - 1:].view(np.uint32))
    cin = np.random.default_rng(3).standard_normal((M, N)).astype(np.float32)
    C = empty((M, N), torch.float32)
    tbn_hip.call("tbn_hip_gemm_f32_quantized", tbn_hip.WEIGHTS_BINARY, P(to_dev(A)), lda, M, N, K, P(packed), K_pad,
                 N_pad, P(to_dev(scale)), 1.0, None, P(to_dev(cin)), 0, -0.5, 0, P(C), N, None)
    rm.assert_within_tolerance(host(C), _f64_dev_gemm(Ak, binw, scale, 1.0, None, cin=cin, beta=-0.5), K, xmax)
    t = np.random.default_rng(M).choice(np.array([-1, 0, 1], np.int8), size=(K, N))
    K_pad4 = (K + 31) // 32 * 32
    tp = empty(N * K_pad4 // 4, torch.uint8)
    tbn_hip.call("tbn_hip_pack_ternary", P(to_dev(t)), K, N, tbn_hip.LAYOUT_KN, K_pad4, N, P(tp), None)
    out = host(run_gemm("ternary", A, lda, M, N, K, tp, K_pad4, N, scale, 0.9, bias, tbn_hip.EPI_RELU))
    rm.assert_within_tolerance(out, _f64_dev_ternary(Ak, t, scale, 0.9, bias, relu=True), K, xmax)


def test_gemm_special_values(dev, orc):
    M, K, N = 4, 64, 8
    A = np.zeros((M, K), np.float32)
    A[0, 0] = np.inf
    A[1, 3] = -np.inf
    A[2, 5] = np.nan
    A[3, :] = np.float32(1e-30)
    A[3, 1] = -0.0
    binw = np.ones((K, N), np.uint8)
    binw[0, 1] = 0
    packed, K_pad, N_pad = gpu_pack_binary(binw, K, N)
    out = host(run_gemm("binary", A, K, M, N, K, packed, K_pad, N_pad))
    ref = orc.gemm_f32_binary(A, host(packed), K_pad, N)
    assert np.array_equal(np.isinf(out), np.isinf(ref)) and np.array_equal(np.sign(out[:2]), np.sign(ref[:2]))
    assert np.isnan(out[2]).all() and np.isnan(ref[2]).all()
    np.testing.assert_allclose(out[3], ref[3], rtol=1e-6)


def test_gemm_f32_matches_blocked_reference(dev, orc):
    rng = np.random.default_rng(21)
    for (M, K, N, ta, tb) in [(32, 512, 1000, False, False), (1, 256, 10, False, True), (70, 130, 90, True, False)]:
        A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
        B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
        c1 = rng.standard_normal(N).astype(np.float32)
        out = empty((M, N), torch.float32)
        tbn_hip.call("tbn_hip_gemm_f32", P(to_dev(A)), P(to_dev(B)), P(to_dev(c1)), 1, M, K, N, 0.5, 2.0,
                     int(ta), int(tb), 0, P(out), None)
        ref = 0.5 * ((A.T if ta else A).astype(np.float64) @ (B.T if tb else B).astype(np.float64)) + 2.0 * c1
        rm.assert_within_tolerance(host(out), ref, K, np.abs(A).max() * np.abs(B).max())
        rm.assert_within_tolerance(orc.gemm_f32_blocked(A, B, c1, 0.5, 2.0, ta, tb), ref, K,
                                   np.abs(A).max() * np.abs(B).max())


def test_gemm_f32_rows_and_split_k(dev, orc):
    """The many-columns kernel (64 < N <= 4096, 256 <= K <= 4096: k chunks of
    512 staged as fp32, float4 or strided loads, a K that leaves a short last
    chunk) and K split over MFMA blocks (K > 4096, a short last split): 2-D
    addend, ReLU, transposed operands; rows are bit-identical whatever the
    number of rows (the path and the split count depend on N and K only)."""
    rng = np.random.default_rng(22)
    for (M, K, N, ta, tb, relu) in [(33, 600, 70, True, False, True), (5, 1030, 257, False, True, False),
                                     (64, 512, 1000, False, True, True), (96, 520, 130, False, False, False),
                                     (40, 4616, 70, False, True, True)]:
        A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
        B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
        c2 = rng.standard_normal((M, N)).astype(np.float32)
        out = empty((M, N), torch.float32)
        flags = tbn_hip.EPI_RELU if relu else 0
        tbn_hip.call("tbn_hip_gemm_f32", P(to_dev(A)), P(to_dev(B)), P(to_dev(c2)), 0, M, K, N, 1.5, -0.5,
                     int(ta), int(tb), flags, P(out), None)
        ref = 1.5 * ((A.T if ta else A).astype(np.float64) @ (B.T if tb else B).astype(np.float64)) - 0.5 * c2
        if relu:
            ref = np.maximum(ref, 0.0)
        rm.assert_within_tolerance(host(out), ref, K, np.abs(A).max() * np.abs(B).max())
        if not ta:
            few = empty((2, N), torch.float32)
            tbn_hip.call("tbn_hip_gemm_f32", P(to_dev(A[3:5].copy())), P(to_dev(B)), P(to_dev(c2[3:5].copy())), 0,
                         2, K, N, 1.5, -0.5, 0, int(tb), flags, P(few), None)
            assert np.array_equal(host(few), host(out)[3:5])


def test_gemm_error_codes(dev):
    packed = empty(64, torch.uint8)
    A = empty((4, 64), torch.float32)
    C = empty((4, 8), torch.float32)
    with pytest.raises(tbn_hip.TbnError) as e:
        tbn_hip.call("tbn_hip_gemm_f32_binary", P(A), 64, 4, 8, 64, P(packed), 40, 8, None, 1.0, None, 0, P(C), 8, None)
    assert e.value.code == tbn_hip.INVALID_SHAPE
    with pytest.raises(tbn_hip.TbnError) as e:
        tbn_hip.call("tbn_hip_gemm_f32_binary", P(A), 64, 4, 8, 64, None, 64, 8, None, 1.0, None, 0, P(C), 8, None)
    assert e.value.code == tbn_hip.INVALID_ARGUMENT
    # empty problems are no-ops
    tbn_hip.call("tbn_hip_gemm_f32_binary", None, 0, 0, 8, 64, None, 64, 8, None, 1.0, None, 0, None, 8, None)


# (tile, forced splits) -> (M, K, N): each shape gives the forced tile enough
# blocks to run on the wide kernels (gemm_wide_fits), with ragged M and N and
# a partial last K step (K = 1100); the K-group tile ignores a forced split.
WIDE_CASES = {(0, 1): (1100, 1100, 4000), (0, 3): (300, 1100, 3600), (0, 8): (300, 1100, 1600),
              (1, 1): (300, 1100, 3300), (1, 2): (300, 1100, 1700), (1, 5): (300, 1100, 700),
              (1, 8): (300, 1100, 700), (2, 1): (300, 1100, 1000), (2, 4): (300, 1100, 1000)}
WIDE_FAMILY = {0: "gemm_wide_kernel<WideCfg<128, 512,", 1: "gemm_mid_kernel<WideCfg<64, 128,",
               2: "gemm_mid_kernel<WideCfg<32, 128,"}


def gemm_kernel_name(ternary, M, N, K, K_pad, N_pad):
    name = ctypes.create_string_buffer(256)
    tbn_hip.call("tbn_hip_gemm_kernel_name", int(ternary), M, N, K, K, K_pad, N_pad, name, 256)
    return name.value.decode()


def make_wide_operands(rng, M, K, N, ternary):
    """A, scale, bias and the packed weights of one wide-tile case, with the
    float64 product of its sign matrix for the checker."""
    A = rng.standard_normal((M, K)).astype(np.float32)
    scale = rng.uniform(0.5, 1.5, N).astype(np.float32)
    bias = (rng.standard_normal(N) * 0.01).astype(np.float32)
    K_pad, N_pad = tbn_hip.padded_dims(K, N)
    if ternary:
        t = rng.choice(np.int8([-1, 0, 1]), size=(K, N), p=[0.3, 0.4, 0.3])
        packed = empty(N_pad * K_pad // 4, torch.uint8)
        tbn_hip.call("tbn_hip_pack_ternary", P(to_dev(t)), K, N, tbn_hip.LAYOUT_KN, K_pad, N_pad, P(packed), None)
        ref = lambda: _f64_dev_ternary(A, t, scale, bias=bias, relu=True)  # noqa: E731
    else:
        binw = (rng.random((K, N)) < 0.5).astype(np.uint8)
        packed, K_pad, N_pad = gpu_pack_binary(binw, K, N)
        ref = lambda: _f64_dev_gemm(A, binw, scale, bias=bias, relu=True)  # noqa: E731
    return A, scale, bias, packed, K_pad, N_pad, ref


@pytest.mark.parametrize("tile,splits", sorted(WIDE_CASES))
@pytest.mark.parametrize("ternary", [False, True], ids=["binary", "ternary"])
def test_gemm_wide_every_tile_and_split(dev, orc, tile, splits, ternary):
    """Each wide tile (128x512, 64x128, and 32x128 whose two K groups each
    take half of the 18 K steps, the last one partial), whole or with K split
    over blocks whose last finisher adds the splits in split order: the kernel
    the library names is the forced tile's (split-K where forced), the result
    is within the tolerance of the float64 product, and bit-identical on a
    second run (the order does not depend on which block finishes last)."""
    M, K, N = WIDE_CASES[(tile, splits)]
    rng = np.random.default_rng(tile * 10 + splits + 100 * ternary)
    A, scale, bias, packed, K_pad, N_pad, ref = make_wide_operands(rng, M, K, N, ternary)
    kind = "ternary" if ternary else "binary"
    with tbn_hip.tuning(tbn_hip.TUNE_GEMM_TILE, tile), tbn_hip.tuning(tbn_hip.TUNE_GEMM_SPLITS, splits):
        name = gemm_kernel_name(ternary, M, N, K, K_pad, N_pad)
        c1 = host(run_gemm(kind, A, K, M, N, K, packed, K_pad, N_pad, scale, 1.0, bias, tbn_hip.EPI_RELU))
        c2 = host(run_gemm(kind, A, K, M, N, K, packed, K_pad, N_pad, scale, 1.0, bias, tbn_hip.EPI_RELU))
    assert name.startswith(WIDE_FAMILY[tile]), name
    assert name.endswith(", true>" if splits > 1 and tile != 2 else ", false>"), name
    assert np.array_equal(c1.view(np.uint32), c2.view(np.uint32))
    rm.assert_within_tolerance(c1, ref(), K, np.abs(A).max() * 1.5)


@pytest.mark.parametrize("tile,splits", [(0, 1), (0, 8), (1, 5), (2, 1)])
@pytest.mark.parametrize("ternary", [False, True], ids=["binary", "ternary"])
def test_gemm_wide_leaves_memory_past_the_output_alone(dev, orc, tile, splits, ternary):
    """Ragged M through each wide tile, whole and split over K (the partial
    sums' row step lives in the buffer resource's base, so rows past M stay
    range-checked): 32 guard rows of NaN after C, and the columns between N
    and ldc, keep their bits; rows < M equal a plain run's."""
    M, K, N = WIDE_CASES[(tile, splits)]
    ldc = N + 8
    rng = np.random.default_rng(17 + tile + splits + 100 * ternary)
    A, scale, _, packed, K_pad, N_pad, _ = make_wide_operands(rng, M, K, N, ternary)
    kind = "ternary" if ternary else "binary"
    big = empty((M + 32, ldc), torch.float32)
    big.fill_(np.nan)
    guard = host(big).view(np.uint32).copy()
    dA, ds = to_dev(A), to_dev(scale)
    with tbn_hip.tuning(tbn_hip.TUNE_GEMM_TILE, tile), tbn_hip.tuning(tbn_hip.TUNE_GEMM_SPLITS, splits):
        assert gemm_kernel_name(ternary, M, N, K, K_pad, N_pad).startswith(WIDE_FAMILY[tile])
        tbn_hip.call(f"tbn_hip_gemm_f32_{kind}", P(dA), K, M, N, K, P(packed), K_pad, N_pad, P(ds), 1.0, None, 0,
                     P(big), ldc, None)
        plain = host(run_gemm(kind, A, K, M, N, K, packed, K_pad, N_pad, scale, 1.0, None, 0))
    out = host(big)
    assert np.array_equal(out[:M, :N].view(np.uint32), plain.view(np.uint32))
    assert np.array_equal(out[M:].view(np.uint32), guard[M:]), "rows past M were written"
    assert np.array_equal(out[:, N:].view(np.uint32), guard[:, N:]), "columns past N were written"


def test_gemm_split_counters_survive_other_workspace_users(dev, orc):
    """The split-K GEMM's tile counters live at the head of the stream
    workspace that conv split-K and TBN mode also use: alternating those
    calls with split GEMMs of other shapes keeps every GEMM correct."""
    rng = np.random.default_rng(77)
    shapes = [(1024, 1024, 1024), (256, 4096, 2048), (130, 700, 900)]
    probs = []
    for M, K, N in shapes:
        A = rng.standard_normal((M, K)).astype(np.float32)
        binw = (rng.random((K, N)) < 0.5).astype(np.uint8)
        packed, K_pad, N_pad = gpu_pack_binary(binw, K, N)
        probs.append((A, binw, packed, K_pad, N_pad, _f64_dev_gemm(A, binw, np.ones(N, np.float32))))
    x = rng.standard_normal((3, 256, 7, 7)).astype(np.float32)
    wb = (rng.random((96, 256 * 9)) < 0.5).astype(np.uint8)
    Kc_pad, Nc_pad = tbn_hip.padded_dims(256 * 9, 96)
    cpk = empty(Nc_pad * Kc_pad // 8, torch.uint8)
    tbn_hip.call("tbn_hip_pack_binary", P(to_dev(wb)), 256 * 9, 96, tbn_hip.LAYOUT_NK, Kc_pad, Nc_pad, P(cpk), None)
    d = tbn_hip.conv_desc(3, 256, 7, 7, 96, 3, 3, 1, 1, 1, 1)
    dx = to_dev(x)
    for rnd in range(2):
        for A, binw, packed, K_pad, N_pad, ref in probs:
            M, K = A.shape
            N = binw.shape[1]
            C = host(run_gemm("binary", A, K, M, N, K, packed, K_pad, N_pad))
            rm.assert_within_tolerance(C, ref, K, np.abs(A).max())
            y = empty((3, 96, 7, 7), torch.float32)  # a split-K conv in between
            tbn_hip.call("tbn_hip_conv2d_f32_binary", P(dx), d, P(cpk), Kc_pad, Nc_pad, None, 1.0, None, 0, P(y),
                         None)


def test_gemm_mid_tile_graph_replay(dev):
    """The config-2 GEMM (32 x 128 tile, two K groups, no workspace) records
    into a HIP graph; each of several replays, with eager work and
    synchronizations between them, matches the eager result bit for bit."""
    M = N = K = 1024
    rng = np.random.default_rng(31)
    A = to_dev(rng.standard_normal((M, K)).astype(np.float32))
    binw = (rng.random((K, N)) < 0.5).astype(np.uint8)
    packed, K_pad, N_pad = gpu_pack_binary(binw, K, N)
    scale = to_dev(rng.uniform(0.5, 1.5, N).astype(np.float32))
    eager = empty((M, N), torch.float32)
    out = empty((M, N), torch.float32)

    def launch(C, stream):
        tbn_hip.call("tbn_hip_gemm_f32_binary", P(A), K, M, N, K, P(packed), K_pad, N_pad, P(scale), 1.0, None,
                     tbn_hip.EPI_RELU, P(C), N, stream)

    launch(eager, None)
    torch.cuda.synchronize()
    cap = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        launch(out, torch.cuda.current_stream().cuda_stream)
    for r in range(3):
        out.fill_(np.nan)
        noise = torch.randn((M, N), device=dev)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r}"
        del noise
