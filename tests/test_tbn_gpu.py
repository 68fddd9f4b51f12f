"""TBN mode on the GPU (the reference's production arithmetic): ternary
activation bit planes, im2col_ternary_packed, the integer ternary x binary
GEMM and qlinear_matmul_binary as the reference computes it.  Everything is
integer or a single float(int) * scale, so every check is bit-exact: against
the oracle (oracle/tbn_oracle.c, pinned by tests/test_oracle.py on the
reference's golden vectors), the golden vectors themselves, and exact float64
products on the GPU for the full-size shapes."""
import ctypes

import numpy as np
import pytest
import torch

import tbn_hip
from gpu_util import P, empty, host, to_dev

pytestmark = pytest.mark.gpu

LO, HI = -0.1, 0.1
# the oracle's portable tiling that accepts every padded shape used here
TILING = (128, 256, 256, 16, 8)


def gpu_planes(A, rows, cols):
    M, K = A.shape
    pos = empty(rows * cols // 8, torch.uint8)
    neg = empty(rows * cols // 8, torch.uint8)
    tbn_hip.call("tbn_hip_ternary_pack_f32", P(to_dev(A)), K, M, K, rows, cols, LO, HI, P(pos), P(neg), None)
    return pos, neg


def special_matrix(M, K, seed):
    rng = np.random.default_rng(seed)
    A = (rng.standard_normal((M, K)) * 0.2).astype(np.float32)
    flat = A.reshape(-1)
    vals = np.array([0.1, -0.1, np.nextafter(np.float32(0.1), np.float32(1)),
                     np.nextafter(np.float32(-0.1), np.float32(-1)), np.nan, np.inf, -np.inf, -0.0, 0.0,
                     1e-38, -1e-45], np.float32)
    idx = rng.choice(flat.size, size=min(flat.size, 4 * vals.size), replace=False)
    flat[idx] = np.resize(vals, idx.size)
    return A


@pytest.mark.parametrize("M,K,rows,cols", [(1, 1, 8, 64), (5, 70, 8, 128), (96, 200, 96, 256), (300, 1000, 304, 1024)])
def test_ternary_pack_matches_oracle(dev, orc, M, K, rows, cols):
    A = special_matrix(M, K, seed=M + K)
    pos, neg = gpu_planes(A, rows, cols)
    rc, rp, rn = orc.ternary_matrix_pack_from_float(A, rows, cols, LO, HI)
    assert rc == 0
    assert np.array_equal(host(pos), rp) and np.array_equal(host(neg), rn)


def test_ternary_pack_rejects_reference_invalid_dims(dev):
    A = to_dev(np.zeros((10, 10), np.float32))
    buf = empty(4096, torch.uint8)
    for rows, cols in [(10, 64), (16, 60), (8, 64)]:  # rows % 8, cols % 64, rows < M
        with pytest.raises(tbn_hip.TbnError) as e:
            tbn_hip.call("tbn_hip_ternary_pack_f32", P(A), 10, 10, 10, rows, cols, LO, HI, P(buf), P(buf), None)
        assert e.value.code == tbn_hip.INVALID_ARGUMENT


@pytest.mark.parametrize("shape,k,stride,pad,dil", [((2, 3, 9, 7), 3, (1, 1), (0, 0), (1, 1)),
                                                    ((2, 3, 9, 7), 3, (2, 1), (1, 2), (1, 1)),
                                                    ((1, 5, 12, 12), 3, (1, 1), (1, 1), (2, 2)),
                                                    ((3, 16, 14, 14), 5, (2, 2), (2, 2), (1, 1))])
def test_im2col_ternary_matches_oracle(dev, orc, shape, k, stride, pad, dil):
    rng = np.random.default_rng(sum(shape))
    x = (rng.standard_normal(shape) * 0.3).astype(np.float32)
    x.reshape(-1)[::17] = 0.1
    N, C, H, W = shape
    OH = (H + 2 * pad[0] - dil[0] * (k - 1) - 1) // stride[0] + 1
    OW = (W + 2 * pad[1] - dil[1] * (k - 1) - 1) // stride[1] + 1
    m_pad = (N * OH * OW + 15) // 16 * 16
    k_pad = (C * k * k + 127) // 128 * 128
    d = tbn_hip.conv_desc(N, C, H, W, 8, k, k, *stride, *pad, *dil)
    pos = empty(m_pad * k_pad // 8, torch.uint8)
    neg = empty(m_pad * k_pad // 8, torch.uint8)
    tbn_hip.call("tbn_hip_im2col_ternary_packed", P(to_dev(x)), ctypes.byref(d), m_pad, k_pad, LO, HI, P(pos),
                 P(neg), None)
    rc, rp, rn = orc.im2col_ternary_packed(x, k, k, stride, pad, dil, m_pad, k_pad, LO, HI)
    assert rc == 0
    assert np.array_equal(host(pos), rp) and np.array_equal(host(neg), rn)


def run_tbn_gemm(pos, neg, bits, m, n, k):
    C = empty((m, k), torch.int32)
    tbn_hip.call("tbn_hip_tbn_gemm", P(pos), P(neg), P(bits), m, n, k, P(C), None)
    return host(C)


def test_tbn_gemm_golden_128(dev, orc):
    """GeMM/05-final/matrices_to_test.hpp: C = sign(A @ B) (the reference's own
    check), and the full int32 product by brute force."""
    g = dict(np.load(__import__("pathlib").Path(__file__).with_name("golden") / "gemm_golden.npz"))
    A, B, C = g["A128"], g["B128"], g["C128"]
    pos, neg = gpu_planes(A.astype(np.float32), 128, 128)
    rc, bits = orc.binary_matrix_pack(B, 128, 128)
    assert rc == 0
    out = run_tbn_gemm(pos, neg, to_dev(bits), 128, 128, 128)
    assert np.array_equal(np.sign(out), C)
    assert np.array_equal(out, A.astype(np.int64) @ B.astype(np.int64))


def test_tbn_gemm_golden_64_padded(dev, orc):
    g = dict(np.load(__import__("pathlib").Path(__file__).with_name("golden") / "gemm_golden.npz"))
    A = np.zeros((64, 128), np.float32); A[:, :64] = g["A64"]
    B = np.ones((128, 64), np.int8); B[:64] = g["B64"]
    pos, neg = gpu_planes(A, 64, 128)
    _, bits = orc.binary_matrix_pack(B, 128, 64)
    out = run_tbn_gemm(pos, neg, to_dev(bits), 64, 128, 64)
    assert np.array_equal(np.sign(out), g["C64"])


@pytest.mark.parametrize("m,n,k", [(16, 128, 8), (48, 256, 40), (160, 512, 136), (528, 1024, 600), (64, 192, 72),
                                   (128, 320, 104), (296, 2112, 520)])
def test_tbn_gemm_matches_oracle(dev, orc, m, n, k):
    rng = np.random.default_rng(m + n + k)
    A = (rng.standard_normal((m, n)) * 0.2).astype(np.float32)
    B = np.where(rng.random((n, k)) < 0.5, 1, -1).astype(np.int8)
    rc, pos, neg = orc.ternary_matrix_pack_from_float(A, m, n)
    rc2, bits = orc.binary_matrix_pack(B, n, k)
    assert rc == 0 and rc2 == 0
    if n % 128 == 0:
        rc, ref = orc.tbn_gemm(pos, neg, bits, m, n, k, (16, 8, 128, 16, 8))
        assert rc == 0
    else:
        # the reference's tiling needs n % 128 == 0; the GPU GEMM takes any
        # multiple of 64: brute force on the ternarized values
        t = (A > 0.1).astype(np.int64) - (A < -0.1).astype(np.int64)
        ref = t @ B.astype(np.int64)
    out = run_tbn_gemm(to_dev(pos), to_dev(neg), to_dev(bits), m, n, k)
    assert np.array_equal(out, ref)


def test_tbn_gemm_both_plane_bits_contribute_zero(dev, orc):
    # pos and neg both set (not produced by pack_from_float): the reference's
    # word formula gives +1 and -1, i.e. 0, for every weight sign
    m, n, k = 16, 128, 16
    rng = np.random.default_rng(9)
    pos = rng.integers(0, 256, m * n // 8, dtype=np.uint8)
    neg = rng.integers(0, 256, m * n // 8, dtype=np.uint8)
    bits = rng.integers(0, 256, k * n // 8, dtype=np.uint8)
    rc, ref = orc.tbn_gemm(pos, neg, bits, m, n, k, (16, 16, 128, 16, 16))
    assert rc == 0
    assert np.array_equal(run_tbn_gemm(to_dev(pos), to_dev(neg), to_dev(bits), m, n, k), ref)


def run_qlinear_tbn(A, packed, M, K, K_pad, N, N_pad, scale):
    out = empty((M, N), torch.float32)
    out.fill_(np.nan)
    dA = A if isinstance(A, torch.Tensor) else to_dev(A)
    tbn_hip.call("tbn_hip_qlinear_matmul_binary_tbn", P(dA), K, M, K, P(packed), K_pad, N, N_pad, scale, LO, HI,
                 P(out), N, None)
    return out


def gpu_pack_binary(binw, K, N):
    K_pad, N_pad = tbn_hip.padded_dims(K, N)
    packed = empty(N_pad * K_pad // 8, torch.uint8)
    tbn_hip.call("tbn_hip_pack_binary", P(to_dev(binw)), K, N, tbn_hip.LAYOUT_KN, K_pad, N_pad, P(packed), None)
    return packed, K_pad, N_pad


def test_qlinear_tbn_known_answer(dev):
    # test_quantized_operators.cpp:165-179 inputs through the reference's
    # operator: activations ternarize to sign, giving 1.4, -1.4, 1.4, -1.4
    A = np.array([[1.0, -2.0], [3.0, -4.0]], np.float32)
    packed, K_pad, N_pad = gpu_pack_binary(np.array([[1, 0], [0, 1]], np.uint8), 2, 2)
    out = host(run_qlinear_tbn(A, packed, 2, 2, K_pad, 2, N_pad, 0.7))
    assert out.reshape(-1).tolist() == (np.array([2, -2, 2, -2], np.float32) * np.float32(0.7)).tolist()


@pytest.mark.parametrize("M,K,N", [(16, 25, 6), (96, 200, 40), (256, 576, 128), (1040, 1000, 700)])
def test_qlinear_tbn_matches_oracle(dev, orc, M, K, N):
    rng = np.random.default_rng(M * 7 + N)
    A = special_matrix(M, K, seed=N)
    binw = (rng.random((K, N)) < 0.5).astype(np.uint8)
    packed, K_pad, N_pad = gpu_pack_binary(binw, K, N)
    out = host(run_qlinear_tbn(A, packed, M, K, K_pad, N, N_pad, 0.37))
    rc, ref = orc.qlinear_matmul_binary_tbn(A, binw, 0.37, TILING)
    assert rc == 0
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("M,N,ldo", [(2, 40, 40), (16, 300, 301), (300, 700, 700), (1040, 260, 264)])
def test_qlinear_tbn_leaves_memory_past_the_output_alone(dev, orc, M, N, ldo):
    """Ragged M (not a multiple of the 32-row fragments): the epilogue's
    stores for rows past M are dropped by the buffer range check, so 32 guard
    rows of NaN after the output (and the columns between N and ldo) keep
    their bits."""
    K = 330
    rng = np.random.default_rng(M + N)
    A = special_matrix(M, K, seed=M)
    binw = (rng.random((K, N)) < 0.5).astype(np.uint8)
    packed, K_pad, N_pad = gpu_pack_binary(binw, K, N)
    big = empty((M + 32, ldo), torch.float32)
    big.fill_(np.nan)
    guard = host(big).view(np.uint32).copy()
    tbn_hip.call("tbn_hip_qlinear_matmul_binary_tbn", P(to_dev(A)), K, M, K, P(packed), K_pad, N, N_pad, 0.5, LO,
                 HI, P(big), ldo, None)
    out = host(big)
    rc, ref = orc.qlinear_matmul_binary_tbn(A, binw, 0.5, TILING)
    assert rc == 0
    assert np.array_equal(out[:M, :N].view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(out[M:].view(np.uint32), guard[M:]), "rows past M were written"
    assert np.array_equal(out[:, N:].view(np.uint32), guard[:, N:]), "columns past N were written"


def test_qlinear_tbn_headline_shape_exact(dev):
    """4096^3: every element equals float(exact integer product) * scale
    (the integer product formed in float64 on the GPU, exact below 2^53)."""
    M = N = K = 4096
    g = torch.Generator(device="cuda:0")
    g.manual_seed(5)
    A = torch.randn((M, K), generator=g, device="cuda:0") * 0.3
    binw = (torch.rand((K, N), generator=g, device="cuda:0") < 0.5).to(torch.uint8)
    K_pad, N_pad = tbn_hip.padded_dims(K, N)
    packed = empty(N_pad * K_pad // 8, torch.uint8)
    tbn_hip.call("tbn_hip_pack_binary", P(binw), K, N, tbn_hip.LAYOUT_KN, K_pad, N_pad, P(packed), None)
    out = run_qlinear_tbn(A, packed, M, K, K_pad, N, N_pad, 0.25)
    t = torch.where(A < LO, -1.0, torch.where(A > HI, 1.0, 0.0)).to(torch.float64)
    w = binw.to(torch.float64) * 2.0 - 1.0
    ref = ((t @ w).to(torch.float32) * np.float32(0.25))
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_tbn_error_codes(dev):
    buf = empty(1024, torch.uint8)
    C = empty((4, 4), torch.int32)
    with pytest.raises(tbn_hip.TbnError) as e:
        tbn_hip.call("tbn_hip_tbn_gemm", P(buf), P(buf), P(buf), 4, 96, 4, P(C), None)
    assert e.value.code == tbn_hip.INVALID_ARGUMENT  # n % 64
    with pytest.raises(tbn_hip.TbnError) as e:
        tbn_hip.call("tbn_hip_qlinear_matmul_binary_tbn", P(buf), 4, 4, 4, P(buf), 96, 4, 8, 1.0, LO, HI, P(C), 4,
                     None)
    assert e.value.code == tbn_hip.INVALID_SHAPE  # K_pad % 64
    # empty problems are no-ops
    tbn_hip.call("tbn_hip_tbn_gemm", None, None, None, 0, 64, 4, None, None)


def test_runtime_qlinear_matmul_binary_tbn(dev, tbn, orc):
    """tbn::qlinear_matmul_binary_tbn (C++ runtime, host tensors in and out)
    is the reference operator bit for bit; the packed variant agrees."""
    rng = np.random.default_rng(12)
    M, K, N = 64, 300, 50
    A = special_matrix(M, K, seed=12)
    binw = (rng.random((K, N)) < 0.5).astype(np.uint8)
    out = tbn.qlinear_matmul_binary_tbn(tbn.Tensor(A), tbn.Tensor(binw, "binary"), 0.5).numpy()
    rc, ref = orc.qlinear_matmul_binary_tbn(A, binw, 0.5, TILING)
    assert rc == 0
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    w = tbn.pack_binary_weights(tbn.Tensor(binw, "binary"))
    out2 = tbn.qlinear_matmul_packed_tbn(tbn.Tensor(A), w, 0.5).numpy()
    assert np.array_equal(out2.view(np.uint32), ref.view(np.uint32))
    with pytest.raises(tbn.TBNError):
        tbn.qlinear_matmul_binary_tbn(tbn.Tensor(A), tbn.Tensor(np.zeros((K, N), np.float32)), 1.0)
