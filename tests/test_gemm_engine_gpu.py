"""The GeMM engine API (tbn::TernaryMatrix / BinaryMatrix / GemmEngine /
TilingParams / PackedBinaryWeights, qlinear_matmul_binary_blocked_packed and
_prepacked) through the _tbn module, written after the reference's own test
file GeMM/05-final/test_final.cpp: the golden 128x128 product under the four
tilings it uses (lines 23-70), its exception cases (lines 76-118; the host-only ones
also run without a GPU in tests/test_runtime_cpu.py).  Everything is integer or float(int) *
scale, so every comparison is bit for bit: against the golden vectors
(GeMM/05-final/matrices_to_test.hpp, C = sign(A @ B)), exact int64 products,
and the oracle (oracle/tbn_oracle.c, pinned by tests/test_oracle.py)."""
import pathlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = pathlib.Path(__file__).with_name("golden") / "gemm_golden.npz"
LO, HI = -0.1, 0.1
# the oracle's portable tiling, valid for every shape used here
ORACLE_TILING = (128, 256, 256, 16, 8)


@pytest.fixture(scope="module")
def golden():
    return dict(np.load(GOLDEN))


# GeMM/05-final/test_final.cpp:23-70: single block, default_128x128 (the
# "multiple blocks" case), small micro kernels, and the default argument.
TILINGS = {
    "single_block": (128, 128, 128, 64, 64),
    "multiple_blocks": None,
    "small_microkernels": (32, 32, 128, 16, 16),
    "default_params": "omit",
}


@pytest.mark.parametrize("name", list(TILINGS))
def test_engine_golden_128(dev, tbn, golden, name):
    A, B, C = golden["A128"], golden["B128"], golden["C128"]
    a = tbn.TernaryMatrix.pack(A, 128, 128)
    b = tbn.BinaryMatrix.pack(B, 128, 128)
    engine = tbn.GemmEngine()
    t = TILINGS[name]
    if t == "omit":
        out = engine.compute(a, b)
    elif t is None:
        out = engine.compute(a, b, tbn.TilingParams.default_128x128())
    else:
        out = engine.compute(a, b, tbn.TilingParams(*t))
    assert out.shape == (128, 128) and out.dtype == np.int32
    assert np.array_equal(np.sign(out), C)
    assert np.array_equal(out, A.astype(np.int64) @ B.astype(np.int64))
    assert engine.last_flops() == 128 * 128 * 128 * 2


def test_packers_match_oracle(dev, tbn, orc, golden):
    """The planes and bits are the reference's layouts, byte for byte."""
    A, B = golden["A128"], golden["B128"]
    a = tbn.TernaryMatrix.pack(A, 128, 128)
    rc, pos, neg = orc.ternary_matrix_pack_from_float(A.astype(np.float32), 128, 128)
    assert rc == 0
    assert np.array_equal(a.positive, pos) and np.array_equal(a.negative, neg)
    rc, bits = orc.binary_matrix_pack(B, 128, 128)
    assert rc == 0
    assert np.array_equal(tbn.BinaryMatrix.pack(B, 128, 128).bits, bits)
    rng = np.random.default_rng(5)
    F = (rng.standard_normal((40, 192)) * 0.2).astype(np.float32)
    F[0, :6] = [0.1, -0.1, np.nan, np.inf, -np.inf, -0.0]
    f = tbn.TernaryMatrix.pack_from_float(F, 40, 192, LO, HI)
    rc, pos, neg = orc.ternary_matrix_pack_from_float(F, 40, 192, LO, HI)
    assert (f.rows, f.cols) == (40, 192)
    assert np.array_equal(f.positive, pos) and np.array_equal(f.negative, neg)


@pytest.mark.parametrize("m,n,k", [(64, 256, 96), (256, 1024, 512), (32, 4096, 64)])
def test_engine_random_matches_oracle(dev, tbn, orc, m, n, k):
    rng = np.random.default_rng(m + n + k)
    A = rng.integers(-1, 2, size=(m, n)).astype(np.int8)
    B = np.where(rng.random((n, k)) < 0.5, 1, -1).astype(np.int8)
    out = tbn.GemmEngine().compute(tbn.TernaryMatrix.pack(A, m, n), tbn.BinaryMatrix.pack(B, n, k),
                                   tbn.TilingParams(64, 64, 128, 32, 32))
    rc, pos, neg = orc.ternary_matrix_pack_from_float(A.astype(np.float32), m, n)
    rc2, bits = orc.binary_matrix_pack(B, n, k)
    rc3, ref = orc.tbn_gemm(pos, neg, bits, m, n, k, (64, 64, 128, 32, 32))
    assert rc == rc2 == rc3 == 0
    assert np.array_equal(out, ref)
    assert np.array_equal(out, A.astype(np.int64) @ B.astype(np.int64))


def test_engine_exceptions(dev, tbn, golden):
    """test_final.cpp:76-118: invalid ternary / binary values, dimensions and
    tiling throw std::invalid_argument (ValueError in Python)."""
    bad = np.zeros(8 * 64, np.int8); bad[0] = 2
    with pytest.raises(ValueError, match="values must be -1, 0, or \\+1"):
        tbn.TernaryMatrix.pack(bad, 8, 64)
    bad = np.ones(64 * 8, np.int8); bad[0] = 0
    with pytest.raises(ValueError, match="values must be -1 or \\+1"):
        tbn.BinaryMatrix.pack(bad, 64, 8)
    with pytest.raises(ValueError, match="rows must be multiple of 8"):
        tbn.TernaryMatrix.pack(np.zeros(100, np.int8), 10, 10)
    with pytest.raises(ValueError, match="cols must be multiple of 64"):
        tbn.TernaryMatrix.pack(np.zeros(8 * 60, np.int8), 8, 60)
    with pytest.raises(ValueError, match="data size"):
        tbn.TernaryMatrix.pack(np.zeros(8 * 64 - 1, np.int8), 8, 64)
    with pytest.raises(ValueError, match="rows must be multiple of 64"):
        tbn.BinaryMatrix.pack(np.ones(32 * 8, np.int8), 32, 8)
    with pytest.raises(ValueError, match="cols must be multiple of 8"):
        tbn.BinaryMatrix.pack(np.ones(64 * 6, np.int8), 64, 6)
    a = tbn.TernaryMatrix.pack(golden["A128"], 128, 128)
    b = tbn.BinaryMatrix.pack(golden["B128"], 128, 128)
    engine = tbn.GemmEngine()
    with pytest.raises(ValueError, match="kblk must be multiple of 128"):
        engine.compute(a, b, tbn.TilingParams(64, 64, 64, 32, 32))
    with pytest.raises(ValueError, match="m must be multiple of mmk"):
        engine.compute(a, b, tbn.TilingParams(64, 64, 128, 48, 32))
    with pytest.raises(ValueError, match="k must be multiple of nmk"):
        engine.compute(a, b, tbn.TilingParams(64, 64, 128, 32, 48))
    a64 = tbn.TernaryMatrix.pack(np.zeros(64 * 64, np.int8), 64, 64)
    b64 = tbn.BinaryMatrix.pack(np.ones(64 * 64, np.int8), 64, 64)
    with pytest.raises(ValueError, match="n must be multiple of 128"):
        engine.compute(a64, b64)
    b256 = tbn.BinaryMatrix.pack(np.ones(256 * 64, np.int8), 256, 64)
    with pytest.raises(ValueError, match="A cols"):
        engine.compute(a, b256)


def test_packed_binary_weights_from_int8(dev, tbn, orc):
    """GeMM.cpp:369-398: rows padded to 64, columns to 8, with +1."""
    rng = np.random.default_rng(9)
    W = np.where(rng.random((100, 13)) < 0.5, 1, -1).astype(np.int8)
    p = tbn.PackedBinaryWeights.from_int8(W, 100, 13)
    assert p.valid() and (p.b_packed.rows, p.b_packed.cols) == (128, 16)
    assert (p.original_m, p.original_n, p.original_k) == (100, 13, 100)
    padded = np.ones((128, 16), np.int8); padded[:100, :13] = W
    rc, bits = orc.binary_matrix_pack(padded, 128, 16)
    assert rc == 0 and np.array_equal(p.b_packed.bits, bits)


@pytest.mark.parametrize("M,K,N", [(1, 128, 8), (37, 256, 100), (256, 1024, 1000), (512, 4096, 512)])
@pytest.mark.parametrize("on_device", [False, True])
def test_blocked_packed_matches_oracle(dev, tbn, orc, M, K, N, on_device):
    """quantized_gemm_neon.cpp:249-309 on the oracle's qlinear_matmul_binary
    (mode TBN) with the same weights."""
    rng = np.random.default_rng(M + K + N)
    A = (rng.standard_normal((M, K)) * 0.2).astype(np.float32)
    A.reshape(-1)[:4] = [0.1, -0.1, np.nan, -0.0]
    W = np.where(rng.random((K, N)) < 0.5, 1, -1).astype(np.int8)
    p = tbn.PackedBinaryWeights.from_int8(W, K, N)
    params = tbn.TilingParams(16, 8, 128, 16, 8)
    a = tbn.Tensor(A, "", "hip") if on_device else A
    out = tbn.qlinear_matmul_binary_blocked_packed(a, p.b_packed, N, 0.75, params, LO, HI)
    assert out.device == ("hip" if on_device else "cpu")
    rc, ref = orc.qlinear_matmul_binary_tbn(A, (W == 1).astype(np.uint8), 0.75, ORACLE_TILING)
    assert rc == 0
    assert np.array_equal(out.numpy(), ref)


def test_blocked_packed_checks_tiling_like_the_reference(dev, tbn):
    """The reference runs the engine on ceil16(M) rows: M = 40 pads to 48,
    which default_128x128 (mmk = 32) rejects."""
    p = tbn.PackedBinaryWeights.from_int8(np.ones((128, 8), np.int8), 128, 8)
    A = np.zeros((40, 128), np.float32)
    with pytest.raises(ValueError, match="m must be multiple of mmk"):
        tbn.qlinear_matmul_binary_blocked_packed(A, p.b_packed, 8)
    out = tbn.qlinear_matmul_binary_blocked_packed(A, p.b_packed, 8, 1.0, tbn.TilingParams(16, 8, 128, 16, 8))
    assert out.numpy().shape == (40, 8) and not out.numpy().any()


@pytest.mark.parametrize("m_orig,n_orig", [(128, 128), (100, 77), (1, 1)])
def test_blocked_prepacked(dev, tbn, golden, m_orig, n_orig):
    """quantized_gemm_neon.cpp:314-350: float(C) * scale of the leading
    m_orig x n_orig block."""
    A, B = golden["A128"], golden["B128"]
    a = tbn.TernaryMatrix.pack(A, 128, 128)
    b = tbn.BinaryMatrix.pack(B, 128, 128)
    out = tbn.qlinear_matmul_binary_blocked_prepacked(a, b, m_orig, n_orig, 0.5)
    assert out.device == "cpu"
    ref = (A.astype(np.int64) @ B.astype(np.int64))[:m_orig, :n_orig].astype(np.float32) * np.float32(0.5)
    assert np.array_equal(out.numpy(), ref)
