"""numpy wrappers over oracle/libtbn_oracle.so (the CPU oracle).

Test infrastructure only: used by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker or the timed CPU baseline.
"""
import ctypes
import pathlib
import subprocess

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[1]
LIB_PATH = ROOT / "oracle" / "libtbn_oracle.so"

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            subprocess.run(["make", "-C", str(ROOT / "oracle")], check=True, capture_output=True)
        _lib = ctypes.CDLL(str(LIB_PATH))
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


I64 = ctypes.c_int64
U32 = ctypes.c_uint32
F32 = ctypes.c_float


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


# ---- quantization ----------------------------------------------------------

def quantize_to_binary_f32(w, thr=0.0):
    w = _c(w, np.float32); out = np.empty(w.shape, np.uint8)
    lib().tbo_quantize_to_binary_f32(_p(w), I64(w.size), F32(thr), _p(out)); return out


def quantize_to_binary_i8(w):
    w = _c(w, np.int8); out = np.empty(w.shape, np.uint8)
    lib().tbo_quantize_to_binary_i8(_p(w), I64(w.size), _p(out)); return out


def quantize_to_ternary_f32(w, lo=-0.1, hi=0.1):
    w = _c(w, np.float32); out = np.empty(w.shape, np.int8)
    lib().tbo_quantize_to_ternary_f32(_p(w), I64(w.size), F32(lo), F32(hi), _p(out)); return out


def sign_ge0_f32(w):
    w = _c(w, np.float32); out = np.empty(w.shape, np.uint8)
    lib().tbo_sign_ge0_f32(_p(w), I64(w.size), _p(out)); return out


def channel_mean_abs(w):
    w = _c(w, np.float32); ch = w.shape[0]; per = w.size // ch
    out = np.empty(ch, np.float32)
    lib().tbo_channel_mean_abs(_p(w), I64(ch), I64(per), _p(out)); return out


def already_binary(w, scale):
    w = _c(w, np.float32); scale = _c(scale, np.float32); ch = w.shape[0]
    lib().tbo_already_binary.restype = ctypes.c_int
    return bool(lib().tbo_already_binary(_p(w), I64(ch), I64(w.size // ch), _p(scale)))


# ---- packing -------------------------------------------------------------------

def binary_matrix_pack(data, rows, cols):
    data = _c(data, np.int8); bits = np.zeros(cols * rows // 8, np.uint8)
    rc = lib().tbo_binary_matrix_pack(_p(data), U32(rows), U32(cols), _p(bits))
    return rc, bits


def pack_binary(binw, K, N, layout, K_pad, N_pad):
    """BINARY bytes in layout 0 (KN) or 1 (NK) -> BinaryMatrix bits."""
    binw = _c(binw, np.uint8); out = np.zeros(N_pad * K_pad // 8, np.uint8)
    fn = lib().tbo_pack_binary_kn if layout == 0 else lib().tbo_pack_binary_nk
    rc = fn(_p(binw), I64(K if layout == 0 else N), I64(N if layout == 0 else K), I64(K_pad), I64(N_pad), _p(out))
    assert rc == 0, rc
    return out


def ternary_pack2(t):
    t = _c(t, np.int8); out = np.zeros((t.size + 3) // 4, np.uint8)
    lib().tbo_ternary_pack2(_p(t), I64(t.size), _p(out)); return out


def ternary_get2(packed, n):
    packed = _c(packed, np.uint8)
    lib().tbo_ternary_get2.restype = ctypes.c_int8
    return np.array([lib().tbo_ternary_get2(_p(packed), I64(i)) for i in range(n)], np.int8)


def pack_ternary(t, K, N, layout, K_pad, N_pad):
    t = _c(t, np.int8); out = np.zeros(N_pad * K_pad // 4, np.uint8)
    fn = lib().tbo_pack_ternary_kn if layout == 0 else lib().tbo_pack_ternary_nk
    rc = fn(_p(t), I64(K if layout == 0 else N), I64(N if layout == 0 else K), I64(K_pad), I64(N_pad), _p(out))
    assert rc == 0, rc
    return out


# ---- mode F32 ---------------------------------------------------------------------

def _gemm(fn, A, packed, K_pad, N, scale, alpha, bias, relu, out_dtype):
    A = _c(A, np.float32); M, K = A.shape
    C = np.empty((M, N), out_dtype)
    fn(_p(A), I64(K), I64(M), I64(K), _p(_c(packed, np.uint8)), I64(K_pad), I64(N),
       _p(_c(scale, np.float32)), F32(alpha), _p(_c(bias, np.float32)), ctypes.c_int(int(relu)),
       _p(C), I64(N))
    return C


def gemm_f32_binary(A, packed, K_pad, N, scale=None, alpha=1.0, bias=None, relu=False):
    return _gemm(lib().tbo_gemm_f32_binary, A, packed, K_pad, N, scale, alpha, bias, relu, np.float32)


def gemm_f64_binary(A, packed, K_pad, N, scale=None, alpha=1.0, bias=None, relu=False):
    return _gemm(lib().tbo_gemm_f64_binary, A, packed, K_pad, N, scale, alpha, bias, relu, np.float64)


def gemm_f32_ternary(A, packed, K_pad, N, scale=None, alpha=1.0, bias=None, relu=False):
    return _gemm(lib().tbo_gemm_f32_ternary, A, packed, K_pad, N, scale, alpha, bias, relu, np.float32)


def gemm_f64_ternary(A, packed, K_pad, N, scale=None, alpha=1.0, bias=None, relu=False):
    return _gemm(lib().tbo_gemm_f64_ternary, A, packed, K_pad, N, scale, alpha, bias, relu, np.float64)


def qlinear_matmul_binary_naive(A, binw, scale):
    A = _c(A, np.float32); binw = _c(binw, np.uint8); M, K = A.shape; N = binw.shape[1]
    out = np.empty((M, N), np.float32)
    lib().tbo_qlinear_matmul_binary_naive(_p(A), I64(M), I64(K), _p(binw), I64(N), F32(scale), _p(out))
    return out


# ---- fp32 operators ---------------------------------------------------------------

def _conv(fn, x, w, bias, stride, pad, dil, dtype):
    x = _c(x, np.float32); w = _c(w, np.float32)
    N, C, H, W = x.shape; M, _, kh, kw = w.shape
    OH = (H + 2 * pad[0] - dil[0] * (kh - 1) - 1) // stride[0] + 1
    OW = (W + 2 * pad[1] - dil[1] * (kw - 1) - 1) // stride[1] + 1
    y = np.empty((N, M, OH, OW), dtype)
    rc = fn(_p(x), I64(N), I64(C), I64(H), I64(W), _p(w), I64(M), I64(kh), I64(kw),
            _p(_c(bias, np.float32)), I64(stride[0]), I64(stride[1]), I64(pad[0]), I64(pad[1]),
            I64(dil[0]), I64(dil[1]), _p(y))
    assert rc == 0, rc
    return y


def conv2d_f32(x, w, bias=None, stride=(1, 1), pad=(0, 0), dil=(1, 1)):
    return _conv(lib().tbo_conv2d_f32, x, w, bias, stride, pad, dil, np.float32)


def conv2d_f64(x, w, bias=None, stride=(1, 1), pad=(0, 0), dil=(1, 1)):
    return _conv(lib().tbo_conv2d_f64, x, w, bias, stride, pad, dil, np.float64)


def maxpool2d(x, k, s, p=(0, 0), d=(1, 1), ceil_mode=False):
    x = _c(x, np.float32); N, C, H, W = x.shape
    hw = np.zeros(2, np.int64)
    args = [I64(N), I64(C), I64(H), I64(W), I64(k[0]), I64(k[1]), I64(s[0]), I64(s[1]),
            I64(p[0]), I64(p[1]), I64(d[0]), I64(d[1]), ctypes.c_int(int(ceil_mode))]
    lib().tbo_maxpool2d(_p(x), *args, None, _p(hw))
    y = np.empty((N, C, int(hw[0]), int(hw[1])), np.float32)
    lib().tbo_maxpool2d(_p(x), *args, _p(y), _p(hw))
    return y


def avgpool2d(x, k, s, p=(0, 0), d=(1, 1), ceil_mode=False, count_include_pad=False):
    x = _c(x, np.float32); N, C, H, W = x.shape
    hw = np.zeros(2, np.int64)
    args = [I64(N), I64(C), I64(H), I64(W), I64(k[0]), I64(k[1]), I64(s[0]), I64(s[1]),
            I64(p[0]), I64(p[1]), I64(d[0]), I64(d[1]), ctypes.c_int(int(ceil_mode)),
            ctypes.c_int(int(count_include_pad))]
    lib().tbo_avgpool2d(_p(x), *args, None, _p(hw))
    y = np.empty((N, C, int(hw[0]), int(hw[1])), np.float32)
    lib().tbo_avgpool2d(_p(x), *args, _p(y), _p(hw))
    return y


def global_maxpool2d(x):
    x = _c(x, np.float32); N, C, H, W = x.shape
    y = np.empty((N, C), np.float32)
    lib().tbo_global_maxpool2d(_p(x), I64(N), I64(C), I64(H), I64(W), _p(y)); return y


def global_avgpool2d(x):
    x = _c(x, np.float32); N, C, H, W = x.shape
    y = np.empty((N, C), np.float32)
    lib().tbo_global_avgpool2d(_p(x), I64(N), I64(C), I64(H), I64(W), _p(y)); return y


def gemm_f32_blocked(A, B, Cin=None, alpha=1.0, beta=0.0, transA=False, transB=False):
    A = _c(A, np.float32); B = _c(B, np.float32)
    M = A.shape[1] if transA else A.shape[0]; K = A.shape[0] if transA else A.shape[1]
    N = B.shape[0] if transB else B.shape[1]
    out = np.empty((M, N), np.float32)
    cin = _c(Cin, np.float32)
    lib().tbo_gemm_f32_blocked(_p(A), _p(B), _p(cin), ctypes.c_int(int(cin is not None and cin.ndim == 1)),
                               I64(M), I64(K), I64(N), F32(alpha), F32(beta),
                               ctypes.c_int(int(transA)), ctypes.c_int(int(transB)), _p(out))
    return out


# ---- mode TBN -----------------------------------------------------------------------

def ternary_matrix_pack_from_float(A, rows, cols, lo=-0.1, hi=0.1):
    A = _c(A, np.float32); M, K = A.shape
    pos = np.zeros(rows * cols // 8, np.uint8); neg = np.zeros_like(pos)
    rc = lib().tbo_ternary_matrix_pack_from_float(_p(A), I64(K), I64(M), I64(K), U32(rows), U32(cols),
                                                  F32(lo), F32(hi), _p(pos), _p(neg))
    return rc, pos, neg


def tbn_gemm(pos, neg, bits, m, n, k, tiling=(64, 64, 128, 32, 32)):
    C = np.zeros((m, k), np.int32)
    rc = lib().tbo_tbn_gemm(_p(_c(pos, np.uint8)), _p(_c(neg, np.uint8)), _p(_c(bits, np.uint8)),
                            U32(m), U32(n), U32(k), *[U32(t) for t in tiling], _p(C))
    return rc, C


def qlinear_matmul_binary_tbn(A, binw, scale, tiling=(64, 64, 128, 32, 32)):
    A = _c(A, np.float32); binw = _c(binw, np.uint8); M, K = A.shape; N = binw.shape[1]
    out = np.empty((M, N), np.float32)
    rc = lib().tbo_qlinear_matmul_binary_tbn(_p(A), I64(M), I64(K), _p(binw), I64(N), F32(scale),
                                             *[U32(t) for t in tiling], _p(out))
    return rc, out


def im2col_ternary_packed(x, kh, kw, stride, pad, dil, m_pad, k_pad, lo=-0.1, hi=0.1):
    x = _c(x, np.float32); N, C, H, W = x.shape
    pos = np.zeros(m_pad * k_pad // 8, np.uint8); neg = np.zeros_like(pos)
    rc = lib().tbo_im2col_ternary_packed(_p(x), I64(N), I64(C), I64(H), I64(W), I64(kh), I64(kw),
                                         I64(stride[0]), I64(stride[1]), I64(pad[0]), I64(pad[1]),
                                         I64(dil[0]), I64(dil[1]), U32(m_pad), U32(k_pad), F32(lo), F32(hi),
                                         _p(pos), _p(neg))
    return rc, pos, neg
