"""TBN-mode reference arithmetic for the tests, built from the oracle's
pinned functions (oracle/tbn_oracle.c: im2col_ternary_packed and the
ternarization, pinned by tests/test_oracle.py on the reference's golden
vectors) plus exact integer products and plain float32 epilogues.

The reference Session's quantized convolution (model.hpp:482-557; conv2d_
binary, conv2d.cpp:220-316) forms the integer C = t(im2col(x)) . sign(w)
exactly, then float(C) + b, or (float(C) + b) * s on its cached path; its
quantized Gemm (model.hpp:835-870) forms float(C) * alpha then r += beta * c,
which the AArch64 compilers the reference targets contract into one fused
multiply-add (numpy has no fma: the fused step is evaluated exactly with
Python's fractions and rounded once to float32)."""
from fractions import Fraction

import numpy as np

LO, HI = -0.1, 0.1


def conv_out_hw(H, W, kh, kw, stride, pad, dil):
    OH = (H + 2 * pad[0] - dil[0] * (kh - 1) - 1) // stride[0] + 1
    OW = (W + 2 * pad[1] - dil[1] * (kw - 1) - 1) // stride[1] + 1
    return OH, OW


def ternary_im2col(orc, x, kh, kw, stride, pad, dil, lo=LO, hi=HI):
    """The reference's ternarized im2col matrix as int8 [N*OH*OW, C*kh*kw]
    (column (c*kh + r)*kw + s), decoded from the oracle's bit planes."""
    N, C, H, W = x.shape
    OH, OW = conv_out_hw(H, W, kh, kw, stride, pad, dil)
    Q, K = N * OH * OW, C * kh * kw
    m_pad, k_pad = (Q + 15) // 16 * 16, (K + 127) // 128 * 128
    rc, pos, neg = orc.im2col_ternary_packed(x, kh, kw, stride, pad, dil, m_pad, k_pad, lo, hi)
    assert rc == 0
    p = np.unpackbits(pos.reshape(m_pad, k_pad // 8), axis=1, bitorder="little")[:Q, :K]
    m = np.unpackbits(neg.reshape(m_pad, k_pad // 8), axis=1, bitorder="little")[:Q, :K]
    assert not np.any(p & m)
    return p.astype(np.int8) - m.astype(np.int8), OH, OW


def tbn_conv_int(orc, x, wsign, stride=(1, 1), pad=(0, 0), dil=(1, 1), lo=LO, hi=HI):
    """Exact integer C [N, M, OH, OW] of the TBN conv: ternarized taps times
    the +-1 weights wsign [M, C, kh, kw]."""
    M, C, kh, kw = wsign.shape
    t, OH, OW = ternary_im2col(orc, x, kh, kw, stride, pad, dil, lo, hi)
    # integer products summed in float64: exact (|C| <= K < 2^53)
    acc = t.astype(np.float64) @ wsign.reshape(M, -1).astype(np.float64).T
    return acc.reshape(x.shape[0], OH, OW, M).transpose(0, 3, 1, 2).astype(np.int64)


def tbn_conv_epilogue(C, scale=None, alpha=1.0, bias=None, residual=None, bias_then_scale=False, relu=False,
                      pool=False):
    """float32 epilogue, one rounding per operation in the reference's order."""
    M = C.shape[1]
    v = C.astype(np.float32)
    mult = np.float32(alpha) * (np.ones(M, np.float32) if scale is None else np.asarray(scale, np.float32))
    b = np.zeros(M, np.float32) if bias is None else np.asarray(bias, np.float32)
    mult, b = mult[None, :, None, None], b[None, :, None, None]
    if bias_then_scale:
        v = (v + b) * mult
    else:
        v = v * mult + b  # numpy rounds the product, then the sum
    if residual is not None:
        v = v + np.asarray(residual, np.float32)
    if relu:
        v = np.where(v > 0, v, np.float32(0))
    if pool:
        N, M, OH, OW = v.shape
        v = v[:, :, :OH // 2 * 2, :OW // 2 * 2].reshape(N, M, OH // 2, 2, OW // 2, 2).max(axis=(3, 5))
    return v.astype(np.float32)


def fma32(a, b, c):
    """float32 fma(a, b, c) elementwise: a*b + c exact, rounded once to
    float32 (round to nearest, ties to even)."""
    a, b, c = np.broadcast_arrays(np.asarray(a, np.float32), np.asarray(b, np.float32), np.asarray(c, np.float32))
    out = np.empty(a.shape, np.float32)
    fa, fb, fc, fo = a.reshape(-1), b.reshape(-1), c.reshape(-1), out.reshape(-1)
    for i in range(fa.size):
        x, y, z = float(fa[i]), float(fb[i]), float(fc[i])
        if not (np.isfinite(x) and np.isfinite(y) and np.isfinite(z)):
            fo[i] = np.float32(x * y + z)
            continue
        fo[i] = _round_f32(Fraction(x) * Fraction(y) + Fraction(z))
    return out


def _round_f32(q):
    """The float32 nearest to the rational q (ties to even)."""
    if q == 0:
        return np.float32(0.0)
    f = np.float32(float(q))  # within one float32 ulp of q (a double rounding at most)
    for cand in (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))):
        if not np.isfinite(cand):
            continue
        lo_n = np.nextafter(cand, np.float32(-np.inf))
        hi_n = np.nextafter(cand, np.float32(np.inf))
        c = Fraction(float(cand))
        lo_m = (c + Fraction(float(lo_n))) / 2 if np.isfinite(lo_n) else None
        hi_m = (c + Fraction(float(hi_n))) / 2 if np.isfinite(hi_n) else None
        above = lo_m is None or q > lo_m or (q == lo_m and (cand.view(np.uint32) & 1) == 0)
        below = hi_m is None or q < hi_m or (q == hi_m and (cand.view(np.uint32) & 1) == 0)
        if above and below:
            return cand
    return f


def tbn_gemm_session(orc, A, sign, alpha=1.0, cin=None, beta=0.0, lo=LO, hi=HI):
    """The reference Session's quantized Gemm on the ternarized A [M, K]:
    float(C) * alpha, then fma(beta, cin, .) where cin is given and beta != 0.
    C exact from the oracle's ternarization (pack_from_float)."""
    A = np.asarray(A, np.float32)
    M, K = A.shape
    rows, cols = (M + 7) // 8 * 8, (K + 63) // 64 * 64
    rc, pos, neg = orc.ternary_matrix_pack_from_float(A, rows, cols, lo, hi)
    assert rc == 0
    p = np.unpackbits(pos.reshape(rows, cols // 8), axis=1, bitorder="little")[:M, :K]
    m = np.unpackbits(neg.reshape(rows, cols // 8), axis=1, bitorder="little")[:M, :K]
    t = p.astype(np.float64) - m.astype(np.float64)
    C = (t @ np.asarray(sign, np.float64)).astype(np.int64)
    out = C.astype(np.float32) * np.float32(alpha)
    if cin is not None and beta != 0.0:
        c = np.asarray(cin, np.float32)
        c = np.broadcast_to(c.reshape(1, -1) if c.ndim == 1 else c, out.shape)
        out = fma32(np.float32(beta), c, out)
    return out.astype(np.float32)
