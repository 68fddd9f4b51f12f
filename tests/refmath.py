"""Independent numpy formulations used to pin the oracle (and the GPU path).

Nothing here shares code with oracle/tbn_oracle.c: the packed layouts are
built with np.packbits / vectorised shifts from their closed-form definitions,
and the arithmetic references are float64 matrix products.
"""
import numpy as np


def np_pack_binary(binw, K, N, layout, K_pad, N_pad):
    """BinaryMatrix bits from the closed form: column n, bit k set iff -1."""
    w = np.asarray(binw, np.uint8).reshape((K, N) if layout == 0 else (N, K))
    neg = np.zeros((N_pad, K_pad), np.uint8)
    neg[:N, :K] = (w.T if layout == 0 else w) != 1
    return np.packbits(neg, axis=1, bitorder="little").reshape(-1)


def np_unpack_binary(packed, K, N, K_pad):
    bits = np.unpackbits(np.asarray(packed, np.uint8).reshape(-1, K_pad // 8), axis=1, bitorder="little")
    return np.where(bits[:N, :K] == 1, -1, 1).astype(np.int8).T  # [K, N]


def ternary_codes(t):
    t = np.asarray(t, np.int8)
    return np.where(t == -1, 0, np.where(t == 1, 2, 1)).astype(np.uint8)


def np_ternary_pack2(t):
    c = ternary_codes(np.asarray(t).reshape(-1))
    n = c.size
    c = np.concatenate([c, np.zeros((-n) % 4, np.uint8)])  # unused slots of a fresh buffer stay 00
    c = c.reshape(-1, 4).astype(np.uint32)
    return (c[:, 0] | (c[:, 1] << 2) | (c[:, 2] << 4) | (c[:, 3] << 6)).astype(np.uint8)


def np_ternary_unpack2(packed, n):
    p = np.asarray(packed, np.uint8).astype(np.uint32)
    codes = np.stack([(p >> s) & 3 for s in (0, 2, 4, 6)], axis=1).reshape(-1)[:n]
    return np.where(codes == 0, -1, np.where(codes == 2, 1, 0)).astype(np.int8)


def np_pack_ternary(t, K, N, layout, K_pad, N_pad):
    w = np.asarray(t, np.int8).reshape((K, N) if layout == 0 else (N, K))
    full = np.zeros((N_pad, K_pad), np.int8)
    full[:N, :K] = w.T if layout == 0 else w
    return np_ternary_pack2(full.reshape(-1))


def np_unpack_ternary(packed, K, N, K_pad):
    n_pad = len(packed) * 4 // K_pad
    vals = np_ternary_unpack2(packed, n_pad * K_pad).reshape(n_pad, K_pad)
    return vals[:N, :K].T  # [K, N]


def f64_gemm(A, W, scale=None, alpha=1.0, bias=None, relu=False, bias_then_scale=False):
    """(A @ W) * alpha*scale + bias in float64, W given as +-1/0 [K, N]."""
    acc = np.asarray(A, np.float64) @ np.asarray(W, np.float64)
    # the ABI forms the per-column multiplier alpha*s[n] in fp32
    s = np.ones(W.shape[1], np.float32) if scale is None else np.asarray(scale, np.float32)
    mult = (np.float32(alpha) * s).astype(np.float64)
    b = 0.0 if bias is None else np.asarray(bias, np.float64)
    out = (acc + b) * mult if bias_then_scale else acc * mult + b
    return np.maximum(out, 0.0) if relu else out


def np_im2col(x, kh, kw, stride=(1, 1), pad=(0, 0), dil=(1, 1)):
    """[N*OH*OW, C*kh*kw] im2col with zero padding (float64)."""
    x = np.asarray(x, np.float64)
    N, C, H, W = x.shape
    OH = (H + 2 * pad[0] - dil[0] * (kh - 1) - 1) // stride[0] + 1
    OW = (W + 2 * pad[1] - dil[1] * (kw - 1) - 1) // stride[1] + 1
    xp = np.zeros((N, C, H + 2 * pad[0], W + 2 * pad[1]))
    xp[:, :, pad[0]:pad[0] + H, pad[1]:pad[1] + W] = x
    cols = np.empty((N, OH, OW, C, kh, kw))
    for r in range(kh):
        for s in range(kw):
            h0, w0 = r * dil[0], s * dil[1]
            patch = xp[:, :, h0:h0 + stride[0] * (OH - 1) + 1:stride[0], w0:w0 + stride[1] * (OW - 1) + 1:stride[1]]
            cols[:, :, :, :, r, s] = patch.transpose(0, 2, 3, 1)
    return cols.reshape(N * OH * OW, C * kh * kw), OH, OW


def f64_conv(x, w, bias=None, stride=(1, 1), pad=(0, 0), dil=(1, 1)):
    w = np.asarray(w, np.float64)
    M, C, kh, kw = w.shape
    cols, OH, OW = np_im2col(x, kh, kw, stride, pad, dil)
    y = cols @ w.reshape(M, -1).T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)
    N = np.asarray(x).shape[0]
    return y.reshape(N, OH, OW, M).transpose(0, 3, 1, 2)


def np_maxpool(x, k, s, p=(0, 0), ceil_mode=False):
    x = np.asarray(x, np.float32)
    N, C, H, W = x.shape
    if ceil_mode:
        OH = (H + 2 * p[0] - k[0] + s[0] - 1) // s[0] + 1
        OW = (W + 2 * p[1] - k[1] + s[1] - 1) // s[1] + 1
    else:
        OH = (H + 2 * p[0] - k[0]) // s[0] + 1
        OW = (W + 2 * p[1] - k[1]) // s[1] + 1
    xp = np.full((N, C, max(H + 2 * p[0], OH * s[0] + k[0]), max(W + 2 * p[1], OW * s[1] + k[1])), -np.inf, np.float32)
    xp[:, :, p[0]:p[0] + H, p[1]:p[1] + W] = x
    y = np.full((N, C, OH, OW), -np.inf, np.float32)
    for r in range(k[0]):
        for c in range(k[1]):
            y = np.maximum(y, xp[:, :, r:r + s[0] * (OH - 1) + 1:s[0], c:c + s[1] * (OW - 1) + 1:s[1]])
    return y


def seq_sum_f32(values):
    """Left-to-right float32 sum (the order of the reference's scalar loops)."""
    acc = np.float32(0.0)
    for v in np.asarray(values, np.float32).reshape(-1):
        acc = np.float32(acc + v)
    return acc


def rel_l2(x, ref):
    x = np.asarray(x, np.float64); ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(x - ref) / (den if den > 0 else 1.0))


def assert_within_tolerance(out, ref, K, x_absmax, rel=1e-5):
    """north_star tolerance: rel-L2 <= 1e-5 and max-abs <= 1e-4*sqrt(K)*max|x|."""
    out = np.asarray(out, np.float64); ref = np.asarray(ref, np.float64)
    assert out.shape == ref.shape, (out.shape, ref.shape)
    r = rel_l2(out, ref)
    m = float(np.max(np.abs(out - ref))) if out.size else 0.0
    bound = 1e-4 * np.sqrt(max(K, 1)) * max(float(x_absmax), 1e-30)
    assert r <= rel, f"rel-L2 {r:.3e} > {rel:.0e}"
    assert m <= bound, f"max-abs {m:.3e} > {bound:.3e}"
    return r, m
