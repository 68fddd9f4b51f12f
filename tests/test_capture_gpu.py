"""No allocation is recorded into a captured graph.

The calls that need the library's stream workspace -- the reference-layout
conv (it re-orders its weights there), a conv on pre-packed weights that
splits K, and a float x binary GEMM that splits K (their partial sums and
tile counters) -- return TBN_NOT_IMPLEMENTED while their stream captures,
before they record anything.  The capture is ended and its graph discarded;
no graph is launched.  The same calls then run eagerly and give the same bits
as before the capture."""
import ctypes

import numpy as np
import pytest
import torch

import tbn_hip
from gpu_util import P, empty, host, to_dev

pytestmark = pytest.mark.gpu


def _pack_nk(wbits, M, K):
    K_pad, N_pad = tbn_hip.padded_dims(K, M)
    packed = empty(N_pad * K_pad // 8, torch.uint8)
    tbn_hip.call("tbn_hip_pack_binary", P(to_dev(wbits)), K, M, tbn_hip.LAYOUT_NK, K_pad, N_pad, P(packed), None)
    return packed, K_pad, N_pad


def test_capture_refuses_workspace_users(dev):
    rng = np.random.default_rng(77)
    # reference-layout conv (weights re-ordered per call)
    d1 = tbn_hip.conv_desc(2, 64, 14, 14, 128, 3, 3, ph=1, pw=1)
    x1 = to_dev(rng.standard_normal((2, 64, 14, 14)).astype(np.float32))
    w1, K1_pad, N1_pad = _pack_nk((rng.random((128, 576)) < 0.5).astype(np.uint8), 128, 576)
    y1 = empty((2, 128, 14, 14), torch.float32)
    # conv on conv-layout weights whose geometry splits K (512 channels, 7 x 7)
    d2 = tbn_hip.conv_desc(2, 512, 7, 7, 64, 3, 3, ph=1, pw=1)
    x2 = to_dev(rng.standard_normal((2, 512, 7, 7)).astype(np.float32))
    w2, K2_pad, N2_pad = _pack_nk((rng.random((64, 4608)) < 0.5).astype(np.uint8), 64, 4608)
    nbytes = ctypes.c_int64(0)
    tbn_hip.call("tbn_hip_conv_weights_bytes", tbn_hip.WEIGHTS_BINARY, d2, ctypes.byref(nbytes))
    cw2 = empty(nbytes.value, torch.uint8)
    tbn_hip.call("tbn_hip_pack_conv_weights", tbn_hip.WEIGHTS_BINARY, P(w2), K2_pad, N2_pad, d2, P(cw2), None)
    y2 = empty((2, 64, 7, 7), torch.float32)
    # GEMM forced to split K over 5 blocks per 64 x 128 tile
    M, K, N = 300, 1100, 700
    A = to_dev(rng.standard_normal((M, K)).astype(np.float32))
    wg, Kg_pad, Ng_pad = _pack_nk((rng.random((N, K)) < 0.5).astype(np.uint8), N, K)
    C = empty((M, N), torch.float32)

    def conv_ref_layout(stream):
        tbn_hip.call("tbn_hip_conv2d_f32_binary", P(x1), d1, P(w1), K1_pad, N1_pad, None, 1.0, None,
                     tbn_hip.EPI_RELU, P(y1), stream)

    def conv_split(stream):
        with tbn_hip.tuning(tbn_hip.TUNE_CONV_SPLITS, 2):
            tbn_hip.call("tbn_hip_conv2d_f32_prepacked", tbn_hip.WEIGHTS_BINARY, P(x2), d2, P(cw2), None, 1.0,
                         None, None, 0, P(y2), stream)

    def gemm_split(stream):
        with tbn_hip.tuning(tbn_hip.TUNE_GEMM_TILE, 1), tbn_hip.tuning(tbn_hip.TUNE_GEMM_SPLITS, 5):
            name = ctypes.create_string_buffer(256)
            tbn_hip.call("tbn_hip_gemm_kernel_name", 0, M, N, K, K, Kg_pad, Ng_pad, name, 256)
            assert name.value.decode().endswith(", true>"), name.value  # a split-K kernel
            tbn_hip.call("tbn_hip_gemm_f32_binary", P(A), K, M, N, K, P(wg), Kg_pad, Ng_pad, None, 1.0, None, 0,
                         P(C), N, stream)

    calls = {"conv reference layout": conv_ref_layout, "conv split-K": conv_split, "gemm split-K": gemm_split}
    outs = {"conv reference layout": y1, "conv split-K": y2, "gemm split-K": C}
    before = {}
    for name, f in calls.items():
        f(None)
        before[name] = host(outs[name]).copy()

    codes = {}
    marker = empty((1024,), torch.float32)
    cap = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        marker.fill_(1.0)  # one kernel node, so the graph is not empty
        s = torch.cuda.current_stream().cuda_stream
        for name, f in calls.items():
            try:
                f(s)
                codes[name] = (tbn_hip.SUCCESS, "")
            except tbn_hip.TbnError as e:
                codes[name] = (e.code, e.message)
    del g  # discarded, never launched
    torch.cuda.synchronize()
    for name, (code, msg) in codes.items():
        assert code == tbn_hip.NOT_IMPLEMENTED, f"{name}: {code} {msg}"
        assert "captur" in msg, f"{name}: {msg}"

    for name, f in calls.items():
        outs[name].fill_(float("nan"))
        f(None)
        assert np.array_equal(host(outs[name]), before[name]), name
