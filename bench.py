"""Benchmark of the tbn quantized compute path on one MI355X.

A "step" is one float x binary GEMM at the headline shape M = N = K = 4096
(fp32 activations ~ N(0,1) resident in HBM, +-1 weights pre-packed in the
reference's BinaryMatrix layout, per-column fp32 scale ~ U[0.5, 1.5]):
`value` is its GFLOP/s-equivalent (2*M*N*K / t).  The same JSON line carries
the other BASELINE.json configs as secondary figures -- config-4 binary
Conv2D (us per batch of 64), config-3 float x ternary GEMM, config-2 1024^3
GEMM, config-1 LeNet and config-5 ResNet-18 through the device-resident
Session -- the roofline of the GEMM kernel, and the reference's portable CPU
path (restated in oracle/) timed on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                       [--only gemm|conv|ternary|tbn|gemm1024|lenet|resnet]
"""
import argparse
import ctypes
import json
import os
import pathlib
import platform
import sys
import time

import numpy as np

# Kernel arguments in device memory.  Where HIP places them in host memory,
# every kernel's start waits on a read across PCIe (about 2 us per launch:
# ResNet-18 batch 32 through the eager Session, 22 launches, 626 -> 580 us on
# one box, A/B/A/B).  Read by HIP when it initializes, so set before torch.
os.environ.setdefault("HIP_FORCE_DEV_KERNARG", "1")

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "fast-arm-tbcnn_amd" / "python"))
sys.path.insert(0, str(ROOT / "fast-arm-tbcnn_amd" / "lib"))

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA: the pipe every exact fp32 x +-1 product runs on
FP32_PEAK_TFLOPS = 157.3    # MI355X dense fp32 (vector or matrix), for comparison only
TRAFFIC_FILE = ROOT / "profiles" / "traffic.json"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_stream(fn, stream, steps, warmup, torch):
    """Runs fn() `warmup` times, then times `steps` calls with HIP events
    recorded on the stream the kernels are launched on; returns ms per call."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        fn()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def prewarm(fn, seconds, torch):
    """Launches fn() untimed for about `seconds` so the GPU reaches its
    sustained clocks before the warmup steps and the timed region (a cold
    MI355X runs the first few hundred microseconds of work ~10 % slower)."""
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()


def time_graph(step, steps, warmup, torch):
    """Device time of one launch for microsecond-scale kernels: `steps`
    launches captured into a HIP graph and replayed, timed with HIP events, so
    the Python launch overhead (about 10 us per ctypes call) is not counted.
    Only for entry points that allocate nothing."""
    for _ in range(warmup):
        step(None)
    torch.cuda.synchronize()
    cap = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        sh = torch.cuda.current_stream().cuda_stream
        for _ in range(steps):
            step(sh)
    g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    reps = 3
    for _ in range(reps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / (reps * steps)


# ---- workloads --------------------------------------------------------------------------

def packed_gemm(torch, tbn_hip, M, N, K, seed, ternary=False):
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    A = torch.randn((M, K), generator=g, device=dev, dtype=torch.float32)
    K_pad, N_pad = tbn_hip.padded_dims(K, N)
    if ternary:
        u = torch.rand((K, N), generator=g, device=dev)
        t = torch.where(u < 0.3, -1, torch.where(u < 0.7, 0, 1)).to(torch.int8)  # p = 0.3/0.4/0.3
        packed = torch.empty(N_pad * K_pad // 4, dtype=torch.uint8, device=dev)
        tbn_hip.call("tbn_hip_pack_ternary", t.data_ptr(), K, N, tbn_hip.LAYOUT_KN, K_pad, N_pad,
                     packed.data_ptr(), None)
    else:
        binw = (torch.rand((K, N), generator=g, device=dev) < 0.5).to(torch.uint8)
        packed = torch.empty(N_pad * K_pad // 8, dtype=torch.uint8, device=dev)
        tbn_hip.call("tbn_hip_pack_binary", binw.data_ptr(), K, N, tbn_hip.LAYOUT_KN, K_pad, N_pad,
                     packed.data_ptr(), None)
    scale = torch.rand(N, generator=g, device=dev, dtype=torch.float32) + 0.5
    C = torch.empty((M, N), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    fn_name = "tbn_hip_gemm_f32_ternary" if ternary else "tbn_hip_gemm_f32_binary"

    def step(sh):
        tbn_hip.call(fn_name, A.data_ptr(), K, M, N, K, packed.data_ptr(), K_pad, N_pad,
                     scale.data_ptr(), 1.0, 0, 0, C.data_ptr(), N, sh)
    keep = (A, packed, scale, C)
    return step, keep, K_pad, N_pad


def conv_cfg4(torch, tbn_hip, seed):
    """Config 4: x[64,64,14,14] ~ N(0,1), W[128,64,3,3] +-1, per-channel scale,
    bias ~ N(0, 0.01), stride 1, pad 1, ReLU."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = torch.randn((64, 64, 14, 14), generator=g, device=dev)
    wb = (torch.rand((128, 64 * 9), generator=g, device=dev) < 0.5).to(torch.uint8)
    scale = torch.rand(128, generator=g, device=dev) + 0.5
    bias = torch.randn(128, generator=g, device=dev) * 0.01
    K_pad, N_pad = tbn_hip.padded_dims(576, 128)
    packed = torch.empty(N_pad * K_pad // 8, dtype=torch.uint8, device=dev)
    tbn_hip.call("tbn_hip_pack_binary", wb.data_ptr(), 576, 128, tbn_hip.LAYOUT_NK, K_pad, N_pad,
                 packed.data_ptr(), None)
    y = torch.empty((64, 128, 14, 14), device=dev)
    desc = tbn_hip.conv_desc(64, 64, 14, 14, 128, 3, 3, 1, 1, 1, 1)
    # weights re-ordered once into the conv layout, as a Session does at init
    wbytes = ctypes.c_int64()
    tbn_hip.call("tbn_hip_conv_weights_bytes", tbn_hip.WEIGHTS_BINARY, desc, ctypes.byref(wbytes))
    conv_w = torch.empty(wbytes.value, dtype=torch.uint8, device=dev)
    tbn_hip.call("tbn_hip_pack_conv_weights", tbn_hip.WEIGHTS_BINARY, packed.data_ptr(), K_pad, N_pad, desc,
                 conv_w.data_ptr(), None)
    # the tile is timed once per geometry, as a Session does when it compiles
    tbn_hip.call("tbn_hip_conv2d_tune_prepacked", tbn_hip.WEIGHTS_BINARY, x.data_ptr(), desc, conv_w.data_ptr(),
                 scale.data_ptr(), 1.0, bias.data_ptr(), None, tbn_hip.EPI_RELU, y.data_ptr(), None)
    torch.cuda.synchronize()

    def step(sh):
        tbn_hip.call("tbn_hip_conv2d_f32_prepacked", tbn_hip.WEIGHTS_BINARY, x.data_ptr(), desc, conv_w.data_ptr(),
                     scale.data_ptr(), 1.0, bias.data_ptr(), None, tbn_hip.EPI_RELU, y.data_ptr(), sh)

    def step_reference_layout(sh):
        tbn_hip.call("tbn_hip_conv2d_f32_binary", x.data_ptr(), desc, packed.data_ptr(), K_pad, N_pad,
                     scale.data_ptr(), 1.0, bias.data_ptr(), tbn_hip.EPI_RELU, y.data_ptr(), sh)
    return step, step_reference_layout, (x, packed, conv_w, scale, bias, y, desc)


def conv_cfg4_tbn(torch, tbn_hip, keep):
    """Config 4's layer in TBN arithmetic (the reference's own quantized
    conv: taps ternarized at +-0.1, integer products, float(C) * s + b, ReLU)
    on the same inputs and weights, the weights in the TBN conv layout."""
    x, packed, _, scale, bias, y, desc = keep
    K_pad, N_pad = tbn_hip.padded_dims(576, 128)
    nbytes = ctypes.c_int64()
    tbn_hip.call("tbn_hip_tbn_conv_weights_bytes", desc, ctypes.byref(nbytes))
    w4 = torch.empty(nbytes.value, dtype=torch.uint8, device=x.device)
    tbn_hip.call("tbn_hip_pack_tbn_conv_weights", packed.data_ptr(), K_pad, N_pad, desc, w4.data_ptr(), None)
    tbn_hip.call("tbn_hip_tbn_conv_scratch_bytes", desc, ctypes.byref(nbytes))
    scratch = torch.empty(nbytes.value, dtype=torch.uint8, device=x.device)
    torch.cuda.synchronize()

    def step(sh):
        tbn_hip.call("tbn_hip_conv2d_tbn_prepacked", x.data_ptr(), desc, w4.data_ptr(), scale.data_ptr(), 1.0,
                     bias.data_ptr(), None, tbn_hip.EPI_RELU, -0.1, 0.1, scratch.data_ptr(), y.data_ptr(), sh)
    return step, (w4, scratch)


def session_workload(torch, _tbn, which, stream, replay, arithmetic="f32"):
    """Config 1 (LeNet, batch 1) or config 5 (ResNet-18, batch 32) through
    TBNModel::Session with quantization on, eager or replaying the Session's
    HIP graph of the forward (the same kernels, launched without the host);
    the input is already in HBM, the output stays there.  arithmetic "tbn":
    the reference's own quantized arithmetic (QuantArithmetic::TBN)."""
    sys.path.insert(0, str(ROOT / "tests"))
    import models
    if which == "lenet":
        spec, x = models.lenet(seed=1), models.lenet_input(1)
    else:
        spec, x = models.resnet18(batch=32, seed=5), models.resnet_input(32, seed=5)
    model = _tbn.TBNModel(models.build_graph(spec, _tbn))
    sess = model.create_session()
    sess.set_quantization(True)
    sess.set_quant_arithmetic(arithmetic)
    xd = torch.from_numpy(x).cuda()
    torch.cuda.synchronize()
    _tbn.set_current_stream(stream.cuda_stream)
    sess.set_input("input", _tbn.Tensor.wrap(xd.data_ptr(), list(x.shape), "float32", "hip"))
    if replay:
        sess.set_graph_replay(True)

    def step(sh):
        sess.run()
    return step, (model, sess, xd)


def mfma_roofline(flops, ms, kernel, algo_bytes, traffic_entry):
    """Roofline object for a kernel on the bf16 matrix pipe: algorithmic
    flop rate over the dense bf16 peak, the issued-MFMA rate (3 bf16 products
    per fp32 x +-1 product), and HBM traffic from the calibrated counters."""
    tflops = flops / (ms * 1e-3) / 1e12
    out = {
        "bound": "mfma",
        "achieved": round(tflops, 2),
        "peak": BF16_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
        "traffic": None,
        "kernel": kernel,
        "mfma_issued": {"dtype": "bf16", "per_product": 3, "tflops": round(3.0 * tflops, 1),
                        "peak": BF16_PEAK_TFLOPS, "frac": round(3.0 * tflops / BF16_PEAK_TFLOPS, 4)},
        "fp32_peak_ratio": round(tflops / FP32_PEAK_TFLOPS, 3),
        "algorithmic_bytes": int(algo_bytes),
        "hbm_gbs_algorithmic": round(algo_bytes / (ms * 1e-3) / 1e9, 1),
    }
    if traffic_entry:
        out["traffic"] = traffic_entry.get("bytes_per_launch")
        out["traffic_kernel"] = traffic_entry.get("kernel")
    return out


def cpu_baseline(M, N, K, budget_s):
    """The reference's portable CPU path for qlinear_matmul_binary (ternarized
    activations, BinaryMatrix re-pack, scalar popcount GemmEngine), restated in
    oracle/tbn_oracle.c, one thread, on a bounded sample of the workload."""
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_api as orc

    rng = np.random.default_rng(7)
    A = rng.standard_normal((M, K)).astype(np.float32)
    binw = (rng.random((K, N)) < 0.5).astype(np.uint8)
    tiling = (128, 256, 256, 16, 8)  # the reference's fastest portable tiling (gemm.cpp:323-329)
    times = []
    t_end = time.perf_counter() + budget_s
    while not times or (time.perf_counter() < t_end and len(times) < 5):
        t0 = time.perf_counter()
        rc, _ = orc.qlinear_matmul_binary_tbn(A, binw, 1.0, tiling)
        times.append(time.perf_counter() - t0)
        assert rc == 0, rc
    best = min(times)
    rows = 64  # the true fp32-activation reference loop (qlinear_matmul_binary_naive), on 64 rows
    t0 = time.perf_counter()
    orc.qlinear_matmul_binary_naive(A[:rows], binw, 1.0)
    naive_s = time.perf_counter() - t0
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(2.0 * M * N * K / best / 1e9, 2),
        "unit": "GFLOP/s-equiv",
        "cores": 1,
        "kind": "port",
        "sample": (f"{M}x{K}x{N} qlinear_matmul_binary, mode TBN (reference portable path: pack_from_float, "
                   f"BinaryMatrix::pack, scalar popcount GemmEngine, tiling 128/256/256/16/8), best of "
                   f"{len(times)} runs, 1 thread, gcc -O3 -march=x86-64-v3, host {cpu}"),
        "fp32_naive_gflops": round(2.0 * rows * N * K / naive_s / 1e9, 3),
        "fp32_naive_sample": f"{rows}x{K}x{N} qlinear_matmul_binary_naive (true fp32 x binary), 1 thread",
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--prewarm", type=float, default=0.3,
                    help="seconds of untimed headline launches before its warmup steps (GPU clock ramp); "
                         "the other lines prewarm for a third of it")
    ap.add_argument("--only", choices=["gemm", "conv", "conv_tbn", "ternary", "tbn", "gemm1024", "lenet", "resnet",
                                       "lenet_tbn", "resnet_tbn", "groups"],
                    help="run one workload only (for profiling)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run 3 device copies of 1 GiB (known bytes) for counter calibration")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build runs on a single GPU (batch/M sharding with "
              "replicated packed weights needs no exchange); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import tbn_hip
    import _tbn

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    tbn_hip.call("tbn_hip_device_check")
    stream = torch.cuda.Stream()
    sh = stream.cuda_stream
    want = (lambda name: args.only is None or args.only == name)

    def timed(step, warm=True):
        # every line after a short prewarm of its own, so each is measured at
        # the sustained clocks the headline is
        with torch.cuda.stream(stream):
            if warm:
                prewarm(lambda: step(sh), args.prewarm / 3, torch)
            return time_stream(lambda: step(sh), stream, args.steps, args.warmup, torch)

    extra = {}
    M = N = K = 4096
    ms = None
    K_pad = N_pad = None
    if want("gemm"):
        step, keep, K_pad, N_pad = packed_gemm(torch, tbn_hip, M, N, K, seed=1)
        with torch.cuda.stream(stream):
            prewarm(lambda: step(sh), args.prewarm, torch)
        ms = timed(step, warm=False)
        log(f"gemm 4096^3 float x binary: {ms * 1e3:.1f} us/launch, {2.0 * M * N * K / ms / 1e9:.1f} TFLOP/s-eq")
        del keep
    if want("conv") or want("conv_tbn"):
        step, step_ref, keep = conv_cfg4(torch, tbn_hip, seed=2)
    if want("conv_tbn"):
        tstep, w4 = conv_cfg4_tbn(torch, tbn_hip, keep)
        with torch.cuda.stream(stream):
            prewarm(lambda: tstep(sh), args.prewarm / 3, torch)
        tc_ms = time_graph(tstep, args.steps, args.warmup, torch)
        kname = ctypes.create_string_buffer(160)
        tbn_hip.call("tbn_hip_conv2d_tbn_kernel_name", keep[-1], tbn_hip.EPI_RELU, kname, len(kname))
        # HBM-bound: the fp32 input read once, the fp4 weights, the fp32 output
        tc_bytes = 4.0 * 64 * 64 * 196 + w4[0].numel() + 8.0 * 128 + 4.0 * 64 * 128 * 196
        extra["conv_tbn_us_per_batch"] = round(tc_ms * 1e3, 2)
        extra["roofline_conv_tbn"] = {
            "bound": "hbm", "achieved": round(tc_bytes / (tc_ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(tc_bytes / (tc_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": kname.value.decode(), "algorithmic_bytes": int(tc_bytes),
            "gops_equiv": round(2.0 * 64 * 196 * 576 * 128 / (tc_ms * 1e-3) / 1e9, 1)}
        log(f"conv cfg4 batch 64, TBN arithmetic: {tc_ms * 1e3:.2f} us/batch ({kname.value.decode()})")
        del w4
    if want("conv"):
        with torch.cuda.stream(stream):
            prewarm(lambda: step(sh), args.prewarm / 3, torch)
        conv_ms = time_graph(step, args.steps, args.warmup, torch)
        conv_flops = 2.0 * 64 * 196 * 576 * 128
        extra["conv_us_per_batch"] = round(conv_ms * 1e3, 2)
        extra["conv_gflops_equiv"] = round(conv_flops / (conv_ms * 1e-3) / 1e9, 1)
        # the tile this process's tuner chose (it can differ between runs
        # within a few percent; all tiles sum in the same order)
        kname = ctypes.create_string_buffer(160)
        tbn_hip.call("tbn_hip_conv2d_kernel_name", tbn_hip.WEIGHTS_BINARY, keep[-1], tbn_hip.EPI_RELU, 0, kname,
                     len(kname))
        extra["conv_kernel"] = kname.value.decode()
        ref_ms = timed(step_ref)
        extra["conv_reference_layout_us_per_batch"] = round(ref_ms * 1e3, 2)
        log(f"conv cfg4 batch 64: {conv_ms * 1e3:.1f} us/batch pre-packed, {ref_ms * 1e3:.1f} us with the "
            f"per-call weight re-order of the reference-layout entry point")
    if want("conv") or want("conv_tbn"):
        del keep
    if want("ternary"):
        step, keep, _, _ = packed_gemm(torch, tbn_hip, 256, 4096, 4096, seed=3, ternary=True)
        t_ms = timed(step)
        extra["ternary_cfg3_us"] = round(t_ms * 1e3, 2)
        extra["ternary_cfg3_gflops_equiv"] = round(2.0 * 256 * 4096 * 4096 / (t_ms * 1e-3) / 1e9, 1)
        log(f"ternary cfg3 256x4096x4096: {t_ms * 1e3:.1f} us")
        del keep
    if want("tbn"):
        # TBN mode (the reference's production arithmetic): activations
        # ternarized at +-0.1, integer ternary x binary GEMM, float(C) * scale
        dev = torch.device("cuda:0")
        g = torch.Generator(device=dev)
        g.manual_seed(6)
        A = torch.randn((M, K), generator=g, device=dev)
        binw = (torch.rand((K, N), generator=g, device=dev) < 0.5).to(torch.uint8)
        Kp, Np = tbn_hip.padded_dims(K, N)
        packed = torch.empty(Np * Kp // 8, dtype=torch.uint8, device=dev)
        tbn_hip.call("tbn_hip_pack_binary", binw.data_ptr(), K, N, tbn_hip.LAYOUT_KN, Kp, Np, packed.data_ptr(), None)
        out = torch.empty((M, N), device=dev)

        def tbn_step(sh):
            tbn_hip.call("tbn_hip_qlinear_matmul_binary_tbn", A.data_ptr(), K, M, K, packed.data_ptr(), Kp, N, Np,
                         1.0, -0.1, 0.1, out.data_ptr(), N, sh)
        tb_ms = timed(tbn_step)
        extra["tbn_mode_4096_us"] = round(tb_ms * 1e3, 2)
        extra["tbn_mode_4096_gops"] = round(2.0 * M * N * K / (tb_ms * 1e-3) / 1e9, 1)
        log(f"TBN mode qlinear_matmul_binary 4096^3: {tb_ms * 1e3:.1f} us")
        del A, binw, packed, out
    if want("gemm1024"):
        step, keep, _, _ = packed_gemm(torch, tbn_hip, 1024, 1024, 1024, seed=4)
        # stream-timed: a K-split launch takes the stream workspace, which
        # graph capture refuses; each launch outlasts the Python call
        g_ms = timed(step)
        extra["gemm_cfg2_us"] = round(g_ms * 1e3, 2)
        extra["gemm_cfg2_gflops_equiv"] = round(2.0 * 1024 ** 3 / (g_ms * 1e-3) / 1e9, 1)
        log(f"binary cfg2 1024^3: {g_ms * 1e3:.1f} us")
        del keep
    if want("groups"):
        # depthwise 3x3 (MobileNet-style, batch 32, 128 channels, 56x56) and an
        # unfolded BatchNormalization over the same tensor: both HBM-bound
        dev = torch.device("cuda:0")
        g = torch.Generator(device=dev)
        g.manual_seed(7)
        n, c, h = 32, 128, 56
        x = torch.randn((n, c, h, h), generator=g, device=dev)
        w = torch.randn((c, 1, 3, 3), generator=g, device=dev)
        kk = torch.rand(c, generator=g, device=dev) + 0.5
        tt = torch.randn(c, generator=g, device=dev)
        y = torch.empty_like(x)
        d = tbn_hip.conv_desc(n, c, h, h, c, 3, 3, 1, 1, 1, 1)

        def dw_step(sh):
            tbn_hip.call("tbn_hip_conv2d_depthwise", x.data_ptr(), ctypes.byref(d), w.data_ptr(), None, 1.0, None,
                         None, tbn_hip.EPI_RELU, y.data_ptr(), sh)

        def bn_step(sh):
            tbn_hip.call("tbn_hip_channel_affine", x.data_ptr(), n, c, h * h, kk.data_ptr(), tt.data_ptr(), 0,
                         y.data_ptr(), sh)
        nbytes = 2 * 4.0 * x.numel()
        for name, fn in (("depthwise3x3", dw_step), ("batchnorm", bn_step)):
            t_ms = timed(fn)
            extra[name + "_32x128x56x56_us"] = round(t_ms * 1e3, 2)
            extra[name + "_32x128x56x56_GBps"] = round(nbytes / (t_ms * 1e-3) / 1e9, 1)
            log(f"{name} 32x128x56x56: {t_ms * 1e3:.1f} us, {nbytes / (t_ms * 1e-3) / 1e9:.0f} GB/s")
        del x, y, w, kk, tt
    for which, key, replay, arith in (("lenet", "lenet_session_us_per_forward", False, "f32"),
                                      ("lenet", "lenet_session_replay_us_per_forward", True, "f32"),
                                      ("resnet", "resnet18_session_ms_per_batch32", False, "f32"),
                                      ("lenet", "lenet_tbn_session_replay_us_per_forward", True, "tbn"),
                                      ("resnet", "resnet18_tbn_session_ms_per_batch32", False, "tbn")):
        if not want(which if arith == "f32" else which + "_tbn"):
            continue
        step, keep = session_workload(torch, _tbn, which, stream, replay, arith)
        s_ms = timed(step)
        extra[key] = round(s_ms * (1e3 if which == "lenet" else 1.0), 3)
        extra[which + ("_tbn" if arith == "tbn" else "") + "_session_launches"] = keep[1].planned_launches()
        log(f"{which} session ({arith}, {'graph replay' if replay else 'eager'}): {s_ms * 1e3:.1f} us per "
            f"forward ({keep[1].planned_launches()} launches)")
        _tbn.set_current_stream(0)
        del keep

    if args.copy_calibration:
        # an elementwise kernel that reads 1 GiB and writes 1 GiB (known bytes)
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        with torch.cuda.stream(stream):
            for _ in range(3):
                torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        log("copy calibration: 3 x (read 1 GiB, write 1 GiB) elementwise kernels")

    if ms is None:
        print(json.dumps({"only": args.only, **extra}), flush=True)
        return

    flops = 2.0 * M * N * K
    gflops = flops / (ms * 1e-3) / 1e9
    algo_bytes = 4.0 * M * K + K_pad * N_pad / 8 + 4.0 * N + 4.0 * M * N
    traffic = json.loads(TRAFFIC_FILE.read_text()) if TRAFFIC_FILE.exists() else {}
    # Every fp32 x +-1 product runs on the bf16 matrix pipe (three exact bf16
    # products per fp32 one), so the roofline is the dense bf16 MFMA peak and
    # `frac` is the algorithmic rate over it; `mfma_issued` counts the three
    # products actually issued, and `fp32_peak_ratio` compares with the fp32
    # peak a plain fp32 kernel would be bound by.
    kname = ctypes.create_string_buffer(256)
    tbn_hip.call("tbn_hip_gemm_kernel_name", tbn_hip.WEIGHTS_BINARY, M, N, K, K, K_pad, N_pad, kname, 256)
    gemm_traffic = traffic.get("gemm_f32_binary_4096")
    if gemm_traffic and gemm_traffic.get("kernel") != kname.value.decode():
        gemm_traffic = None  # counters of another kernel do not describe this one
    roofline = mfma_roofline(flops, ms, kname.value.decode(), algo_bytes, gemm_traffic)
    if "conv_us_per_batch" in extra:
        conv_bytes = 4.0 * 64 * 64 * 196 + 128 * 640 / 8 + 8.0 * 128 + 4.0 * 64 * 128 * 196
        # counter traffic measured on the kernel this run timed (one entry per
        # tile the tuner takes on this shape), else none
        conv_traffic = next((e for k, e in traffic.items() if k.startswith("conv_cfg4") and isinstance(e, dict)
                             and e.get("kernel") == extra.get("conv_kernel")), None)
        extra["roofline_conv"] = mfma_roofline(2.0 * 64 * 196 * 576 * 128, extra["conv_us_per_batch"] * 1e-3,
                                               extra.get("conv_kernel", "conv_patch_kernel"), conv_bytes,
                                               conv_traffic)

    result = {
        "metric": "float×binary GEMM GFLOP/s-equiv @4096³; Conv2D 64→128 14×14 µs/batch",
        "value": round(gflops, 1),
        "unit": "GFLOP/s-equiv",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "strong",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (A ~ N(0,1), W +-1 p=0.5, scale ~ U[0.5,1.5]; generated on device, seeded)",
        "prewarm_s": args.prewarm,
        "config": {
            "workload": "float x binary GEMM M=N=K=4096, fp32 activations, BinaryMatrix-packed +-1 weights, "
                        "per-column fp32 scale (mode F32: exact products, fp32 accumulation)",
            "M": M, "N": N, "K": K, "K_pad": K_pad, "N_pad": N_pad,
            "conv_workload": "binary Conv2D 64x14x14 -> 128x14x14, 3x3, s1 p1, batch 64, per-channel scale, "
                             "bias, ReLU (config 4)",
        },
        **extra,
        "roofline": roofline,
    }
    if not args.no_cpu_baseline and args.only is None:
        log("timing the CPU baseline ...")
        result["cpu_baseline"] = cpu_baseline(M, N, K, args.cpu_budget)
    else:
        result["cpu_baseline"] = None
    result["host"] = platform.node()
    result["hip_env"] = {"HIP_FORCE_DEV_KERNARG": os.environ.get("HIP_FORCE_DEV_KERNARG")}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
