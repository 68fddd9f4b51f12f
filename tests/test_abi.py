"""The C-ABI library loads and exports every symbol include/tbn_hip.h declares;
host-side argument validation returns tbn::ErrorCode values before any device
work (no compute calls here, so this runs on the CPU)."""
import ctypes
import re

import tbn_hip


def test_library_exports_every_declared_symbol():
    lib = tbn_hip.lib()
    declared = tbn_hip.header_symbols()
    assert len(declared) >= 25
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(tbn_hip._SIGNATURES), "ctypes signatures out of sync with the header"


def test_version_and_error_string():
    assert tbn_hip.lib().tbn_hip_version() == 100
    assert isinstance(tbn_hip.last_error(), str)


def test_argument_errors_are_reported_before_device_use():
    lib = tbn_hip.lib()
    # negative sizes -> INVALID_SHAPE, no device touched
    assert lib.tbn_hip_quantize_to_binary_f32(None, -1, 0.0, None, None) == tbn_hip.INVALID_SHAPE
    assert "non-negative" in tbn_hip.last_error()
    # K_pad not a multiple of 32 -> INVALID_SHAPE
    rc = lib.tbn_hip_gemm_f32_binary(None, 64, 4, 4, 64, None, 40, 8, None, 1.0, None, 0, None, 4, None)
    assert rc == tbn_hip.INVALID_SHAPE
    # lda < K -> INVALID_ARGUMENT
    rc = lib.tbn_hip_gemm_f32_binary(None, 10, 4, 4, 64, None, 64, 8, None, 1.0, None, 0, None, 4, None)
    assert rc == tbn_hip.INVALID_ARGUMENT
    # unknown layout / sign rule
    assert lib.tbn_hip_pack_binary(None, 64, 8, 7, 64, 8, None, None) == tbn_hip.INVALID_ARGUMENT
    assert lib.tbn_hip_quantize_pack_binary_f32(None, 64, 8, 0, 9, 0.0, 64, 8, None, None) == tbn_hip.INVALID_ARGUMENT
    # conv with an empty output
    d = tbn_hip.conv_desc(1, 1, 2, 2, 1, 5, 5)
    rc = lib.tbn_hip_conv2d_f32_binary(None, ctypes.byref(d), None, 32, 8, None, 1.0, None, 0, None, None)
    assert rc == tbn_hip.INVALID_SHAPE
    # maxpool shape query is host-only
    hw = (ctypes.c_int64 * 2)()
    assert lib.tbn_hip_maxpool2d(None, 1, 1, 112, 112, 3, 3, 2, 2, 1, 1, 1, 1, 0, None, hw, None) == 0
    assert list(hw) == [56, 56]


def test_conv_weight_sizes_are_host_only():
    wb = ctypes.c_int64()
    lib = tbn_hip.lib()
    d = tbn_hip.conv_desc(64, 64, 14, 14, 128, 3, 3, 1, 1, 1, 1)
    assert lib.tbn_hip_conv_weights_bytes(0, ctypes.byref(d), ctypes.byref(wb)) == 0
    assert wb.value == 128 * 2 * 9 * 32 // 8          # two 32-channel chunks x 9 taps
    assert lib.tbn_hip_conv_weights_bytes(1, ctypes.byref(d), ctypes.byref(wb)) == 0
    assert wb.value == 128 * 2 * 9 * 32 // 4
    assert lib.tbn_hip_conv_weights_bytes(5, ctypes.byref(d), ctypes.byref(wb)) == tbn_hip.INVALID_ARGUMENT
    big = tbn_hip.conv_desc(1, 64, 200, 200, 8, 15, 15, 1, 1, 28, 28, 4, 4)  # patch cannot fit the LDS
    assert lib.tbn_hip_conv_weights_bytes(0, ctypes.byref(big), ctypes.byref(wb)) == tbn_hip.INVALID_SHAPE


def test_conv_kernel_name_is_host_only():
    """The diagnostic names the patch kernel a pre-packed conv launches (the
    static rule here: nothing was tuned in this process), with the template
    arguments the launch picks, and rejects bad arguments."""
    lib = tbn_hip.lib()
    buf = ctypes.create_string_buffer(160)
    d = tbn_hip.conv_desc(64, 64, 14, 14, 128, 3, 3, 1, 1, 1, 1)  # config 4
    assert lib.tbn_hip_conv2d_kernel_name(0, ctypes.byref(d), tbn_hip.EPI_RELU, 0, buf, len(buf)) == 0
    name = buf.value.decode()
    # 3x3 taps: the staging items per thread are the smallest of 1, 2, 4, 8 that covers the patch
    assert name.startswith("conv_patch_kernel<PatchCfg<") and re.search(r">, false, 9, [1248], false, false>$", name), name
    assert name.count(",") == 10 and ", 1>" in name, name  # two chunks of 32 channels, summed in turn
    assert lib.tbn_hip_conv2d_kernel_name(1, ctypes.byref(d), 0, 1, buf, len(buf)) == 0
    assert re.search(r">, true, 9, [1248], false, false>$", buf.value.decode()), buf.value.decode()
    d5 = tbn_hip.conv_desc(2, 96, 19, 23, 72, 5, 5, 1, 2, 2, 2)  # a 5x5 kernel: the any-size variant
    assert lib.tbn_hip_conv2d_kernel_name(0, ctypes.byref(d5), 0, 0, buf, len(buf)) == 0
    assert ">, false, 0, " in buf.value.decode() and buf.value.decode().endswith(", false>")
    assert lib.tbn_hip_conv2d_kernel_name(7, ctypes.byref(d), 0, 0, buf, len(buf)) == tbn_hip.INVALID_ARGUMENT
    assert lib.tbn_hip_conv2d_kernel_name(0, ctypes.byref(d), 0, 0, None, 0) == tbn_hip.INVALID_ARGUMENT


def test_fused_stem_pool_shape_rule():
    """TBN_EPI_MAXPOOL3X3S2 is taken on the stem shape (3 channels, 7x7,
    stride 2, M <= 64) with ReLU and refused (NOT_IMPLEMENTED) otherwise; the
    query runs on the host."""
    lib = tbn_hip.lib()
    pool = tbn_hip.EPI_RELU | tbn_hip.EPI_MAXPOOL3X3S2
    stem = tbn_hip.conv_desc(32, 3, 224, 224, 64, 7, 7, 2, 2, 3, 3)
    assert lib.tbn_hip_conv2d_f32_supported(ctypes.byref(stem), pool) == tbn_hip.SUCCESS
    assert lib.tbn_hip_conv2d_f32_supported(ctypes.byref(stem), tbn_hip.EPI_RELU) == tbn_hip.SUCCESS
    # no ReLU, too many channels, another kernel size or stride
    assert lib.tbn_hip_conv2d_f32_supported(ctypes.byref(stem), tbn_hip.EPI_MAXPOOL3X3S2) == tbn_hip.NOT_IMPLEMENTED
    for d in [tbn_hip.conv_desc(1, 3, 64, 64, 65, 7, 7, 2, 2, 3, 3), tbn_hip.conv_desc(1, 4, 64, 64, 64, 7, 7, 2, 2, 3, 3),
              tbn_hip.conv_desc(1, 3, 64, 64, 64, 5, 5, 2, 2, 2, 2), tbn_hip.conv_desc(1, 3, 64, 64, 64, 7, 7, 1, 1, 3, 3)]:
        assert lib.tbn_hip_conv2d_f32_supported(ctypes.byref(d), pool) == tbn_hip.NOT_IMPLEMENTED
        assert "stem shape" in tbn_hip.last_error()
    assert lib.tbn_hip_conv2d_f32_supported(ctypes.byref(stem), 16) == tbn_hip.INVALID_ARGUMENT


def test_tbn_conv_tiles_and_pair_query_are_host_only():
    """TBN conv tiles hold one pixel fragment (the kernel name's first
    argument), and the pair query (mode 2) answers without a GPU: ResNet-18's
    stride-2 downsampling convs pair at batch 2 and 32; a 5x5 conv, a pad-0
    3x3 conv and a geometry forced onto the two-pass kernels do not; a pooled
    epilogue is rejected."""
    lib = tbn_hip.lib()
    buf = ctypes.create_string_buffer(160)
    for d in (tbn_hip.conv_desc(32, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1), tbn_hip.conv_desc(32, 512, 7, 7, 512, 3, 3, 1, 1, 1, 1),
              tbn_hip.conv_desc(1, 1, 28, 28, 6, 5, 5), tbn_hip.conv_desc(64, 64, 14, 14, 128, 3, 3, 1, 1, 1, 1)):
        assert lib.tbn_hip_conv2d_tbn_kernel_name(ctypes.byref(d), tbn_hip.EPI_RELU, buf, len(buf)) == 0
        assert buf.value.decode().startswith("tbn_conv_fused_kernel<1, "), buf.value.decode()

    def pair(d, flags=tbn_hip.EPI_RELU):
        return lib.tbn_hip_conv2d_tbn_prepacked_pair(None, ctypes.byref(d), None, None, ctypes.c_float(1.0), None, None,
                                                     flags, ctypes.c_float(-0.1), ctypes.c_float(0.1), None, None, None,
                                                     ctypes.c_float(1.0), None, 0, None, 2, None)
    for n in (2, 32):
        for c, hw in ((64, 56), (128, 28), (256, 14)):
            assert pair(tbn_hip.conv_desc(n, c, hw, hw, 2 * c, 3, 3, 2, 2, 1, 1)) == 0, (n, c)
    assert pair(tbn_hip.conv_desc(2, 64, 16, 16, 64, 5, 5, 1, 1, 2, 2)) == tbn_hip.NOT_IMPLEMENTED
    assert pair(tbn_hip.conv_desc(2, 64, 16, 16, 64, 3, 3, 1, 1, 0, 0)) == tbn_hip.NOT_IMPLEMENTED
    with tbn_hip.tuning(tbn_hip.TUNE_TBN_CONV, 2):
        assert pair(tbn_hip.conv_desc(2, 64, 16, 16, 64, 3, 3, 2, 2, 1, 1)) == tbn_hip.NOT_IMPLEMENTED
    assert pair(tbn_hip.conv_desc(2, 64, 16, 16, 64, 3, 3, 1, 1, 1, 1),
                tbn_hip.EPI_RELU | tbn_hip.EPI_MAXPOOL2X2) == tbn_hip.INVALID_ARGUMENT
