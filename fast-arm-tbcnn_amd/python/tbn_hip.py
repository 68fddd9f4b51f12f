"""ctypes binding of libtbn_hip.so, the C ABI declared in include/tbn_hip.h.

Every function takes DEVICE pointers (ints, e.g. ``tensor.data_ptr()``) and an
optional HIP stream handle; a non-zero status raises :class:`TbnError` carrying
the tbn::ErrorCode value and the library's message.  There is no fallback: if
the shared library is missing, :func:`lib` raises immediately.
"""
import ctypes
import pathlib
import re

PACKAGE_DIR = pathlib.Path(__file__).resolve().parents[1]
LIB_PATH = PACKAGE_DIR / "lib" / "libtbn_hip.so"
HEADER_PATH = PACKAGE_DIR.parent / "include" / "tbn_hip.h"

# tbn::ErrorCode (tbn-runtime/include/tbn/utils/errors.hpp:10-22)
SUCCESS = 0
INVALID_ARGUMENT = -1
OUT_OF_MEMORY = -2
NOT_IMPLEMENTED = -3
INVALID_MODEL = -4
RUNTIME_ERROR = -5
QUANTIZATION_ERROR = -6
INVALID_SHAPE = -7
DEVICE_NOT_SUPPORTED = -8

LAYOUT_KN = 0
LAYOUT_NK = 1
SIGN_GT_THRESHOLD = 0
SIGN_GE_ZERO = 1
SIGN_GEMM_SAMPLED = 2
EPI_NONE = 0
EPI_RELU = 1
EPI_BIAS_THEN_SCALE = 2
EPI_MAXPOOL2X2 = 4
EPI_MAXPOOL3X3S2 = 8
NOALLOC_SCRATCH_BYTES = 16 << 20
WEIGHTS_BINARY = 0
WEIGHTS_TERNARY = 1
TUNE_CONV_TILE = 1
TUNE_CONV_SPLITS = 2
TUNE_GEMM_SPLITS = 3
TUNE_GEMM_TILE = 4
TUNE_TBN_CONV = 5
OP_SUB = 0
OP_GREATER = 1
OP_LESS = 2


class TbnError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(f"tbn_hip error {code}: {message}")
        self.code = code
        self.message = message


class ConvDesc(ctypes.Structure):
    _fields_ = [(name, ctypes.c_int64) for name in
                ("n", "c", "h", "w", "m", "kh", "kw", "sh", "sw", "ph", "pw", "dh", "dw")]


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F32 = ctypes.c_float

_SIGNATURES = {
    "tbn_hip_last_error": ([], ctypes.c_char_p),
    "tbn_hip_version": ([], _I32),
    "tbn_hip_device_check": ([], _I32),
    "tbn_hip_synchronize": ([_P], _I32),
    "tbn_hip_set_tuning": ([_I32, _I32], _I32),
    "tbn_hip_get_tuning": ([_I32, ctypes.POINTER(ctypes.c_int)], _I32),
    "tbn_hip_quantize_to_binary_f32": ([_P, _I64, _F32, _P, _P], _I32),
    "tbn_hip_quantize_to_binary_i8": ([_P, _I64, _P, _P], _I32),
    "tbn_hip_quantize_to_ternary_f32": ([_P, _I64, _F32, _F32, _P, _P], _I32),
    "tbn_hip_sign_ge0_f32": ([_P, _I64, _P, _P], _I32),
    "tbn_hip_channel_mean_abs": ([_P, _I64, _I64, _P, _P], _I32),
    "tbn_hip_pack_binary": ([_P, _I64, _I64, _I32, _I64, _I64, _P, _P], _I32),
    "tbn_hip_quantize_pack_binary_f32": ([_P, _I64, _I64, _I32, _I32, _F32, _I64, _I64, _P, _P], _I32),
    "tbn_hip_unpack_binary": ([_P, _I64, _I64, _I32, _I64, _P, _P], _I32),
    "tbn_hip_pack_ternary2": ([_P, _I64, _P, _P], _I32),
    "tbn_hip_unpack_ternary2": ([_P, _I64, _P, _P], _I32),
    "tbn_hip_pack_ternary": ([_P, _I64, _I64, _I32, _I64, _I64, _P, _P], _I32),
    "tbn_hip_quantize_pack_ternary_f32": ([_P, _I64, _I64, _I32, _F32, _F32, _I64, _I64, _P, _P], _I32),
    "tbn_hip_gemm_f32_binary": ([_P, _I64, _I64, _I64, _I64, _P, _I64, _I64, _P, _F32, _P, _I32, _P, _I64, _P], _I32),
    "tbn_hip_gemm_f32_ternary": ([_P, _I64, _I64, _I64, _I64, _P, _I64, _I64, _P, _F32, _P, _I32, _P, _I64, _P], _I32),
    "tbn_hip_conv2d_f32_binary": ([_P, ctypes.POINTER(ConvDesc), _P, _I64, _I64, _P, _F32, _P, _I32, _P, _P], _I32),
    "tbn_hip_conv2d_f32_ternary": ([_P, ctypes.POINTER(ConvDesc), _P, _I64, _I64, _P, _F32, _P, _I32, _P, _P], _I32),
    "tbn_hip_conv2d_f32": ([_P, ctypes.POINTER(ConvDesc), _P, _P, _I32, _P, _P], _I32),
    "tbn_hip_conv2d_f32_supported": ([ctypes.POINTER(ConvDesc), _I32], _I32),
    "tbn_hip_gemm_f32": ([_P, _P, _P, _I32, _I64, _I64, _I64, _F32, _F32, _I32, _I32, _I32, _P, _P], _I32),
    "tbn_hip_maxpool2d": ([_P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P,
                           ctypes.POINTER(ctypes.c_int64), _P], _I32),
    "tbn_hip_global_avgpool2d": ([_P, _I64, _I64, _I64, _I64, _P, _P], _I32),
    "tbn_hip_global_maxpool2d": ([_P, _I64, _I64, _I64, _I64, _P, _P], _I32),
    "tbn_hip_avgpool2d": ([_P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _I32,
                           _P, ctypes.POINTER(ctypes.c_int64), _P], _I32),
    "tbn_hip_add": ([_P, _P, _I64, _I64, _I64, _I64, _I32, _P, _P], _I32),
    "tbn_hip_relu": ([_P, _I64, _P, _P], _I32),
    "tbn_hip_conv2d_depthwise": ([_P, ctypes.POINTER(ConvDesc), _P, _P, _F32, _P, _P, _I32, _P, _P], _I32),
    "tbn_hip_copy_channels": ([_P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I64, _P], _I32),
    "tbn_hip_channel_affine": ([_P, _I64, _I64, _I64, _P, _P, _I32, _P, _P], _I32),
    "tbn_hip_gemm_f32_quantized": ([_I32, _P, _I64, _I64, _I64, _I64, _P, _I64, _I64, _P, _F32, _P, _P, _I32,
                                    _F32, _I32, _P, _I64, _P], _I32),
    "tbn_hip_conv2d_f32_quantized": ([_I32, _P, ctypes.POINTER(ConvDesc), _P, _I64, _I64, _P, _F32, _P, _P,
                                      _I32, _P, _P], _I32),
    "tbn_hip_conv2d_f32_quantized_noalloc": ([_I32, _P, ctypes.POINTER(ConvDesc), _P, _I64, _I64, _P, _F32, _P,
                                              _P, _I32, _P, _P], _I32),
    "tbn_hip_pack_f4_weights": ([_P, _I64, _I64, _P, _P], _I32),
    "tbn_hip_gemm_tbn_prepacked": ([_P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _F32, _P, _I32, _F32, _F32, _F32, _I32,
                                    _P, _P, _I64, _P], _I32),
    "tbn_hip_tbn_conv_weights_bytes": ([ctypes.POINTER(ConvDesc), ctypes.POINTER(ctypes.c_int64)], _I32),
    "tbn_hip_pack_tbn_conv_weights": ([_P, _I64, _I64, ctypes.POINTER(ConvDesc), _P, _P], _I32),
    "tbn_hip_tbn_conv_scratch_bytes": ([ctypes.POINTER(ConvDesc), ctypes.POINTER(ctypes.c_int64)], _I32),
    "tbn_hip_conv2d_tbn_prepacked": ([_P, ctypes.POINTER(ConvDesc), _P, _P, _F32, _P, _P, _I32, _F32, _F32, _P, _P,
                                      _P], _I32),
    "tbn_hip_conv2d_tbn_prepacked_pair": ([_P, ctypes.POINTER(ConvDesc), _P, _P, _F32, _P, _P, _I32, _F32, _F32, _P,
                                           _P, _P, _F32, _P, _I32, _P, _I32, _P], _I32),
    "tbn_hip_conv2d_tbn_kernel_name": ([ctypes.POINTER(ConvDesc), _I32, ctypes.c_char_p, ctypes.c_size_t], _I32),
    "tbn_hip_gemm_kernel_name": ([_I32, _I64, _I64, _I64, _I64, _I64, _I64, ctypes.c_char_p, ctypes.c_size_t], _I32),
    "tbn_hip_conv_weights_bytes": ([_I32, ctypes.POINTER(ConvDesc), ctypes.POINTER(ctypes.c_int64)], _I32),
    "tbn_hip_pack_conv_weights": ([_I32, _P, _I64, _I64, ctypes.POINTER(ConvDesc), _P, _P], _I32),
    "tbn_hip_conv2d_f32_prepacked": ([_I32, _P, ctypes.POINTER(ConvDesc), _P, _P, _F32, _P, _P, _I32, _P, _P], _I32),
    "tbn_hip_conv2d_f32_prepacked_pair": ([_I32, _P, ctypes.POINTER(ConvDesc), _P, _P, _F32, _P, _P, _I32, _P,
                                           _P, _P, _F32, _P, _I32, _P, _I32, _P], _I32),
    "tbn_hip_conv2d_tune_prepacked": ([_I32, _P, ctypes.POINTER(ConvDesc), _P, _P, _F32, _P, _P, _I32, _P, _P],
                                      _I32),
    "tbn_hip_conv2d_kernel_name": ([_I32, ctypes.POINTER(ConvDesc), _I32, _I32, ctypes.c_char_p, ctypes.c_size_t],
                                   _I32),
    "tbn_hip_elementwise": ([_I32, _P, _I64, _P, _I64, _F32, _P, _P], _I32),
    "tbn_hip_ternary_activation": ([_P, _I64, _F32, _P, _P], _I32),
    "tbn_hip_ternary_pack_f32": ([_P, _I64, _I64, _I64, _I64, _I64, _F32, _F32, _P, _P, _P], _I32),
    "tbn_hip_im2col_ternary_packed": ([_P, ctypes.POINTER(ConvDesc), _I64, _I64, _F32, _F32, _P, _P, _P], _I32),
    "tbn_hip_tbn_gemm": ([_P, _P, _P, _I64, _I64, _I64, _P, _P], _I32),
    "tbn_hip_tbn_gemm_scaled": ([_P, _P, _P, _I64, _I64, _I64, _I64, _F32, _P, _I64, _P], _I32),
    "tbn_hip_ternary_pack_i8": ([_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P], _I32),
    "tbn_hip_qlinear_matmul_binary_tbn": ([_P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _F32, _F32, _F32, _P, _I64,
                                           _P], _I32),
}

_lib = None


def lib():
    """Loads libtbn_hip.so once; raises FileNotFoundError if it was not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(f"{LIB_PATH} not built; run __graft_entry__.build()")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        _lib = handle
    return _lib


def header_symbols():
    """Names of the functions declared in include/tbn_hip.h."""
    text = HEADER_PATH.read_text()
    return sorted(set(re.findall(r"\b(tbn_hip_\w+)\s*\(", text)))


def last_error():
    return lib().tbn_hip_last_error().decode()


def check(status):
    if status != SUCCESS:
        raise TbnError(status, last_error())
    return status


def call(name, *args):
    """Calls ``name`` and raises TbnError on a non-zero status."""
    return check(getattr(lib(), name)(*args))


def ptr(t):
    """Device pointer of a tensor (or None)."""
    return None if t is None else t.data_ptr()


def conv_desc(n, c, h, w, m, kh, kw, sh=1, sw=1, ph=0, pw=0, dh=1, dw=1):
    return ConvDesc(n, c, h, w, m, kh, kw, sh, sw, ph, pw, dh, dw)


def conv_out_hw(d):
    oh = (d.h + 2 * d.ph - d.dh * (d.kh - 1) - 1) // d.sh + 1
    ow = (d.w + 2 * d.pw - d.dw * (d.kw - 1) - 1) // d.sw + 1
    return oh, ow


def padded_dims(K, N):
    """K_pad = ceil128(K), N_pad = ceil8(N) as the reference runtime pads
    (tbn-runtime/src/operators/quantized_gemm_neon.cpp:53-55)."""
    return (K + 127) // 128 * 128, (N + 7) // 8 * 8


class tuning:
    """Context manager that sets a tuning control (TUNE_*) and restores it."""

    def __init__(self, option, value):
        self.option, self.value = option, value

    def __enter__(self):
        old = ctypes.c_int()
        call("tbn_hip_get_tuning", self.option, ctypes.byref(old))
        self.old = old.value
        call("tbn_hip_set_tuning", self.option, self.value)
        return self

    def __exit__(self, *exc):
        call("tbn_hip_set_tuning", self.option, self.old)
        return False
