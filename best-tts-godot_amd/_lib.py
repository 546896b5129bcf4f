"""ctypes binding of libkk (include/kk.h).

Loading fails loudly: there is no CPU path behind this module.  Every entry
point returns a status; a non-zero status raises :class:`KKError` carrying
``kk_last_error()``.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkk.so")

KK_MAX_RANK = 8

# dtype codes (KPK1, tools/kpk_runtime.py:21-24)
F32, I8, U8, I32, I64, BOOL, F16 = 0, 1, 2, 3, 4, 5, 6

# elementwise op codes (include/kk.h)
OP = {
    "Add": 0, "Sub": 1, "Mul": 2, "Div": 3, "Pow": 4, "Sqrt": 5, "Exp": 6,
    "Sin": 7, "Cos": 8, "Atan": 9, "Tanh": 10, "Sigmoid": 11, "Floor": 12,
    "Round": 13, "LeakyRelu": 14, "Equal": 16, "Greater": 17, "Less": 18,
    "GreaterOrEqual": 19, "And": 20, "Identity": 24, "Neg": 25, "Abs": 26,
    "Log": 27, "Min": 28, "Max": 29, "Erf": 30,
}
REDUCE_SUM, REDUCE_MEAN, REDUCE_MAX = 0, 1, 2

KK_E = {-1: "KK_E_ARG", -2: "KK_E_HIP", -3: "KK_E_NOMEM", -4: "KK_E_STATE",
        -5: "KK_E_UNSUPPORTED"}


class KKError(RuntimeError):
    """A libkk entry point returned an error status."""

    def __init__(self, fn, code, msg):
        super().__init__(f"{fn}: {KK_E.get(code, code)}: {msg}")
        self.code = code


class KKTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("dtype", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("shape", ctypes.c_int64 * KK_MAX_RANK),
        ("strides", ctypes.c_int64 * KK_MAX_RANK),
    ]


_T = ctypes.POINTER(KKTensor)
_i, _f, _d, _sz, _vp = ctypes.c_int, ctypes.c_float, ctypes.c_double, ctypes.c_size_t, ctypes.c_void_p

# name -> argument types (all return int status, except kk_last_error)
PROTOTYPES = {
    "kk_init": [_i],
    "kk_shutdown": [],
    "kk_sync": [],
    "kk_device_count": [ctypes.POINTER(_i)],
    "kk_alloc": [_sz, ctypes.POINTER(_vp)],
    "kk_free": [_vp],
    "kk_pool_stats": [ctypes.POINTER(_sz)] * 3,
    "kk_pool_trim": [_sz],
    "kk_upload": [_vp, _vp, _sz],
    "kk_download": [_vp, _vp, _sz],
    "kk_binary": [_i, _T, _T, _T],
    "kk_unary": [_i, _T, _T, _f],
    "kk_where": [_T, _T, _T, _T],
    "kk_clip": [_T, _T, _T, _T],
    "kk_snake": [_T, _T, _T, _T],
    "kk_fast_gelu": [_T, _T, _T],
    "kk_dequantize": [_T, _T, _T, _T],
    "kk_copy": [_T, _T],
    "kk_fill": [_T, _d],
    "kk_gather": [_T, _T, _T, _i],
    "kk_reduce": [_i, _T, _T, ctypes.c_uint32],
    "kk_instance_norm_affine": [_T, _T, _T, _f],
    "kk_adain": [_T, _T, _T, _T, _T, _T, _T, _f],
    "kk_layernorm": [_T, _T, _T, _T, _T, _T, _i, _f],
    "kk_softmax": [_T, _T, _i],
    "kk_gemm": [_T, _T, _T, _T, _T, _f],
    "kk_gemm_packed_bytes": [ctypes.c_int64, ctypes.c_int64, _i, ctypes.POINTER(ctypes.c_int64)],
    "kk_gemm_pack": [_T, _T, _T],
    "kk_gemm_packed": [_T] * 6 + [_f],
    "kk_conv1d": [_T, _T, _T, _T, _T, _T, _i, _i, _i, _i, _i],
    "kk_conv_transpose1d": [_T, _T, _T, _T, _T, _T, _i, _i, _i, _i, _i, _i],
    "kk_conv_packed_bytes": [_i, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _i,
                             ctypes.POINTER(ctypes.c_int64)],
    "kk_conv_pack": [_T, _T, _T, _i, _i],
    "kk_conv1d_packed": [_T] * 7 + [_i, _i, _i, _i],
    "kk_conv_transpose1d_packed": [_T] * 7 + [_i, _i, _i, _i],
    "kk_event_record": [_i],
    "kk_event_elapsed": [_i, _i, ctypes.POINTER(_f)],
    "kk_dynamic_quantize_linear": [_T, _T, _T, _T],
    "kk_matmul_integer": [_T, _T, _T, _T, _T],
    "kk_matmul_integer_scaled": [_T, _T, _T, _T, _T, _T, _T, _T],
    "kk_matmul_integer_packed": [_T, _T, _T, _T, _T, _T],
    "kk_matmul_integer_scaled_packed": [_T, _T, _T, _T, _T, _T, _T, _T, _T],
    "kk_matmul_integer_pack_bytes": [_T, ctypes.POINTER(_sz)],
    "kk_matmul_integer_pack": [_T, _T],
    "kk_conv_integer": [_T, _T, _T, _T, _T, _i, _i, _i, _i, _i],
    "kk_conv_integer_scaled": [_T] * 7 + [_i, _i, _i, _i, _i],
    "kk_conv_integer_scaled_qbias": [_T] * 8 + [_i, _i, _i, _i, _i],
    "kk_conv_integer_scaled_add": [_T] * 8 + [_i, _i, _i, _i, _i],
    "kk_conv_integer_scaled_qbias_add": [_T] * 9 + [_i, _i, _i, _i, _i],
    "kk_conv_integer_packed_bytes": [ctypes.c_int64] * 3 + [ctypes.POINTER(ctypes.c_int64)],
    "kk_conv_integer_pack": [_T] * 3,
    "kk_conv_integer_scaled_qbias_packed": [_T] * 10 + [_i] * 5,
    "kk_conv_integer_scaled_qbias_packed_leaves": [_T] * 11 + [_i] * 5,
    "kk_conv_integer_scaled_qbias_noalloc": [_T] * 8 + [_i, _i, _i, _i, _i],
    "kk_instance_norm_scale_shift": [_T, _T, _T, _T, _f, _i, _f],
    "kk_instance_norm_scale_shift_snake": [_T, _T, _T, _T, _T, _T, _f],
    "kk_instance_norm_quant": [_T, _T, _T, _T, _T, _T, _T, _T, _f, _i, _f],
    "kk_instance_norm_quant_leaves": [_T, _T, _T, _T, _T, _T, _T, _T, _f, _i, _f, _T],
    "kk_lstm": [_T] * 13 + [_i, _i],
    "kk_stft": [_T, _T, _T, ctypes.c_int64, ctypes.c_int64, _i],
    "kk_resize": [_T, _T, _i, _d],
    "kk_pad": [_T, _T, ctypes.POINTER(ctypes.c_int64), _i, _f],
    "kk_cumsum": [_T, _T, _i],
    "kk_scatter_nd": [_T, _T, ctypes.POINTER(ctypes.c_int64), ctypes.c_int64, ctypes.c_int64],
    "kk_fir": [_T, _T, _T, _i],
    "kk_pcm16": [_T, _T, _f],
    "kk_fir_pcm16": [_T, _T, _T, _i, _f],
    "kk_graph_begin": [],
    "kk_graph_begin_arena": [_sz],
    "kk_graph_abort": [],
    "kk_graph_end": [ctypes.POINTER(_i)],
    "kk_graph_launch": [_i],
    "kk_graph_destroy": [_i],
    "kk_graph_nodes": [_i, ctypes.POINTER(ctypes.c_int64)],
    "kk_dispatch_count": [ctypes.POINTER(ctypes.c_uint64)],
}

_lib = None


def load(path=LIB_PATH):
    """Load libkk.so (once) and attach prototypes.  Raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"libkk.so not found at {path}: build it with "
            "`python best-tts-godot_amd/build_lib.py` (there is no CPU fallback)")
    lib = ctypes.CDLL(path)
    for name, argtypes in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    lib.kk_last_error.argtypes = []
    lib.kk_last_error.restype = ctypes.c_char_p
    _lib = lib
    return lib


_bound = {}  # name -> bound entry point


def raise_error(name, rc):
    """Raise KKError for status `rc` of entry point `name`."""
    msg = load().kk_last_error().decode(errors="replace")
    raise KKError(name, rc, msg)


def call(name, *args):
    """Call entry point `name`; raise KKError on a non-zero status."""
    fn = _bound.get(name)
    if fn is None:
        fn = _bound[name] = getattr(load(), name)
    rc = fn(*args)
    if rc != 0:
        raise_error(name, rc)
    return rc


def exported_symbols():
    """Names declared in PROTOTYPES plus kk_last_error."""
    return sorted(list(PROTOTYPES) + ["kk_last_error"])
