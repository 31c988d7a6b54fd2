"""
Library loading and ctypes bindings for libneural_hip.so.

Mirrors the reference's ``pyneural/core.py`` (error codes, dtype codes,
``NeuralException``, ``_check_error``, ``init``/``shutdown``/``version``) but
binds the MI355X library.  The search order follows the reference loader
(core.py:49-73): the package's parent directory, the working directory,
``/usr/local/lib``, ``/usr/lib`` and ``LD_LIBRARY_PATH``; ``NEURAL_HIP_LIB``
overrides it.  A missing library raises ImportError -- there is no CPU
fallback.
"""

import ctypes
import os
from pathlib import Path

LIB_NAME = "libneural_hip.so"


class NeuralError:
    """Error codes of neural_api.h:15-35."""
    OK = 0
    NULL_POINTER = 1
    OUT_OF_MEMORY = 2
    INVALID_ARGUMENT = 3
    SHAPE_MISMATCH = 4
    DTYPE_MISMATCH = 5
    FILE_NOT_FOUND = 6
    FILE_READ = 7
    FILE_WRITE = 8
    PARSE_ERROR = 9
    INVALID_CONFIG = 10
    TENSOR_TOO_LARGE = 11
    INVALID_DTYPE = 12
    DIM_MISMATCH = 13
    NOT_IMPLEMENTED = 14
    INTERNAL = 15
    GRAD_CHECK = 16
    NAN_DETECTED = 17
    INF_DETECTED = 18


class NeuralDtype:
    FLOAT32 = 0
    FLOAT64 = 1


class NeuralException(Exception):
    """Raised when a library call returns a nonzero NeuralError code."""

    def __init__(self, error_code: int, message: str = None):
        self.error_code = error_code
        if message is None:
            message = get_error_message(error_code)
        super().__init__(f"NeuralError({error_code}): {message}")


def _find_library() -> str:
    env = os.environ.get("NEURAL_HIP_LIB")
    if env:
        return env
    candidates = [
        Path(__file__).resolve().parent.parent / LIB_NAME,
        Path.cwd() / LIB_NAME,
        Path("/usr/local/lib") / LIB_NAME,
        Path("/usr/lib") / LIB_NAME,
    ]
    for d in os.environ.get("LD_LIBRARY_PATH", "").split(":"):
        if d:
            candidates.append(Path(d) / LIB_NAME)
    for c in candidates:
        if c.exists():
            return str(c)
    return LIB_NAME


def _preload_torch_hip():
    """PyTorch ships its own libamdhip64.so.  Loading it first (by path,
    without importing torch) makes this library bind to the same HIP runtime
    (same SONAME), so torch device pointers, streams and events are valid
    handles here whichever package the process imports first.  Set
    NEURAL_HIP_RUNTIME=system to use the ROCm installation's runtime instead."""
    if os.environ.get("NEURAL_HIP_RUNTIME", "") == "system":
        return None
    try:
        import importlib.util
        spec = importlib.util.find_spec("torch")
        if spec is None or not spec.origin:
            return None
        p = Path(spec.origin).parent / "lib" / "libamdhip64.so"
        if p.exists():
            ctypes.CDLL(str(p), mode=ctypes.RTLD_GLOBAL)
            return str(p)
    except OSError:
        return None
    return None


_hip_runtime = _preload_torch_hip()
_lib_path = _find_library()
try:
    _lib = ctypes.CDLL(_lib_path)
except OSError as e:  # no silent fallback
    raise ImportError(
        f"could not load {LIB_NAME} from {_lib_path}; build it with "
        f"`make -C neural-assembly_amd/csrc` (original error: {e})"
    ) from e


class QuantParamsC(ctypes.Structure):
    """QuantParams (quantize.c:39-45): 40 bytes with natural padding."""
    _fields_ = [
        ("scale", ctypes.c_double),
        ("zero_point", ctypes.c_int32),
        ("min_val", ctypes.c_double),
        ("max_val", ctypes.c_double),
        ("symmetric", ctypes.c_int),
    ]


class NeuralBufferInfo(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("itemsize", ctypes.c_uint64),
        ("ndim", ctypes.c_uint64),
        ("shape", ctypes.POINTER(ctypes.c_uint64)),
        ("strides", ctypes.POINTER(ctypes.c_int64)),
        ("readonly", ctypes.c_int),
        ("format", ctypes.c_char * 8),
    ]


_vp, _i, _i64, _u64, _d, _f = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64,
                                ctypes.c_double, ctypes.c_float)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_i64p = ctypes.POINTER(ctypes.c_int64)
_ip = ctypes.POINTER(ctypes.c_int)
_dp = ctypes.POINTER(ctypes.c_double)
_qp = ctypes.POINTER(QuantParamsC)

_SIGS = {
    # framework
    "neural_init": (_i, []),
    "neural_shutdown": (None, []),
    "neural_version": (ctypes.c_char_p, []),
    "neural_clear_error": (None, []),
    "neural_get_last_error": (_i, []),
    "neural_get_error_message": (ctypes.c_char_p, [_i]),
    # tensors
    "neural_tensor_create": (_vp, [_u64p, _u64, _i]),
    "neural_tensor_zeros": (_vp, [_u64p, _u64, _i]),
    "neural_tensor_ones": (_vp, [_u64p, _u64, _i]),
    "neural_tensor_from_data": (_vp, [_vp, _u64p, _u64, _i]),
    "neural_tensor_from_buffer": (_vp, [_vp, _u64p, _u64, _i, _i64p]),
    "neural_tensor_stride": (_i64p, [_vp]),
    "neural_tensor_is_contiguous": (_i, [_vp]),
    "neural_tensor_make_contiguous": (_vp, [_vp]),
    "neural_buffer_info": (_i, [_vp, ctypes.POINTER(NeuralBufferInfo)]),
    "neural_tensor_free": (None, [_vp]),
    "neural_tensor_data": (_vp, [_vp]),
    "neural_tensor_ndim": (_u64, [_vp]),
    "neural_tensor_shape": (_u64p, [_vp]),
    "neural_tensor_numel": (_u64, [_vp]),
    "neural_tensor_dtype": (_i, [_vp]),
    "neural_tensor_bytes": (_u64, [_vp]),
    "neural_tensor_fill": (_i, [_vp, _d]),
    "neural_tensor_copy": (_i, [_vp, _vp]),
    "neural_tensor_reshape": (_vp, [_vp, _u64p, _u64]),
    "neural_tensor_upload": (_i, [_vp, _vp, _u64]),
    "neural_tensor_download": (_i, [_vp, _vp, _u64]),
    "neural_tensor_device_data": (_vp, [_vp]),
    # elementwise
    "neural_add": (_i, [_vp, _vp, _vp]),
    "neural_sub": (_i, [_vp, _vp, _vp]),
    "neural_mul": (_i, [_vp, _vp, _vp]),
    "neural_div": (_i, [_vp, _vp, _vp]),
    "neural_maximum": (_i, [_vp, _vp, _vp]),
    "neural_scalar_add": (_i, [_vp, _vp, _d]),
    "neural_scalar_mul": (_i, [_vp, _vp, _d]),
    "neural_neg": (_i, [_vp, _vp]),
    "neural_bias_add": (_i, [_vp, _vp, _vp]),
    "neural_add_relu": (_i, [_vp, _vp, _vp]),
    "neural_bias_add_act": (_i, [_vp, _vp, _vp, _i, _d]),
    "vec_add_relu_fusion": (None, [_vp, _vp, _vp, _i64]),
    "simd_add_f32": (_i, [_vp, _vp, _vp, _u64]),
    "simd_mul_f32": (_i, [_vp, _vp, _vp, _u64]),
    "simd_fma_f32": (_i, [_vp, _vp, _vp, _vp, _u64]),
    "simd_dot_f32": (_f, [_vp, _vp, _u64]),
    "simd_sum_f32": (_f, [_vp, _u64]),
    # reductions
    "neural_sum": (_i, [_vp, _dp]),
    "neural_mean": (_i, [_vp, _dp]),
    "neural_max": (_i, [_vp, _dp]),
    "neural_argmax": (_i, [_vp, _i64p]),
    "neural_reduce_sum": (_i, [_vp, _i64, _vp]),
    "neural_reduce_mean": (_i, [_vp, _i64, _vp]),
    "neural_reduce_max": (_i, [_vp, _i64, _vp]),
    "neural_reduce_argmax": (_i, [_vp, _i64, _vp]),
    "neural_row_stats": (_i, [_vp, _vp, _vp, _vp, _vp]),
    "neural_bias_add_row_stats": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    # activations
    "neural_relu": (_i, [_vp, _vp]),
    "neural_sigmoid": (_i, [_vp, _vp]),
    "neural_tanh": (_i, [_vp, _vp]),
    "neural_softmax": (_i, [_vp, _vp]),
    "neural_log_softmax": (_i, [_vp, _vp]),
    "neural_gelu": (_i, [_vp, _vp]),
    "neural_leaky_relu": (_i, [_vp, _vp, _d]),
    "neural_elu": (_i, [_vp, _vp, _d]),
    "neural_selu": (_i, [_vp, _vp]),
    "neural_swish": (_i, [_vp, _vp]),
    "neural_mish": (_i, [_vp, _vp]),
    "neural_hardswish": (_i, [_vp, _vp]),
    "neural_softplus": (_i, [_vp, _vp]),
    "neural_hardtanh": (_i, [_vp, _vp]),
    "act_tanh": (_i, [_vp, _vp]),
    "act_gelu": (_i, [_vp, _vp]),
    "act_leaky_relu": (_i, [_vp, _vp, _d]),
    "act_elu": (_i, [_vp, _vp, _d]),
    "act_selu": (_i, [_vp, _vp]),
    "act_swish": (_i, [_vp, _vp]),
    "act_mish": (_i, [_vp, _vp]),
    "act_hardswish": (_i, [_vp, _vp]),
    "act_softplus": (_i, [_vp, _vp]),
    "act_hardtanh": (_i, [_vp, _vp]),
    # optimizers
    "opt_sgd_create": (_vp, [_d, _d]),
    "opt_adam_create": (_vp, [_d, _d, _d, _d]),
    "opt_adamw_create": (_vp, [_d, _d, _d, _d, _d]),
    "opt_step": (_i, [_vp, ctypes.POINTER(_vp), ctypes.POINTER(_vp), _i64]),
    "opt_free": (None, [_vp]),
    "opt_get_lr": (_d, [_vp]),
    "opt_set_lr": (None, [_vp, _d]),
    "opt_state_bytes": (_i64, [_vp]),
    "opt_state_export": (_i, [_vp, _vp, _i64]),
    "opt_state_import": (_i, [_vp, _vp, _i64]),
    "neural_clip_grad_norm": (_i, [_vp, _d]),
    "neural_clip_grad_value": (_i, [_vp, _d, _d]),
    "neural_clip_grad_norm_list": (_i, [ctypes.POINTER(_vp), _i64, _d, _dp]),
    "neural_clip_grad_value_list": (_i, [ctypes.POINTER(_vp), _i64, _d, _d]),
    # quantization
    "calibrate_minmax": (_i, [_vp, _i64, _i, _qp]),
    "quantized_matmul": (_i, [_vp, _vp, _vp, _i64, _i64, _i64, _qp, _qp]),
    "calibrate_percentile": (_i, [_vp, _i64, _d, _i, _qp]),
    "quantize_tensor": (_i, [_vp, _vp, _i64, _qp]),
    "dequantize_tensor": (_i, [_vp, _vp, _i64, _qp]),
    "quantization_error": (_d, [_vp, _i64, _qp]),
    "quantization_snr": (_d, [_vp, _i64, _qp]),
    "calibrate_minmax_f32": (_i, [_vp, _i64, _i, _qp]),
    "quantize_tensor_f32": (_i, [_vp, _vp, _i64, _qp]),
    "dequantize_tensor_f32": (_i, [_vp, _vp, _i64, _qp]),
    "quantization_error_f32": (_d, [_vp, _i64, _qp]),
    "quantization_snr_f32": (_d, [_vp, _i64, _qp]),
    "calibrate_minmax_f32_dev": (_i, [_vp, _i64, _i, _vp]),
    "calibrate_minmax_f32_dev_noalloc": (_i, [_vp, _i64, _i, _vp]),
    "quantize_tensor_f32_dev": (_i, [_vp, _vp, _i64, _vp]),
    "dequantize_tensor_f32_dev": (_i, [_vp, _vp, _i64, _vp]),
    # training ops
    "neural_tensor_has_nan": (_i, [_vp, _u64]),
    "neural_tensor_has_inf": (_i, [_vp, _u64]),
    "neural_tensor_grad_l2_norm": (_f, [_vp, _u64]),
    "neural_scan_nan_inf_l2": (_i, [_vp, _u64, _ip, _ip, _dp]),
    "neural_tensor_scan": (_i, [_vp, _ip, _ip, _dp]),
    # per-feature transforms
    "transform_compute_stats": (_i, [_vp, _i64, _i64, _vp, _vp, _vp, _vp]),
    "transform_normalize": (_i, [_vp, _vp, _i64, _i64, _vp, _vp, _d]),
    "transform_unnormalize": (_i, [_vp, _vp, _i64, _i64, _vp, _vp, _d]),
    "transform_minmax": (_i, [_vp, _vp, _i64, _i64, _vp, _vp, _d]),
    "neural_dropout_forward": (_i, [_vp, _vp, _vp, _u64, _f]),
    "neural_dropout_backward": (_i, [_vp, _vp, _vp, _u64, _f]),
    "neural_dropout_seed": (_i, [ctypes.c_uint32]),
    "neural_dropout_draws": (_u64, []),
    # tensor ops
    "tensor_concat_2d": (_i, [_vp, _vp, _i64, _i64, _i64, _i64, _i64, _vp, _i64p, _i64p]),
    "tensor_split_2d": (_i, [_vp, _i64, _i64, _i64, _i64, _vp, _vp, _i64p, _i64p, _i64p, _i64p]),
    "tensor_pad_2d": (_i, [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _d, _vp, _i64p, _i64p]),
    "tensor_transpose2d_array": (_i, [_vp, _i64, _i64, _vp]),
    # cross-entropy losses
    "label_smoothing_ce_forward": (_i, [_vp, _vp, _i64, _i64, _d, _dp]),
    "label_smoothing_ce_backward": (_i, [_vp, _vp, _i64, _i64, _d, _vp]),
    "label_smoothing_ce_fused": (_i, [_vp, _vp, _i64, _i64, _d, _dp, _vp]),
    "label_smoothing_ce_fused_f32": (_i, [_vp, _vp, _i64, _i64, _d, _dp, _vp]),
    "label_smoothing_ce_forward_dev": (_i, [_vp, _vp, _i64, _i64, _d, _vp]),
    "label_smoothing_ce_fused_dev": (_i, [_vp, _vp, _i64, _i64, _d, _vp, _vp]),
    "label_smoothing_ce_fused_f32_dev": (_i, [_vp, _vp, _i64, _i64, _d, _vp, _vp]),
    "neural_cross_entropy_loss": (_i, [_vp, _vp, _dp]),
    # HIP runtime controls
    "neural_hip_set_stream": (_i, [_vp]),
    "neural_hip_time_next_launch": (_i, [_vp, _vp, _i]),
    "neural_hip_time_launches": (_i, [_vp, _vp, _i, _i]),
    "neural_hip_launch_count": (ctypes.c_ulonglong, []),
    "neural_hip_alloc_stats": (_i, [ctypes.POINTER(ctypes.c_ulonglong), ctypes.POINTER(ctypes.c_ulonglong)]),
    "neural_hip_stream_copy": (_i, [_vp, _vp, _u64]),
    "neural_hip_time_cancel": (_i, []),
    "neural_hip_reset_stream": (_i, []),
    "neural_hip_get_stream": (_vp, []),
    "neural_hip_synchronize": (_i, []),
    "neural_hip_empty_cache": (_i, []),
    "neural_hip_device_info": (_i, [_ip, _ip, ctypes.c_char_p, _i]),
}

for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(_lib, _name)  # AttributeError here means a stale library build
    _fn.restype = _res
    _fn.argtypes = _args


def _check_error(result: int, operation: str = "operation"):
    """Raise NeuralException for a nonzero code (core.py:1376-1379)."""
    if result != NeuralError.OK:
        raise NeuralException(result, f"{operation} failed")


_initialized = False


def init() -> None:
    """Initialise the runtime (device, stream, workspaces)."""
    global _initialized
    if _initialized:
        return
    rc = _lib.neural_init()
    if rc != NeuralError.OK:
        raise NeuralException(rc, "failed to initialise the HIP runtime (no GPU visible?)")
    _initialized = True


def shutdown() -> None:
    global _initialized
    if _initialized:
        _lib.neural_shutdown()
        _initialized = False


def version() -> str:
    return _lib.neural_version().decode("utf-8")


def get_last_error() -> int:
    return _lib.neural_get_last_error()


def get_error_message(error_code: int) -> str:
    msg = _lib.neural_get_error_message(error_code)
    return msg.decode("utf-8") if msg else f"Unknown error ({error_code})"


def clear_error() -> None:
    _lib.neural_clear_error()


def set_stream(stream_handle) -> None:
    """Launch on an existing HIP stream: an int handle such as torch's
    ``torch.cuda.current_stream().cuda_stream`` (0 is the HIP null stream,
    torch's default); ``None`` returns to the library's own stream."""
    if stream_handle is None:
        _check_error(_lib.neural_hip_reset_stream(), "reset_stream")
    else:
        _check_error(_lib.neural_hip_set_stream(ctypes.c_void_p(stream_handle)), "set_stream")


def synchronize() -> None:
    _check_error(_lib.neural_hip_synchronize(), "synchronize")


def device_info() -> dict:
    ordinal, cus = ctypes.c_int(), ctypes.c_int()
    name = ctypes.create_string_buffer(256)
    _check_error(_lib.neural_hip_device_info(ctypes.byref(ordinal), ctypes.byref(cus), name, 256), "device_info")
    return {"ordinal": ordinal.value, "num_cus": cus.value, "arch": name.value.decode()}


# The reference initialises on import and swallows failures (core.py:1454-1458);
# later calls then report the init error code.
try:
    init()
except Exception:
    pass
