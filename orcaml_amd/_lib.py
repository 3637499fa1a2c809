"""ctypes binding of liborca_hip.so (the C ABI declared in include/orca_hip.h).

There is no fallback: if the library is missing or fails to load, every entry
point raises, so nothing can silently run on the CPU.
"""
from __future__ import annotations

import ctypes
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "liborca_hip.so")

# Status codes (orca-core/src/error.rs:5-31 variants).
OK = 0
ERR_SHAPE = -1
ERR_UNSUPPORTED_DTYPE = -2
ERR_DTYPE_MISMATCH = -3
ERR_DEVICE_MISMATCH = -4
ERR_INTERNAL = -5
ERROR_NAMES = {
    ERR_SHAPE: "ShapeMismatch",
    ERR_UNSUPPORTED_DTYPE: "UnsupportedDType",
    ERR_DTYPE_MISMATCH: "DTypeMismatch",
    ERR_DEVICE_MISMATCH: "DeviceMismatch",
    ERR_INTERNAL: "InternalError",
}

# DType codes in orca_core::DType order (orca-core/src/dtype.rs:5-22).
F32, F64, F16, BF16, I32, I64, U8, BOOL = range(8)

VIEW_CONTIGUOUS = 0
VIEW_TRANSPOSED = 1

EPI_NONE, EPI_BIAS, EPI_BIAS_RELU, EPI_RELU_MASK, EPI_BIAS_RELU_PRE, EPI_RELU_MASK_PRE = range(6)

# Elementwise program opcodes and interpreter limits (include/orca_hip.h ORCA_HIP_EW_*).
EW_ADD, EW_SUB, EW_MUL, EW_DIV, EW_MUL_SCALAR, EW_RELU, EW_RELU_BW, EW_EXP, EW_LOG, EW_SQRT = range(10)
EW_SIGMOID, EW_EXP_BW, EW_LOG_BW, EW_SQRT_BW, EW_SIGMOID_BW, EW_DIV_BW_RHS, EW_SUM_VISIT, EW_MAX_VISIT = range(10, 18)
EW_COPY, EW_ADD_SCALAR = 18, 19
EW_MAX_INPUTS, EW_MAX_OUTPUTS, EW_MAX_OPS, EW_MAX_REGS = 8, 8, 64, 16


class EwInput(ctypes.Structure):
    """orca_hip_ew_input: element e of a program reads ptr[(e / div) % mod]."""
    _fields_ = [("ptr", ctypes.c_void_p), ("div", ctypes.c_uint64), ("mod", ctypes.c_uint64)]


class OrcaHipError(ValueError):
    """A failed C-ABI call; `.code` is the ORCA_HIP_ERR_* status and `.fields` the OrcaError
    variant's fields (orca_hip_last_error_info: op, expected, got, dtype, dtype_got, devices).
    It is a ValueError because orca-python maps every OrcaError to ValueError
    (orca-python/src/lib.rs:124,128)."""

    def __init__(self, code: int, message: str, fields: dict | None = None):
        super().__init__(f"{ERROR_NAMES.get(code, code)}: {message}")
        self.code = code
        self.fields = fields or {}


class Epilogue(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int),
        ("bias", ctypes.c_void_p),
        ("mask", ctypes.c_void_p),
        ("ldmask", ctypes.c_size_t),
        ("colsum", ctypes.c_void_p),
        ("pre", ctypes.c_void_p),
        ("done", ctypes.POINTER(ctypes.c_void_p)),
    ]


class Optim(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int),
        ("lr", ctypes.c_double),
        ("weight_decay", ctypes.c_double),
        ("beta1", ctypes.c_double),
        ("beta2", ctypes.c_double),
        ("eps", ctypes.c_double),
    ]


class BackendOptions(ctypes.Structure):
    """orca_hip_backend_options."""
    _fields_ = [("lazy", ctypes.c_int), ("deferred", ctypes.c_int), ("fold", ctypes.c_int), ("overlap", ctypes.c_int),
                ("side_frac", ctypes.c_double), ("side_bpc", ctypes.c_int)]


class OptRow(ctypes.Structure):
    """orca_hip_opt_row: storage handles of one parameter's optimizer update."""
    _fields_ = [("p_src", ctypes.c_void_p), ("p_dst", ctypes.c_void_p), ("g", ctypes.c_void_p),
                ("m", ctypes.c_void_p), ("v", ctypes.c_void_p), ("n", ctypes.c_size_t)]


class ErrorInfo(ctypes.Structure):
    """orca_hip_error_info: the last failure as its OrcaError variant's fields."""
    _fields_ = [("code", ctypes.c_int), ("op", ctypes.c_char_p), ("expected", ctypes.c_char_p),
                ("got", ctypes.c_char_p), ("dtype", ctypes.c_int), ("dtype_got", ctypes.c_int),
                ("device_kind", ctypes.c_int * 2), ("device_index", ctypes.c_int * 2), ("message", ctypes.c_char_p)]


_P = ctypes.c_void_p
_PP = ctypes.POINTER(ctypes.c_void_p)
_SZ = ctypes.c_size_t
_SZP = ctypes.POINTER(ctypes.c_size_t)
_I = ctypes.c_int
_F = ctypes.c_float
_D = ctypes.c_double

_EW1 = [_P, _P, _SZP, _SZ, _I, _PP]
_EW2 = [_P, _P, _P, _SZP, _SZ, _I, _PP]
_RESHAPE = [_P, _P, _SZP, _SZ, _SZP, _SZ, _I, _PP]

_TB = [_P, _P, _P, _SZP, _SZ, _I, _PP]  # trait binary: backend, lhs, rhs, shape, rank, dtype, out
_TU = [_P, _P, _SZP, _SZ, _I, _PP]  # trait unary
_TR = [_P, _P, _SZP, _SZ, _SZP, _SZ, _I, _PP]  # trait reshape-like
_TIDX = [_P, _P, _SZ, _P, _SZP, _SZ, _SZP, _SZ, _I, _PP]  # gather / scatter backward

SIGNATURES = {
    "orca_hip_last_error_info": [ctypes.POINTER(ErrorInfo)],
    "orca_hip_backend_default_options": [ctypes.POINTER(BackendOptions)],
    "orca_hip_backend_create": [_P, ctypes.POINTER(BackendOptions), _PP],
    "orca_hip_backend_destroy": [_P],
    "orca_hip_storage_retain": [_P],
    "orca_hip_storage_release": [_P],
    "orca_hip_storage_len": [_P, _SZP],
    "orca_hip_storage_flags": [_P, ctypes.POINTER(ctypes.c_uint32)],
    "orca_hip_storage_device_ptr": [_P, _P, _PP],
    "orca_hip_trait_device": [_P, ctypes.POINTER(_I), ctypes.POINTER(_I)],
    "orca_hip_trait_zeros": [_P, _SZP, _SZ, _I, _PP],
    "orca_hip_trait_from_f32_slice": [_P, _SZP, _SZ, _P, _SZ, _PP],
    "orca_hip_trait_to_f32_vec": [_P, _P, _P, _SZ],
    "orca_hip_trait_matmul": [_P, _P, _P, _SZP, _SZ, _SZP, _SZ, _I, _PP],
    "orca_hip_trait_transpose": [_P, _P, _SZP, _SZ, _SZ, _SZ, _I, _PP],
    "orca_hip_trait_add": _TB,
    "orca_hip_trait_sub": _TB,
    "orca_hip_trait_mul_scalar": [_P, _P, _F, _SZP, _SZ, _I, _PP],
    "orca_hip_trait_mul": _TB,
    "orca_hip_trait_relu": _TU,
    "orca_hip_trait_sigmoid": _TU,
    "orca_hip_trait_relu_backward": _TB,
    "orca_hip_trait_sigmoid_backward": _TB,
    "orca_hip_trait_expand": _TR,
    "orca_hip_trait_sum_to_shape": _TR,
    "orca_hip_trait_reshape": _TR,
    "orca_hip_trait_exp": _TU,
    "orca_hip_trait_log": _TU,
    "orca_hip_trait_exp_backward": _TB,
    "orca_hip_trait_log_backward": _TB,
    "orca_hip_trait_div": _TB,
    "orca_hip_trait_sqrt": _TU,
    "orca_hip_trait_div_backward_lhs": _TB,
    "orca_hip_trait_div_backward_rhs": [_P, _P, _P, _P, _SZP, _SZ, _I, _PP],
    "orca_hip_trait_sqrt_backward": _TB,
    "orca_hip_trait_accumulate_grad": [_P, _P, _P, _PP],
    "orca_hip_trait_conv2d": [_P, _P, _P, _P, _SZP, _SZ, _SZP, _SZ, _SZ, _SZ, _SZ, _SZ, _I, _PP],
    "orca_hip_trait_conv2d_backward_input": [_P, _P, _P, _SZP, _SZ, _SZP, _SZ, _SZ, _SZ, _SZ, _SZ, _I, _PP],
    "orca_hip_trait_conv2d_backward_weight": [_P, _P, _P, _SZP, _SZ, _SZP, _SZ, _SZ, _SZ, _SZ, _SZ, _I, _PP],
    "orca_hip_trait_conv2d_backward_bias": [_P, _P, _SZP, _SZ, _I, _PP],
    "orca_hip_trait_cast": [_P, _P, _SZP, _SZ, _I, _I, _PP],
    "orca_hip_trait_scatter": [_P, _P, _SZ, _P, _P, _SZP, _SZ, _SZP, _SZ, _I, _PP],
    "orca_hip_trait_gather": [_P, _P, _SZ, _P, _SZP, _SZ, _SZP, _SZ, _I, _PP],
    "orca_hip_trait_scatter_backward_src": _TIDX,
    "orca_hip_trait_scatter_backward_base": _TIDX,
    "orca_hip_trait_gather_backward": _TIDX,
    "orca_hip_trait_from_bytes": [_P, _SZP, _SZ, _P, _SZ, _I, _PP],
    "orca_hip_trait_to_bytes": [_P, _P, _P, _SZ],
    "orca_hip_trait_has_nan_or_inf": [_P, _P, _I, ctypes.POINTER(_I)],
    "orca_hip_trait_max_to_shape": _TR,
    "orca_hip_trait_max_to_shape_backward": [_P, _P, _P, _P, _SZP, _SZ, _SZP, _SZ, _I, _PP],
    "orca_hip_be_softmax_ce": [_P, _P, _P, _SZ, _SZ, _I, _PP, _PP],
    "orca_hip_be_clone": [_P, _P, _PP],
    "orca_hip_be_arena": [_P, _SZ, _I, _F, _PP],
    "orca_hip_be_view": [_P, _P, _SZ, _SZ, _PP],
    "orca_hip_be_copy_into": [_P, _P, _P],
    "orca_hip_be_arena_exclusive": [_P, _P, ctypes.POINTER(_I)],
    "orca_hip_be_adamw_multi": [_P, ctypes.POINTER(OptRow), _SZ, _D, _D, _D, _D, _D, ctypes.c_int64],
    "orca_hip_be_sgd_multi": [_P, ctypes.POINTER(OptRow), _SZ, _D],
    "orca_hip_be_adamw_step": [_P, _P, _P, _P, _P, _SZ, _D, _D, _D, _D, _D, ctypes.c_int64],
    "orca_hip_be_sgd_step": [_P, _P, _P, _SZ, _D],
    "orca_hip_ctx_create": [_I, ctypes.POINTER(_P)],
    "orca_hip_ctx_destroy": [_P],
    "orca_hip_device": [_P, ctypes.POINTER(_I)],
    "orca_hip_alloc": [_P, _SZ, _PP],
    "orca_hip_free": [_P, _P],
    "orca_hip_free_many": [_P, _P, _SZ],
    "orca_hip_empty_cache": [_P],
    "orca_hip_mem_stats": [_P, _SZP, _SZP, _SZP],
    "orca_hip_h2d": [_P, _P, _P, _SZ],
    "orca_hip_d2h": [_P, _P, _P, _SZ],
    "orca_hip_d2d": [_P, _P, _P, _SZ],
    "orca_hip_fill": [_P, _P, _F, _SZ],
    "orca_hip_sync": [_P],
    "orca_hip_use_side_stream": [_P, ctypes.c_int],
    "orca_hip_event_record": [_P, ctypes.POINTER(ctypes.c_void_p)],
    "orca_hip_event_wait": [_P, _P],
    "orca_hip_event_release": [_P, _P],
    "orca_hip_sync_count": [_P, ctypes.POINTER(ctypes.c_uint64)],
    "orca_hip_zeros": [_P, _SZP, _SZ, _I, _PP],
    "orca_hip_from_f32_slice": [_P, _SZP, _SZ, _P, _SZ, _PP],
    "orca_hip_to_f32_vec": [_P, _P, _SZ, _P],
    "orca_hip_from_bytes": [_P, _SZP, _SZ, _P, _SZ, _I, _PP],
    "orca_hip_to_bytes": [_P, _P, _SZ, _P],
    "orca_hip_matmul": [_P, _P, _P, _SZP, _SZ, _SZP, _SZ, _I, _I, _I, _PP],
    "orca_hip_matmul_colsum": [_P, _P, _P, _SZ, _SZ, _SZ, _I, _I, _P, _PP],
    "orca_hip_matmul_ev": [_P, _P, _P, _SZ, _SZ, _SZ, _I, _I, _I, _P, _PP, _PP],
    "orca_hip_transpose": [_P, _P, _SZP, _SZ, _SZ, _SZ, _I, _PP],
    "orca_hip_add": _EW2,
    "orca_hip_sub": _EW2,
    "orca_hip_mul": _EW2,
    "orca_hip_div": _EW2,
    "orca_hip_mul_scalar": [_P, _P, _F, _SZP, _SZ, _I, _PP],
    "orca_hip_relu": _EW1,
    "orca_hip_sigmoid": _EW1,
    "orca_hip_exp": _EW1,
    "orca_hip_log": _EW1,
    "orca_hip_sqrt": _EW1,
    "orca_hip_relu_backward": _EW2,
    "orca_hip_sigmoid_backward": _EW2,
    "orca_hip_exp_backward": _EW2,
    "orca_hip_log_backward": _EW2,
    "orca_hip_sqrt_backward": _EW2,
    "orca_hip_div_backward_lhs": _EW2,
    "orca_hip_div_backward_rhs": [_P, _P, _P, _P, _SZP, _SZ, _I, _PP],
    "orca_hip_accumulate_grad": [_P, _P, _P, _SZ, _PP],
    "orca_hip_expand": _RESHAPE,
    "orca_hip_sum_to_shape": _RESHAPE,
    "orca_hip_reshape": _RESHAPE,
    "orca_hip_max_to_shape": _RESHAPE,
    "orca_hip_max_to_shape_backward": [_P, _P, _P, _P, _SZP, _SZ, _SZP, _SZ, _I, _PP],
    "orca_hip_has_nan_or_inf": [_P, _P, _SZ, _I, ctypes.POINTER(_I)],
    "orca_hip_gemm": [_P, _I, _I, _SZ, _SZ, _SZ, _P, _SZ, _P, _SZ, _P, _SZ, ctypes.POINTER(Epilogue)],
    "orca_hip_narrow_linear_backward": [_P, _P, _SZ, _SZ, _P, _SZ, _P, _P, _P, _P, _P, _P, _PP],
    "orca_hip_softmax_ce": [_P, _P, _SZ, _SZ, _P, _P, _P, _P, _P, _P],
    "orca_hip_head_forward_ce": [_P, _P, _SZ, _SZ, _P, _P, _SZ, _P, _P, _P, _P, _P, _P, _P],
    "orca_hip_head_backward": [_P, _P, _SZ, _SZ, _P, _SZ, _P, _I, _P, _P, _P],
    "orca_hip_ew_program": [_P, _SZ, _P, _SZ, _P, _P, _SZ, _P, _SZ, _SZ],
    "orca_hip_ew_program_rows": [_P, _SZ, _SZ, _P, _SZ, _P, _P, _SZ, _P, _SZ, _SZ, _I, _I, _P],
    "orca_hip_ew_set_jit": [_P, ctypes.c_int],
    "orca_hip_adamw_multi": [_P, _P, _SZ, ctypes.c_double, ctypes.c_double, ctypes.c_double, ctypes.c_double,
                             ctypes.c_double, ctypes.c_int64],
    "orca_hip_sgd_multi": [_P, _P, _SZ, ctypes.c_double],
    "orca_hip_ew_jit_stats": [_P, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64),
                              ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)],
    "orca_hip_ew_jit_source": [_SZ, _P, _SZ, _P, _SZ, _P, _SZ, _SZ, ctypes.c_char_p, _SZ, ctypes.POINTER(_SZ)],
    "orca_hip_ew_jit_headers": [ctypes.POINTER(ctypes.c_char_p)],
    "orca_hip_relu_bw_colsum": [_P, _P, _P, _SZ, _SZ, _P, _P],
    "orca_hip_relu_bw_colsum_noalloc": [_P, _P, _P, _SZ, _SZ, _P, _P],
    "orca_hip_adamw_step": [_P, _P, _P, _P, _P, _SZ, _D, _D, _D, _D, _D, ctypes.c_int64],
    "orca_hip_sgd_step": [_P, _P, _P, _SZ, _D],
    "orca_hip_mlp_create": [_P, _SZP, _SZ, _SZ, ctypes.POINTER(Optim), ctypes.POINTER(_P)],
    "orca_hip_mlp_destroy": [_P],
    "orca_hip_mlp_param_numel": [_P, _SZ, _SZP],
    "orca_hip_mlp_set_param": [_P, _SZ, _P, _SZ],
    "orca_hip_mlp_get_param": [_P, _SZ, _P, _SZ],
    "orca_hip_mlp_get_grad": [_P, _SZ, _P, _SZ],
    "orca_hip_mlp_get_moment": [_P, _I, _SZ, _P, _SZ],
    "orca_hip_mlp_set_moment": [_P, _I, _SZ, _P, _SZ],
    "orca_hip_mlp_set_batch": [_P, _P, _P, _P],
    "orca_hip_mlp_batch_ptrs": [_P, _PP, _PP],
    "orca_hip_mlp_step": [_P],
    "orca_hip_mlp_read_metrics": [_P, ctypes.POINTER(_F), ctypes.POINTER(ctypes.c_int64)],
    "orca_hip_mlp_get_logits": [_P, _P, _SZ],
    "orca_hip_mlp_get_preds": [_P, _P, _SZ],
    "orca_hip_mlp_get_activation": [_P, _SZ, _P, _SZ],
    "orca_hip_mlp_get_step_count": [_P, ctypes.POINTER(ctypes.c_int64)],
    "orca_hip_mlp_set_step_count": [_P, ctypes.c_int64],
    "orca_hip_mlp_set_update_shard": [_P, _SZ, _SZ],
    "orca_hip_prof_enable": [_P, _I],
    "orca_hip_prof_reset": [_P],
    "orca_hip_prof_report": [_P, ctypes.c_char_p, _SZ],
    "orca_hip_timer_start": [_P],
    "orca_hip_timer_stop": [_P, ctypes.POINTER(_F)],
}

_lib = None


def load() -> ctypes.CDLL:
    """Loads liborca_hip.so; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -m orcaml_amd.build` (the HIP backend has no CPU fallback)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    lib.orca_hip_last_error.argtypes = []
    lib.orca_hip_last_error.restype = ctypes.c_char_p
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != OK:
        lib = load()
        info = ErrorInfo()
        fields = {}
        if lib.orca_hip_last_error_info(ctypes.byref(info)) == OK:
            fields = dict(op=(info.op or b"").decode(), expected=(info.expected or b"").decode(),
                          got=(info.got or b"").decode(), dtype=info.dtype, dtype_got=info.dtype_got,
                          devices=[(info.device_kind[i], info.device_index[i]) for i in range(2)])
        msg = lib.orca_hip_last_error()
        raise OrcaHipError(rc, msg.decode() if msg else "", fields)


_FNS: dict = {}


class OptSegment(ctypes.Structure):
    """orca_hip_opt_segment."""
    _fields_ = [("p_src", ctypes.c_void_p), ("p_dst", ctypes.c_void_p), ("g", ctypes.c_void_p),
                ("m", ctypes.c_void_p), ("v", ctypes.c_void_p), ("n", ctypes.c_size_t)]


OPT_MAX_SEGMENTS = 32


def call(name: str, *args) -> None:
    fn = _FNS.get(name)
    if fn is None:
        fn = _FNS[name] = getattr(load(), name)
    rc = fn(*args)
    if rc != OK:
        check(rc)


_DIMS: dict = {}


def dims(shape) -> tuple:
    """(size_t array, rank) of a shape.  The C side only reads the array, so one
    array per distinct shape is built and reused (ops see few distinct shapes)."""
    key = shape if type(shape) is tuple else tuple(shape)
    hit = _DIMS.get(key)
    if hit is not None:
        return hit
    dims_ = tuple(int(s) for s in key)
    hit = ((ctypes.c_size_t * max(1, len(dims_)))(*dims_), len(dims_))
    if len(_DIMS) >= 4096:
        _DIMS.clear()
    _DIMS[key] = hit
    return hit
