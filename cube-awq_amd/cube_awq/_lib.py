"""ctypes binding of libcube_awq_gfx950.so (the C ABI declared in include/awq.h).

torch is imported first on purpose: torch ships its own libamdhip64.so with the
soname libamdhip64.so.7, and loading it before this library makes the dynamic
loader bind our DT_NEEDED libamdhip64.so.7 to that same runtime, so device
pointers and streams from torch are valid here. Loading the library first
would put two HIP runtimes in one process.
"""
import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(_HERE)
LIB_PATH = os.path.join(PKG_ROOT, "lib", "libcube_awq_gfx950.so")

# awq_dtype
AWQ_F32, AWQ_F16, AWQ_BF16, AWQ_U32, AWQ_I32, AWQ_I16, AWQ_I64 = range(7)
# awq_order
AWQ_ORDER_AUTOAWQ, AWQ_ORDER_SEQUENTIAL = 0, 1
# status codes
AWQ_OK, AWQ_ERR_INVALID, AWQ_ERR_HIP, AWQ_ERR_UNSUPPORTED = 0, -1, -2, -3


class AwqShapeConfig(ctypes.Structure):
    _fields_ = [
        ("m", ctypes.c_int64),
        ("k", ctypes.c_int64),
        ("n", ctypes.c_int64),
        ("tile_m", ctypes.c_int64),
        ("tile_n", ctypes.c_int64),
        ("inner_k", ctypes.c_int64),
        ("line_size", ctypes.c_int64),
        ("m_valid", ctypes.c_int64),
    ]


class AwqTensorRef(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("shape", ctypes.POINTER(ctypes.c_int64)),
        ("rank", ctypes.c_int32),
        ("elem_size", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
    ]


# Every function include/awq.h declares, with its ctypes signature.
_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_SC = ctypes.POINTER(AwqShapeConfig)
_TR = ctypes.POINTER(AwqTensorRef)
SIGNATURES = {
    "awq_shape_config_new": (AwqShapeConfig, [_I64] * 6),
    "awq_shape_config_new_with_valid_m": (AwqShapeConfig, [_I64] * 7),
    "awq_validate_launch_params": (ctypes.c_int, [_SC, _I64]),
    "awq_validate_decode_launch_params": (ctypes.c_int, [_SC, _I64]),
    "awq_gemm_linear": (ctypes.c_int, [_TR, _TR, _TR, _TR, _TR, _SC, _I64, _P]),
    "awq_dequantize_native": (ctypes.c_int, [_TR, _TR, _TR, _TR, _I64, _P]),
    "awq_gemm": (ctypes.c_int, [_P, _I32, _P, _P, _P, _I32, _P, _I32, _P, _I32,
                                _I64, _I64, _I64, _I64, _P]),
    "awq_dequantize": (ctypes.c_int, [_P, _P, _P, _I32, _P, _I32, _I64, _I64, _I64, _I32, _P]),
    "awq_validate_gemm": (ctypes.c_int, [_I64, _I64, _I64, _I64]),
    "awq_gemm_ordered": (ctypes.c_int, [_P, _I32, _P, _P, _P, _I32, _P, _I32, _P, _I32,
                                        _I64, _I64, _I64, _I64, _I32, _P]),
    "awq_gemm_noalloc": (ctypes.c_int, [_P, _I32, _P, _P, _P, _I32, _P, _I32, _P, _I32,
                                        _I64, _I64, _I64, _I64, _P]),
    "awq_gemm_silu_mul": (ctypes.c_int, [_P, _I32, _P, _P, _P, _I32, _P, _I32, _P, _I32,
                                         _I64, _I64, _I64, _I64, _P]),
    "awq_select_tile_m": (ctypes.c_int64, [_I64]),
    "awq_select_tile_n": (ctypes.c_int64, [_I64]),
    "awq_decode_m_threshold": (ctypes.c_int64, []),
    "awq_tuning_reload": (None, []),
    "awq_last_error": (ctypes.c_char_p, []),
    "awq_version": (ctypes.c_int32, []),
}

_lib = None


def lib():
    """Load (once) and return the library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it first (python -c "
                f"'import __graft_entry__ as g; g.build()' from the repository root)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


class Panic(RuntimeError):
    """A failed reference assertion (the Rust crate panics with this text)."""


class HipError(RuntimeError):
    """A HIP runtime / launch failure reported by the library."""


def check(rc):
    if rc == AWQ_OK:
        return
    msg = lib().awq_last_error().decode("utf-8", "replace")
    if rc == AWQ_ERR_INVALID:
        raise Panic(msg)
    raise HipError(msg)


_TORCH_TO_AWQ = {
    torch.float32: AWQ_F32,
    torch.float16: AWQ_F16,
    torch.bfloat16: AWQ_BF16,
    torch.uint32: AWQ_U32,
    torch.int32: AWQ_I32,
    torch.int16: AWQ_I16,
    torch.int64: AWQ_I64,
}


def awq_dtype(t):
    try:
        return _TORCH_TO_AWQ[t.dtype]
    except KeyError:
        raise Panic(f"unsupported tensor dtype {t.dtype}") from None


def tensor_ref(t):
    """AwqTensorRef of a contiguous tensor; keeps the shape array alive."""
    if not t.is_contiguous():
        raise Panic("tensors passed to the AWQ library must be contiguous")
    shape = (ctypes.c_int64 * max(t.dim(), 1))(*t.shape)
    ref = AwqTensorRef(t.data_ptr(), ctypes.cast(shape, ctypes.POINTER(ctypes.c_int64)),
                       t.dim(), t.element_size(), awq_dtype(t))
    ref._shape_keepalive = shape
    return ref


def stream_ptr(stream=None, device=None):
    """Raw hipStream_t of `stream` (default: torch's current stream)."""
    if stream is None:
        if not torch.cuda.is_available():
            return None
        stream = torch.cuda.current_stream(device)
    return ctypes.c_void_p(stream.cuda_stream)
