"""cube_awq -- MI355X (gfx950) AWQ INT4 dequant-GEMM and dequantize.

Host-side mirror of the reference crate's public surface (`cube_awq::kernel`
and `cube_awq::modules`) over the C ABI of libcube_awq_gfx950.so.
"""
from ._lib import HipError, LIB_PATH, Panic, lib  # noqa: F401
from .kernel import (  # noqa: F401
    DECODE_M_THRESHOLD, DECODE_TILE_M, ShapeConfig, awq_gemm_linear, dequantize_awq,
    dequantize_native, validate_decode_launch_params, validate_launch_params)
from .modules import (  # noqa: F401
    AWQGateUpSiLU, AWQGEMMLinear, AWQGEMMLinearConfig, AWQLinear, AWQLinearConfig)
from . import checkpoint, pack  # noqa: F401
