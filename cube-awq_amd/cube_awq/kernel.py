"""Kernel-level interface, mirroring the reference's `cube_awq::kernel` module.

Reference items mirrored here (paths relative to the reference root):
  ShapeConfig, DECODE_M_THRESHOLD, DECODE_TILE_M   src/kernel/awq_kernel_gemm.rs:35-87
  validate_launch_params(_decode)                 src/kernel/awq_kernel_gemm.rs:89-171
  awq_gemm_linear                                  src/kernel/awq_kernel_gemm.rs:626-771
  dequantize_native                                src/kernel/awq_kernel.rs:63-111
  dequantize_awq                                   src/kernel/mod.rs:9-51

Tensors are torch tensors used as device memory (contiguous, on the GPU for
anything that launches). Every check and every launch happens in the C++
library behind the C ABI; failed reference assertions raise `Panic` with the
reference's panic text.
"""
import ctypes

import torch

from . import _lib
from ._lib import Panic, check, lib, stream_ptr, tensor_ref

DECODE_M_THRESHOLD = 8
DECODE_TILE_M = 8


class ShapeConfig:
    """Mutable like the reference's (its tests poke `line_size` directly)."""

    __slots__ = ("m", "k", "n", "tile_m", "tile_n", "inner_k", "line_size", "m_valid")

    def __init__(self, m, n, k, m_tile_size, n_tile_size, inner_k_size, m_valid=None):
        # ShapeConfig::new(m, n, k, ...) -- note the m, n, k argument order.
        self.m = m
        self.k = k
        self.n = n
        self.tile_m = m_tile_size
        self.tile_n = n_tile_size
        self.inner_k = inner_k_size
        self.line_size = 4
        self.m_valid = m if m_valid is None else m_valid

    @classmethod
    def new(cls, m, n, k, m_tile_size, n_tile_size, inner_k_size):
        return cls(m, n, k, m_tile_size, n_tile_size, inner_k_size)

    @classmethod
    def new_with_valid_m(cls, m, n, k, m_tile_size, n_tile_size, inner_k_size, m_valid):
        return cls(m, n, k, m_tile_size, n_tile_size, inner_k_size, m_valid)

    def _c(self):
        return _lib.AwqShapeConfig(self.m, self.k, self.n, self.tile_m, self.tile_n,
                                   self.inner_k, self.line_size, self.m_valid)

    def __repr__(self):
        return ("ShapeConfig(m={m}, k={k}, n={n}, tile_m={tile_m}, tile_n={tile_n}, "
                "inner_k={inner_k}, line_size={line_size}, m_valid={m_valid})").format(
                    **{s: getattr(self, s) for s in self.__slots__})


def validate_launch_params(shape, group_size):
    c = shape._c()
    check(lib().awq_validate_launch_params(ctypes.byref(c), group_size))


def validate_decode_launch_params(shape, group_size):
    c = shape._c()
    check(lib().awq_validate_decode_launch_params(ctypes.byref(c), group_size))


def awq_gemm_linear(input, qweight, qzeros, scales, output, shape, group_size, stream=None):
    """output[.., M, N] = input[.., M, K] . dequant(qweight, qzeros, scales).

    Asynchronous on `stream` (default: torch's current stream)."""
    refs = [tensor_ref(t) for t in (input, qweight, qzeros, scales, output)]
    c = shape._c()
    check(lib().awq_gemm_linear(*[ctypes.byref(r) for r in refs], ctypes.byref(c), group_size,
                                stream_ptr(stream, _device_of(input))))


def dequantize_native(q_weight, q_zeros, q_scales, output, group_size, stream=None):
    """output[K, N] = (q - z) * s, sequential nibble order (bit-exact)."""
    refs = [tensor_ref(t) for t in (q_weight, q_zeros, q_scales, output)]
    check(lib().awq_dequantize_native(*[ctypes.byref(r) for r in refs], group_size,
                                      stream_ptr(stream, _device_of(output))))


def dequantize_awq(weight, zeros, scales, group_size, stream=None):
    """Allocates the [qweight.rows, scales.cols] output in the scales' float type
    and dequantizes into it (src/kernel/mod.rs:9-51)."""
    if not scales.is_floating_point():
        raise Panic("dddddd")  # the reference's message for a non-float scales primitive
    if weight.dtype not in (torch.int32, torch.uint32):
        raise Panic("assertion failed: matches!(w_primitive.dtype(), DType::I32 | DType::U32)")
    if zeros.dtype not in (torch.int32, torch.uint32):
        raise Panic("assertion failed: matches!(z_primitive.dtype(), DType::I32 | DType::U32)")
    out = torch.empty((weight.shape[0], scales.shape[-1]), dtype=scales.dtype, device=scales.device)
    dequantize_native(weight, zeros, scales, out, group_size, stream)
    return out


def _device_of(t):
    return t.device if t.device.type == "cuda" else None
