"""Module-level interface, mirroring the reference's `cube_awq::modules`.

  AWQGEMMLinearConfig / AWQGEMMLinear   src/modules/awq_gemm.rs:54-233
  AWQLinearConfig / AWQLinear           src/modules/awq_dequantize.rs:9-109

Same constructors, builder methods, parameter shapes, `group_size()`,
`forward()` / `dequantize()` and panic texts. Differences, all deliberate:
  * AWQGEMMLinear.forward fuses the bias add into the kernel's epilogue (the
    reference launches a separate elementwise add, src/modules/awq_gemm.rs:225-228).
  * M is a runtime argument of one compiled kernel; the reference JIT-compiles
    a kernel per distinct M (M is part of its comptime ShapeConfig).
  * AWQLinear.forward (dequantize, then Burn's autotuned matmul in the
    reference, src/modules/awq_dequantize.rs:74-108) runs as one fused
    dequant-GEMM launch in sequential nibble order when the shapes meet the
    fused kernels' constraints (those of AWQGEMMLinear: K % 64, N % 32,
    g % 64, g >= 64) and the scales share the input's dtype; other shapes
    (e.g. the reference's g = 2 test layer) take dequantize() and torch's
    matmul, the reference's own two steps.
Parameters are plain torch tensors on the module's device: qweight/qzeros
int32 (AutoAWQ checkpoints store int32; uint32 is accepted too), scales and
bias in the backend float type.
"""
import torch

from . import _lib
from ._lib import Panic, check, lib, stream_ptr
from .kernel import dequantize_awq

AWQ_PACK_FACTOR = 8
TILE_N_BASE = 32
INNER_K = 64


def _assert_eq(left, right, msg):
    if left != right:
        raise Panic(f"assertion `left == right` failed: {msg}\n  left: {left}\n right: {right}")


class AWQGEMMLinearConfig:
    def __init__(self, d_input, d_output, group_size):
        self.d_input = d_input
        self.d_output = d_output
        self.group_size = group_size
        self.bias = False

    @classmethod
    def new(cls, d_input, d_output, group_size):
        return cls(d_input, d_output, group_size)

    def with_bias(self, bias):
        self.bias = bool(bias)
        return self

    def build(self, device=None, dtype=torch.float32):
        """Allocates uninitialised qweight [K, N/8], qzeros [K/g, N/8], scales
        [K/g, N] and a zero bias [N] (src/modules/awq_gemm.rs:77-124)."""
        if not self.group_size > 0:
            raise Panic("group_size must be > 0")
        if self.d_output % AWQ_PACK_FACTOR != 0:
            raise Panic(f"d_output must be divisible by {AWQ_PACK_FACTOR}")
        if self.d_output % TILE_N_BASE != 0:
            raise Panic(f"d_output must be divisible by TILE_N ({TILE_N_BASE})")
        if self.d_input % INNER_K != 0:
            raise Panic(f"d_input must be divisible by INNER_K ({INNER_K})")
        if self.d_input % self.group_size != 0:
            raise Panic("d_input must be divisible by group_size")
        n_packed = self.d_output // AWQ_PACK_FACTOR
        groups = self.d_input // self.group_size
        qweight = torch.empty((self.d_input, n_packed), dtype=torch.int32, device=device)
        qzeros = torch.empty((groups, n_packed), dtype=torch.int32, device=device)
        scales = torch.empty((groups, self.d_output), dtype=dtype, device=device)
        bias = torch.zeros((self.d_output,), dtype=dtype, device=device) if self.bias else None
        return AWQGEMMLinear(qweight, qzeros, scales, bias)


class AWQGEMMLinear:
    def __init__(self, qweight, qzeros, scales, bias=None):
        self.qweight = qweight
        self.qzeros = qzeros
        self.scales = scales
        self.bias = bias

    def group_size(self):
        return self.qweight.shape[0] // self.scales.shape[0]

    def forward(self, input, stream=None):
        """input [..., K] (D >= 2) -> [..., N], fused dequant-GEMM (+ bias).
        src/modules/awq_gemm.rs:146-232."""
        if input.dim() < 2:
            raise Panic("input tensor must have at least 2 dims: [..., K]")
        dims = list(input.shape)
        k = dims[-1]
        if not k > 0:
            raise Panic("input last dim (K) must be > 0")
        numel = input.numel()
        if numel % k != 0:
            raise Panic("input elements must be divisible by K")
        m = numel // k
        x = input.reshape(m, k)
        if not x.is_contiguous():
            x = x.contiguous()
        k_from_weight = self.qweight.shape[0]
        n = self.qweight.shape[-1] * 8
        group_size = self.group_size()
        _assert_eq(k, k_from_weight, "input last dim (K) must match qweight rows")
        if self.qweight.dtype not in (torch.int32, torch.uint32):
            raise Panic("qweight must have i32/u32 dtype")
        if self.qzeros.dtype not in (torch.int32, torch.uint32):
            raise Panic("qzeros must have i32/u32 dtype")
        out = torch.empty((m, n), dtype=input.dtype, device=input.device)
        bias = self.bias
        check(lib().awq_gemm(
            x.data_ptr(), _lib.awq_dtype(x),
            self.qweight.data_ptr(), self.qzeros.data_ptr(),
            self.scales.data_ptr(), _lib.awq_dtype(self.scales),
            bias.data_ptr() if bias is not None else None,
            _lib.awq_dtype(bias) if bias is not None else _lib.AWQ_F32,
            out.data_ptr(), _lib.awq_dtype(out),
            m, k, n, group_size,
            stream_ptr(stream, input.device if input.is_cuda else None)))
        dims[-1] = n
        return out.reshape(dims)

    __call__ = forward


class AWQGateUpSiLU:
    """Gate and up projections with the SiLU activation in one launch:
    forward(x) = SiLU(x.Wg + bg) * (x.Wu + bu), SiLU(g) = g / (1 + e^-g), the
    MLP input half of Llama-style blocks. Not a reference module: the
    reference runs gate and up as two AWQGEMMLinear forwards (each a GEMM plus
    a bias op, src/modules/awq_gemm.rs:146-232) and leaves the activation to
    the caller. The parameters hold the two projections interleaved by column
    (column 2j = gate j, 2j + 1 = up j; see `from_gate_up`), so the GEMM
    epilogue has both values of an output in one place."""

    def __init__(self, qweight, qzeros, scales, bias=None):
        self.qweight = qweight
        self.qzeros = qzeros
        self.scales = scales
        self.bias = bias

    @classmethod
    def from_gate_up(cls, gate, up):
        """From two AWQGEMMLinear layers of the same input (same K, group and
        intermediate width); a missing bias counts as zero."""
        from .pack import interleave_columns, interleave_packed
        if tuple(gate.qweight.shape) != tuple(up.qweight.shape) or tuple(gate.scales.shape) != tuple(up.scales.shape):
            raise Panic("gate and up projections must have the same shapes")
        if gate.scales.dtype != up.scales.dtype:
            raise Panic("gate and up scales must share a dtype")
        bias = None
        if gate.bias is not None or up.bias is not None:
            zg = torch.zeros_like(gate.scales[0])
            bg = gate.bias if gate.bias is not None else zg
            bu = up.bias if up.bias is not None else zg
            bias = interleave_columns(bg[None, :], bu[None, :].to(bg.dtype))[0].contiguous()
        return cls(interleave_packed(gate.qweight, up.qweight).contiguous(),
                   interleave_packed(gate.qzeros, up.qzeros).contiguous(),
                   interleave_columns(gate.scales, up.scales).contiguous(), bias)

    def group_size(self):
        return self.qweight.shape[0] // self.scales.shape[0]

    def forward(self, input, stream=None):
        """input [..., K] (D >= 2) -> [..., N/2], N the interleaved width."""
        if input.dim() < 2:
            raise Panic("input tensor must have at least 2 dims: [..., K]")
        dims = list(input.shape)
        k = dims[-1]
        m = input.numel() // k if k > 0 else 0
        x = input.reshape(m, k)
        if not x.is_contiguous():
            x = x.contiguous()
        _assert_eq(k, self.qweight.shape[0], "input last dim (K) must match qweight rows")
        n = self.qweight.shape[-1] * 8
        out = torch.empty((m, n // 2), dtype=input.dtype, device=input.device)
        bias = self.bias
        check(lib().awq_gemm_silu_mul(
            x.data_ptr(), _lib.awq_dtype(x),
            self.qweight.data_ptr(), self.qzeros.data_ptr(),
            self.scales.data_ptr(), _lib.awq_dtype(self.scales),
            bias.data_ptr() if bias is not None else None,
            _lib.awq_dtype(bias) if bias is not None else _lib.AWQ_F32,
            out.data_ptr(), _lib.awq_dtype(out),
            m, k, n, self.group_size(),
            stream_ptr(stream, input.device if input.is_cuda else None)))
        dims[-1] = n // 2
        return out.reshape(dims)

    __call__ = forward


class AWQLinearConfig:
    def __init__(self, d_input, d_output, group_size):
        self.d_input = d_input
        self.d_output = d_output
        self.group_size = group_size

    @classmethod
    def new(cls, d_input, d_output, group_size):
        return cls(d_input, d_output, group_size)

    def build(self, device=None, dtype=torch.float32):
        """src/modules/awq_dequantize.rs:25-41 (stringified asserts)."""
        if not self.d_output % 8 == 0:
            raise Panic("assertion failed: self.d_output % 8 == 0")
        if self.group_size == 0 or not self.d_input % self.group_size == 0:
            raise Panic("assertion failed: self.d_input % self.group_size == 0")
        if not self.d_output % 32 == 0:
            raise Panic("assertion failed: self.d_output % 32 == 0")
        d_out = self.d_output // 8
        groups = self.d_input // self.group_size
        return AWQLinear(
            torch.empty((self.d_input, d_out), dtype=torch.int32, device=device),
            torch.empty((groups, d_out), dtype=torch.int32, device=device),
            torch.empty((groups, self.d_output), dtype=dtype, device=device))


class AWQLinear:
    def __init__(self, qweight, qzeros, scales):
        self.qweight = qweight
        self.qzeros = qzeros
        self.scales = scales

    def group_size(self):
        return self.qweight.shape[0] // self.scales.shape[0]

    def dequantize(self, stream=None):
        """[K, N] weight in the scales' float type, sequential nibble order,
        bit-exact (q - z) * s. src/modules/awq_dequantize.rs:62-72."""
        return dequantize_awq(self.qweight, self.qzeros, self.scales, self.group_size(), stream)

    def forward(self, input, stream=None):
        """input [M, K] -> [M, N] = input @ dequantize(), as
        src/modules/awq_dequantize.rs:74-108. Like the reference (whose 2-D
        weight meets a D-rank input in Burn's matmul), a rank other than 2 is
        rejected (here before any work is queued)."""
        if input.dim() != 2:
            raise Panic(f"RankMismatch {{ lhs: {input.dim()}, rhs: 2 }}")
        m, k = input.shape
        n = self.scales.shape[-1]
        if self._fusable(input, m, k, n):
            x = input if input.is_contiguous() and input.data_ptr() % 16 == 0 else input.clone()
            out = torch.empty((m, n), dtype=input.dtype, device=input.device)
            check(lib().awq_gemm_ordered(
                x.data_ptr(), _lib.awq_dtype(x),
                self.qweight.data_ptr(), self.qzeros.data_ptr(),
                self.scales.data_ptr(), _lib.awq_dtype(self.scales),
                None, _lib.AWQ_F32, out.data_ptr(), _lib.awq_dtype(out),
                m, k, n, self.group_size(), _lib.AWQ_ORDER_SEQUENTIAL,
                stream_ptr(stream, input.device)))
            return out
        weight = self.dequantize(stream)
        return torch.matmul(input, weight.to(input.dtype))

    def _fusable(self, input, m, k, n):
        """True when the fused sequential-order launch takes this problem."""
        return (input.is_cuda and input.dtype == self.scales.dtype and m > 0
                and k == self.qweight.shape[0] and self.qweight.shape[-1] * 8 == n
                and self.qweight.dtype in (torch.int32, torch.uint32)
                and self.qzeros.dtype in (torch.int32, torch.uint32)
                and self.scales.is_contiguous() and self.qweight.is_contiguous()
                and self.qzeros.is_contiguous()
                and lib().awq_validate_gemm(m, k, n, self.group_size()) == 0)

    __call__ = forward
