"""AutoAWQ checkpoint ingestion for the module types.

The reference leaves loading to Burn's record machinery: an
`AWQGEMMLinear` is the four parameters `qweight`, `qzeros`, `scales` and an
optional `bias` (src/modules/awq_gemm.rs:127-133), in the AutoAWQ layout its
README documents (README.md:60-70): qweight [K, N/8] and qzeros [K/g, N/8] as
int32 (or uint32) with 8 nibbles per word, scales [K/g, N] as f16 or f32.
AutoAWQ safetensors files name them `<layer>.qweight`, `<layer>.qzeros`,
`<layer>.scales`, `<layer>.bias`.

This module reads such tensors (from a safetensors file or an in-memory
mapping) into `AWQGEMMLinear` / `AWQLinear`, checking them with the same
constraints and messages the modules' build methods apply, and writes them
back. int32 words are kept bit for bit (no sign conversion): the kernels read
them as uint32.
"""
import torch

from ._lib import Panic
from .modules import AWQ_PACK_FACTOR, INNER_K, TILE_N_BASE, AWQGateUpSiLU, AWQGEMMLinear, AWQLinear

_PACKED_DTYPES = (torch.int32, torch.uint32) if hasattr(torch, "uint32") else (torch.int32,)


def _read(source, name):
    if isinstance(source, dict):
        if name not in source:
            raise Panic(f"checkpoint has no tensor '{name}'")
        return source[name]
    from safetensors import safe_open  # the file format AutoAWQ writes

    with safe_open(source, framework="pt") as f:
        if name not in f.keys():
            raise Panic(f"checkpoint has no tensor '{name}'")
        return f.get_tensor(name)


def _has(source, name):
    if isinstance(source, dict):
        return name in source
    from safetensors import safe_open

    with safe_open(source, framework="pt") as f:
        return name in f.keys()


def _check_awq(qweight, qzeros, scales, need_gemm_constraints):
    if qweight.dim() != 2 or qzeros.dim() != 2 or scales.dim() != 2:
        raise Panic("AWQ tensors must be 2-D: qweight [K, N/8], qzeros [K/g, N/8], scales [K/g, N]")
    if qweight.dtype not in _PACKED_DTYPES or qzeros.dtype not in _PACKED_DTYPES:
        raise Panic("AWQ packed q_weight must use 32-bit elements (i32/u32), "
                    f"got {qweight.dtype} / {qzeros.dtype}.")
    if scales.dtype not in (torch.float16, torch.float32, torch.bfloat16):
        raise Panic(f"AWQ scales must be f16, bf16 or f32, got {scales.dtype}")
    k, n_packed = qweight.shape
    groups, n = scales.shape
    n_out = n_packed * AWQ_PACK_FACTOR
    if n != n_out:
        raise Panic(f"scales has {n} columns, qweight packs {n_out}")
    if tuple(qzeros.shape) != (groups, n_packed):
        raise Panic(f"qzeros must be [{groups}, {n_packed}], got {list(qzeros.shape)}")
    if groups == 0 or k % groups != 0:
        raise Panic("d_input must be divisible by group_size")
    group = k // groups
    if need_gemm_constraints:  # AWQGEMMLinearConfig::build (src/modules/awq_gemm.rs:78-94)
        if n_out % TILE_N_BASE != 0:
            raise Panic(f"d_output must be divisible by TILE_N ({TILE_N_BASE})")
        if k % INNER_K != 0:
            raise Panic(f"d_input must be divisible by INNER_K ({INNER_K})")
    return k, n_out, group


def load_awq_gemm_linear(source, prefix, device=None, scale_dtype=None):
    """`AWQGEMMLinear` from `<prefix>.qweight/.qzeros/.scales[/.bias]` of a
    safetensors file path or a name -> tensor mapping. `scale_dtype` casts the
    scales (and bias) on load, e.g. to match the activations; default keeps
    the stored dtype."""
    qweight = _read(source, f"{prefix}.qweight")
    qzeros = _read(source, f"{prefix}.qzeros")
    scales = _read(source, f"{prefix}.scales")
    _check_awq(qweight, qzeros, scales, need_gemm_constraints=True)
    bias = _read(source, f"{prefix}.bias") if _has(source, f"{prefix}.bias") else None
    if bias is not None and tuple(bias.shape) != (scales.shape[1],):
        raise Panic(f"bias must be [{scales.shape[1]}], got {list(bias.shape)}")
    sd = scale_dtype or scales.dtype
    return AWQGEMMLinear(
        qweight.contiguous().to(device),
        qzeros.contiguous().to(device),
        scales.to(sd).contiguous().to(device),
        None if bias is None else bias.to(sd).contiguous().to(device),
    )


def load_fused_awq_gemm_linear(source, prefixes, device=None, scale_dtype=None):
    """One `AWQGEMMLinear` computing several projections of the same input in
    one launch (e.g. q/k/v or gate/up), by concatenating their tensors along
    N: qweight/qzeros [.., N_i/8] and scales/bias [.., N_i] side by side. Packs
    never straddle projections (each N_i % 32 == 0), so column block i of the
    fused output is exactly projection i. All projections must share K and the
    group size; a bias, if any projection has one, is zero for the others.
    Returns (layer, sizes) with sizes the N_i in order:
    `torch.split(layer.forward(x), sizes, dim=-1)` gives the projections."""
    parts = []
    for prefix in prefixes:
        qweight = _read(source, f"{prefix}.qweight")
        qzeros = _read(source, f"{prefix}.qzeros")
        scales = _read(source, f"{prefix}.scales")
        k, n, group = _check_awq(qweight, qzeros, scales, need_gemm_constraints=True)
        bias = _read(source, f"{prefix}.bias") if _has(source, f"{prefix}.bias") else None
        if bias is not None and tuple(bias.shape) != (n,):
            raise Panic(f"bias must be [{n}], got {list(bias.shape)}")
        parts.append((prefix, qweight, qzeros, scales, bias, k, n, group))
    if not parts:
        raise Panic("no projections to fuse")
    k0, g0 = parts[0][5], parts[0][7]
    for prefix, _, _, _, _, k, _, group in parts:
        if k != k0 or group != g0:
            raise Panic(f"fused projections must share d_input and group_size: {prefix} has "
                        f"({k}, {group}), {parts[0][0]} has ({k0}, {g0})")
    sd = scale_dtype or parts[0][3].dtype
    qweight = torch.cat([p[1].view(torch.int32) if p[1].dtype != torch.int32 else p[1] for p in parts], dim=1)
    qzeros = torch.cat([p[2].view(torch.int32) if p[2].dtype != torch.int32 else p[2] for p in parts], dim=1)
    scales = torch.cat([p[3].to(sd) for p in parts], dim=1)
    bias = None
    if any(p[4] is not None for p in parts):
        bias = torch.cat([p[4].to(sd) if p[4] is not None else torch.zeros(p[6], dtype=sd) for p in parts])
    layer = AWQGEMMLinear(qweight.contiguous().to(device), qzeros.contiguous().to(device),
                          scales.contiguous().to(device), None if bias is None else bias.contiguous().to(device))
    return layer, [p[6] for p in parts]


def load_awq_gate_up_silu(source, gate_prefix, up_prefix, device=None, scale_dtype=None):
    """`AWQGateUpSiLU` from the gate and up projections' tensors (e.g.
    `model.layers.0.mlp.gate_proj` / `.up_proj`): forward(x) = SiLU(gate(x)) *
    up(x) in one launch. Both must share K, the group size and the width."""
    gate = load_awq_gemm_linear(source, gate_prefix, None, scale_dtype)
    up = load_awq_gemm_linear(source, up_prefix, None, scale_dtype)
    layer = AWQGateUpSiLU.from_gate_up(gate, up)
    if layer.scales.shape[1] % 64 != 0:
        raise Panic("gate/up GEMM: N (gate and up interleaved) must be a multiple of 64")
    return AWQGateUpSiLU(layer.qweight.to(device), layer.qzeros.to(device), layer.scales.to(device),
                         None if layer.bias is None else layer.bias.to(device))


def load_awq_linear(source, prefix, device=None, scale_dtype=None):
    """`AWQLinear` (dequantize path, sequential nibble order) from the same
    tensor names; the module's own build checks apply (N % 8, K % g, N % 32,
    src/modules/awq_dequantize.rs:26-28)."""
    qweight = _read(source, f"{prefix}.qweight")
    qzeros = _read(source, f"{prefix}.qzeros")
    scales = _read(source, f"{prefix}.scales")
    _, n_out, _ = _check_awq(qweight, qzeros, scales, need_gemm_constraints=False)
    if n_out % 32 != 0:  # AWQLinearConfig::build's own check
        raise Panic("assertion failed: self.d_output % 32 == 0")
    sd = scale_dtype or scales.dtype
    return AWQLinear(qweight.contiguous().to(device), qzeros.contiguous().to(device),
                     scales.to(sd).contiguous().to(device))


def state_dict(module, prefix):
    """The module's tensors under AutoAWQ names, on the CPU."""
    out = {f"{prefix}.qweight": module.qweight.detach().cpu(),
           f"{prefix}.qzeros": module.qzeros.detach().cpu(),
           f"{prefix}.scales": module.scales.detach().cpu()}
    if getattr(module, "bias", None) is not None:
        out[f"{prefix}.bias"] = module.bias.detach().cpu()
    return out


def save(modules, path):
    """Write {prefix: module} to a safetensors file in AutoAWQ naming."""
    from safetensors.torch import save_file

    tensors = {}
    for prefix, module in modules.items():
        tensors.update(state_dict(module, prefix))
    save_file({k: v.contiguous() for k, v in tensors.items()}, path)
