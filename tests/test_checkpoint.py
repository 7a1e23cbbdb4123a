"""AutoAWQ checkpoint ingestion (safetensors naming, int32 words kept bit for
bit, the module constraints and messages), CPU only; the GPU test runs the
loaded layer against the oracle."""
import numpy as np
import pytest
import torch

from cube_awq import checkpoint, synth
from cube_awq._lib import Panic
from cube_awq.modules import AWQGEMMLinear, AWQLinear


def _tensors(k=256, n=128, g=64, bias=True):
    qw = torch.from_numpy(synth.packed_nibbles(synth.TID_QWEIGHT, k, n // 8).view(np.int32).copy())
    qz = torch.from_numpy(synth.packed_nibbles(synth.TID_QZEROS, k // g, n // 8).view(np.int32).copy())
    sc = torch.from_numpy(synth.uniform(synth.TID_SCALES, (k // g, n), 0.002, 0.02, np.float16))
    d = {"model.layers.0.mlp.up_proj.qweight": qw, "model.layers.0.mlp.up_proj.qzeros": qz,
         "model.layers.0.mlp.up_proj.scales": sc}
    if bias:
        d["model.layers.0.mlp.up_proj.bias"] = torch.from_numpy(
            synth.uniform(synth.TID_BIAS, (n,), -1.0, 1.0, np.float16))
    return d


def test_roundtrip_through_safetensors(tmp_path):
    d = _tensors()
    layer = checkpoint.load_awq_gemm_linear(d, "model.layers.0.mlp.up_proj")
    assert isinstance(layer, AWQGEMMLinear) and layer.group_size() == 64
    path = str(tmp_path / "layer.safetensors")
    checkpoint.save({"model.layers.0.mlp.up_proj": layer}, path)
    again = checkpoint.load_awq_gemm_linear(path, "model.layers.0.mlp.up_proj")
    for name in ("qweight", "qzeros", "scales", "bias"):
        a, b = getattr(layer, name), getattr(again, name)
        assert a.dtype == b.dtype and torch.equal(a, b), name
    # int32 words with the top bit set survive unchanged (read as uint32 by the kernels)
    assert (again.qweight < 0).any()


def test_optional_bias_and_scale_cast():
    d = _tensors(bias=False)
    layer = checkpoint.load_awq_gemm_linear(d, "model.layers.0.mlp.up_proj", scale_dtype=torch.float32)
    assert layer.bias is None and layer.scales.dtype == torch.float32
    lin = checkpoint.load_awq_linear(d, "model.layers.0.mlp.up_proj")
    assert isinstance(lin, AWQLinear) and lin.group_size() == 64


@pytest.mark.parametrize("mutate, msg", [
    (lambda d: d.pop("model.layers.0.mlp.up_proj.qzeros"), "no tensor"),
    (lambda d: d.__setitem__("model.layers.0.mlp.up_proj.qweight",
                             d["model.layers.0.mlp.up_proj.qweight"].to(torch.int64)), "32-bit elements"),
    (lambda d: d.__setitem__("model.layers.0.mlp.up_proj.scales",
                             d["model.layers.0.mlp.up_proj.scales"][:, :64]), "columns"),
    (lambda d: d.__setitem__("model.layers.0.mlp.up_proj.qzeros",
                             d["model.layers.0.mlp.up_proj.qzeros"][:2]), "qzeros must be"),
])
def test_rejections(mutate, msg):
    d = _tensors()
    mutate(d)
    with pytest.raises(Panic, match=msg):
        checkpoint.load_awq_gemm_linear(d, "model.layers.0.mlp.up_proj")


def test_gemm_constraints_apply():
    # K = 96 is a multiple of the group (32) but not of INNER_K (64)
    qw = torch.zeros((96, 4), dtype=torch.int32)
    qz = torch.zeros((3, 4), dtype=torch.int32)
    sc = torch.ones((3, 32), dtype=torch.float16)
    with pytest.raises(Panic, match="INNER_K"):
        checkpoint.load_awq_gemm_linear({"l.qweight": qw, "l.qzeros": qz, "l.scales": sc}, "l")


def _proj(prefix, k, n, g, seed, bias):
    qw = torch.from_numpy(synth.packed_nibbles(seed, k, n // 8).view(np.int32).copy())
    qz = torch.from_numpy(synth.packed_nibbles(seed + 1, k // g, n // 8).view(np.int32).copy())
    sc = torch.from_numpy(synth.uniform(seed + 2, (k // g, n), 0.002, 0.02, np.float16))
    d = {f"{prefix}.qweight": qw, f"{prefix}.qzeros": qz, f"{prefix}.scales": sc}
    if bias:
        d[f"{prefix}.bias"] = torch.from_numpy(synth.uniform(seed + 3, (n,), -1.0, 1.0, np.float16))
    return d


def test_fused_projections_concatenate_along_n():
    a = "model.layers.0.self_attn"
    d = {}
    d.update(_proj(f"{a}.q_proj", 256, 256, 64, 10, bias=True))
    d.update(_proj(f"{a}.k_proj", 256, 64, 64, 20, bias=False))
    d.update(_proj(f"{a}.v_proj", 256, 96, 64, 30, bias=True))
    layer, sizes = checkpoint.load_fused_awq_gemm_linear(d, [f"{a}.q_proj", f"{a}.k_proj", f"{a}.v_proj"])
    assert sizes == [256, 64, 96] and layer.group_size() == 64
    assert tuple(layer.qweight.shape) == (256, 52) and tuple(layer.scales.shape) == (4, 416)
    col = 0
    for name, n in zip(("q_proj", "k_proj", "v_proj"), sizes):
        p = f"{a}.{name}"
        assert torch.equal(layer.qweight[:, col // 8:(col + n) // 8], d[f"{p}.qweight"])
        assert torch.equal(layer.qzeros[:, col // 8:(col + n) // 8], d[f"{p}.qzeros"])
        assert torch.equal(layer.scales[:, col:col + n], d[f"{p}.scales"])
        want_b = d.get(f"{p}.bias", torch.zeros(n, dtype=torch.float16))
        assert torch.equal(layer.bias[col:col + n], want_b)
        col += n


def test_fused_projections_reject_mismatched_k_or_group():
    d = {}
    d.update(_proj("p0", 256, 64, 64, 10, bias=False))
    d.update(_proj("p1", 256, 64, 128, 20, bias=False))
    with pytest.raises(Panic, match="share d_input and group_size"):
        checkpoint.load_fused_awq_gemm_linear(d, ["p0", "p1"])
    d.update(_proj("p2", 128, 64, 64, 30, bias=False))
    with pytest.raises(Panic, match="share d_input and group_size"):
        checkpoint.load_fused_awq_gemm_linear(d, ["p0", "p2"])


def test_gate_up_silu_interleaves_columns():
    """load_awq_gate_up_silu: column 2j of every tensor is gate column j and
    2j + 1 up column j (qweight/qzeros as logical nibbles in AutoAWQ order)."""
    from cube_awq import AWQGateUpSiLU, pack
    m = "model.layers.0.mlp"
    d = {}
    d.update(_proj(f"{m}.gate_proj", 256, 96, 64, 40, bias=True))
    d.update(_proj(f"{m}.up_proj", 256, 96, 64, 50, bias=False))
    layer = checkpoint.load_awq_gate_up_silu(d, f"{m}.gate_proj", f"{m}.up_proj")
    assert isinstance(layer, AWQGateUpSiLU) and layer.group_size() == 64
    assert tuple(layer.qweight.shape) == (256, 24) and tuple(layer.scales.shape) == (4, 192)
    for name in ("qweight", "qzeros"):
        got = pack.unpack(layer.__dict__[name].numpy().view(np.uint32), "awq")
        g = pack.unpack(d[f"{m}.gate_proj.{name}"].numpy().view(np.uint32), "awq")
        u = pack.unpack(d[f"{m}.up_proj.{name}"].numpy().view(np.uint32), "awq")
        assert np.array_equal(got[:, 0::2], g) and np.array_equal(got[:, 1::2], u), name
    assert torch.equal(layer.scales[:, 0::2], d[f"{m}.gate_proj.scales"])
    assert torch.equal(layer.scales[:, 1::2], d[f"{m}.up_proj.scales"])
    assert torch.equal(layer.bias[0::2], d[f"{m}.gate_proj.bias"])
    assert not layer.bias[1::2].any()


def test_gate_up_silu_rejects_mismatched_projections():
    d = {}
    d.update(_proj("g", 256, 32, 64, 40, bias=False))
    d.update(_proj("u", 256, 32, 64, 50, bias=False))
    layer = checkpoint.load_awq_gate_up_silu(d, "g", "u")  # 2 x 32 = 64 interleaved: accepted
    assert tuple(layer.scales.shape) == (4, 64)
    d.update(_proj("u2", 256, 64, 64, 60, bias=False))
    with pytest.raises(Panic, match="same shapes"):
        checkpoint.load_awq_gate_up_silu(d, "g", "u2")
