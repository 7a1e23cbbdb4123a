"""Module-level API on the GPU: AWQGEMMLinear forward shapes/bias, the
reference's module test cases that are valid with INNER_K = 64."""
import numpy as np
import pytest
import torch

import awq_oracle as oracle
from cube_awq import AWQGEMMLinear, AWQGEMMLinearConfig, pack
from helpers import make_problem

pytestmark = pytest.mark.gpu


def _layer(dev, K, N, g, bias=False, s_dtype=torch.float32, seed_scales=(0.002, 0.02)):
    x, qw, qz, sc, b = make_problem(1, K, N, g, x_dt="f32", s_dt="f32", scale_range=seed_scales,
                                    bias=bias)
    lay = AWQGEMMLinearConfig.new(K, N, g).with_bias(bias).build(dev, s_dtype)
    lay.qweight.copy_(torch.from_numpy(pack.as_int32(qw)))
    lay.qzeros.copy_(torch.from_numpy(pack.as_int32(qz)))
    lay.scales.copy_(torch.from_numpy(sc))
    if bias:
        lay.bias.copy_(torch.from_numpy(b))
    return lay, qw, qz, sc, b


@pytest.mark.parametrize("dims", [(2, 32, 128), (1, 16, 14, 128), (3, 1, 128), (5, 128), (2, 7, 128)])
@pytest.mark.parametrize("bias", [False, True])
def test_forward_shapes_and_values(dev, dims, bias):
    K, N, g = 128, 96, 64
    lay, qw, qz, sc, b = _layer(dev, K, N, g, bias)
    x = torch.randn(*dims, generator=torch.Generator().manual_seed(3))
    y = lay.forward(x.to(dev))
    torch.cuda.synchronize()
    assert tuple(y.shape) == tuple(dims[:-1]) + (N,)
    rows = x.reshape(-1, K).numpy()
    ref = oracle.gemm_f64(rows, qw, qz, sc, g, bias=b)
    assert oracle.rel_l2(y.reshape(-1, N).cpu().numpy(), ref) <= 1e-5


def test_forward_handles_non_divisible_m(dev):
    # test_forward_handles_non_divisible_m with g=64 (the module's INNER_K).
    lay, *_ = _layer(dev, 64, 32, 64)
    y = lay.forward(torch.zeros(1, 14, 64, device=dev))
    torch.cuda.synchronize()
    assert tuple(y.shape) == (1, 14, 32)
    assert torch.all(y == 0)


def test_forward_fp16_model(dev):
    K, N, g = 4096, 4096, 128
    lay, qw, qz, sc, _ = _layer(dev, K, N, g, s_dtype=torch.float16)
    sc16 = lay.scales.cpu().numpy()
    for M in (1, 64):
        x = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).to(torch.float16)
        y = lay.forward(x.to(dev))
        torch.cuda.synchronize()
        assert y.dtype == torch.float16
        ref = oracle.gemm_f64(x.float().numpy(), qw, qz, sc16.astype(np.float32), g)
        assert oracle.rel_l2(y.float().cpu().numpy(), ref) <= (1e-3 if M == 1 else 2e-3)


def test_forward_on_non_default_stream(dev):
    K, N, g = 256, 64, 64
    lay, qw, qz, sc, _ = _layer(dev, K, N, g)
    x = torch.randn(3, K, generator=torch.Generator().manual_seed(0))
    s = torch.cuda.Stream()
    xd = x.to(dev)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        y = lay.forward(xd)
    s.synchronize()
    assert oracle.rel_l2(y.cpu().numpy(), oracle.gemm_f64(x.numpy(), qw, qz, sc, g)) <= 1e-5


@pytest.mark.parametrize("M", [1, 300])
def test_checkpoint_loaded_layer_forward(dev, tmp_path, M):
    """An AutoAWQ-named safetensors file (int32 words, f16 scales, bias) loads
    into AWQGEMMLinear and runs on both paths (decode M = 1, prefill M = 300)."""
    from cube_awq import checkpoint
    K, N, g = 512, 256, 128
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt="f16", s_dt="f16", bias=True)
    path = str(tmp_path / "awq.safetensors")
    from safetensors.torch import save_file
    save_file({"blk.qweight": torch.from_numpy(pack.as_int32(qw)),
               "blk.qzeros": torch.from_numpy(pack.as_int32(qz)),
               "blk.scales": torch.from_numpy(sc.astype(np.float16)),
               "blk.bias": torch.from_numpy(b.astype(np.float16))}, path)
    lay = checkpoint.load_awq_gemm_linear(path, "blk", device=dev)
    xt = torch.from_numpy(x.astype(np.float16)).to(dev)
    y = lay.forward(xt)
    torch.cuda.synchronize()
    ref = oracle.gemm_f64(x.astype(np.float16).astype(np.float32), qw, qz,
                          sc.astype(np.float16).astype(np.float32), g,
                          bias=b.astype(np.float16).astype(np.float32))
    assert oracle.rel_l2(y.float().cpu().numpy(), ref) <= 2e-3


@pytest.mark.parametrize("M", [1, 4, 12, 300])
def test_fused_qkv_projection_forward(dev, M):
    """q/k/v fused along N (one launch) against each projection's oracle."""
    from cube_awq import checkpoint, synth
    K, g = 1024, 128
    sizes = [1024, 256, 256]
    tensors, parts = {}, []
    for i, n in enumerate(sizes):
        qw = synth.packed_nibbles(40 + 4 * i, K, n // 8)
        qz = synth.packed_nibbles(41 + 4 * i, K // g, n // 8)
        sc = synth.uniform(42 + 4 * i, (K // g, n), 0.002, 0.02, np.float16)
        tensors[f"p{i}.qweight"] = torch.from_numpy(pack.as_int32(qw))
        tensors[f"p{i}.qzeros"] = torch.from_numpy(pack.as_int32(qz))
        tensors[f"p{i}.scales"] = torch.from_numpy(sc)
        parts.append((qw, qz, sc))
    lay, got_sizes = checkpoint.load_fused_awq_gemm_linear(tensors, ["p0", "p1", "p2"], device=dev)
    assert got_sizes == sizes
    x = synth.normal(synth.TID_X, (M, K), np.float16)
    y = lay.forward(torch.from_numpy(x).to(dev))
    torch.cuda.synchronize()
    outs = torch.split(y.float().cpu(), sizes, dim=-1)
    tol = 1e-3 if M <= 16 else 2e-3  # f16 output
    for (qw, qz, sc), out in zip(parts, outs):
        ref = oracle.gemm_f64(x.astype(np.float32), qw, qz, sc.astype(np.float32), g)
        assert oracle.rel_l2(out.numpy(), ref) <= tol
