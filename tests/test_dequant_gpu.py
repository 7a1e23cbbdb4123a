"""Standalone dequantize on the GPU vs the oracle: bit-exact.

Reference: dequantize_awq_symmetric (src/kernel/awq_kernel.rs:23-61), module
tests src/modules/awq_dequantize.rs:208-237, integration test
tests/awq_test.rs:117-221."""
import ctypes

import numpy as np
import pytest
import torch

import awq_oracle as oracle
import cube_awq
from cube_awq import AWQLinear, _lib
from conftest import load_golden
from helpers import host_f32, make_problem, round_to, to_device, to_host

pytestmark = pytest.mark.gpu

AWQ_DT = {"f32": _lib.AWQ_F32, "f16": _lib.AWQ_F16, "bf16": _lib.AWQ_BF16}


@pytest.mark.parametrize("name", ["dequant_seq_64x32_g2", "dequant_seq_128x32_g128"])
def test_dequantize_matches_reference_golden(dev, name):
    g = load_golden(name)
    layer = AWQLinear(torch.from_numpy(g["qweight"].view(np.int32)).to(dev),
                      torch.from_numpy(g["qzeros"].view(np.int32)).to(dev),
                      torch.from_numpy(g["scales"]).to(dev))
    assert layer.group_size() == int(g["group_size"])
    out = layer.dequantize()
    torch.cuda.synchronize()
    assert tuple(out.shape) == g["expected"].shape
    assert np.array_equal(to_host(out).view(np.uint32), g["expected"].view(np.uint32))


def _dequant_ptr(qw, qz, sc, s_dt, o_dt, K, N, g, order, dev):
    out = torch.full((K, N), float("nan"), dtype={"f32": torch.float32, "f16": torch.float16,
                                                  "bf16": torch.bfloat16}[o_dt], device=dev)
    d_qw = torch.from_numpy(qw.view(np.int32)).to(dev)
    d_qz = torch.from_numpy(qz.view(np.int32)).to(dev)
    d_sc = to_device(sc, s_dt, dev)
    _lib.check(cube_awq.lib().awq_dequantize(
        d_qw.data_ptr(), d_qz.data_ptr(), d_sc.data_ptr(), AWQ_DT[s_dt], out.data_ptr(),
        AWQ_DT[o_dt], K, N, g, order, None))
    torch.cuda.synchronize()
    return to_host(out)


@pytest.mark.parametrize("K,N,g", [(64, 32, 2), (128, 32, 128), (256, 96, 4), (512, 4096, 64),
                                   (4096, 4096, 128), (1024, 2080, 32)])
@pytest.mark.parametrize("s_dt,o_dt", [("f32", "f32"), ("f16", "f16"), ("bf16", "bf16"),
                                       ("f16", "f32"), ("bf16", "f32")])
@pytest.mark.parametrize("order", ["seq", "awq"])
def test_dequantize_bit_exact_random(dev, K, N, g, s_dt, o_dt, order):
    _, qw, qz, sc, _ = make_problem(1, K, N, g, s_dt=s_dt, scale_range=(-0.03, 0.03))
    got = _dequant_ptr(qw, qz, sc, s_dt, o_dt, K, N, g,
                       _lib.AWQ_ORDER_SEQUENTIAL if order == "seq" else _lib.AWQ_ORDER_AUTOAWQ, dev)
    ref32 = oracle.dequant(qw, qz, host_f32(sc, s_dt), g, order)
    want = round_to(ref32, o_dt)
    assert np.array_equal(got.view(np.uint16 if o_dt != "f32" else np.uint32),
                          want.view(np.uint16 if o_dt != "f32" else np.uint32))


def test_dequantize_config4_full_size_bit_exact(dev):
    # K=14336, N=4096, g=64, f32 scales U[0.002, 0.02] -> full [14336, 4096] f32.
    K, N, g = 14336, 4096, 64
    _, qw, qz, sc, _ = make_problem(1, K, N, g, s_dt="f32")
    got = _dequant_ptr(qw, qz, sc, "f32", "f32", K, N, g, _lib.AWQ_ORDER_SEQUENTIAL, dev)
    want = oracle.dequant(qw, qz, sc, g, "seq")
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequantize_special_scales_bit_exact(dev):
    # signed zeros, subnormals, large values: sign of (q - z) * s when q == z is s's.
    K, N, g = 256, 32 * 8, 1
    q = np.repeat(np.arange(256) // 16, 1)[:, None].repeat(N, 1)
    z = np.repeat(np.arange(256) % 16, 1)[:, None].repeat(N, 1)
    from cube_awq import pack
    qw = pack.pack(q, "seq")
    qz = pack.pack(z, "seq")
    vals = np.array([0.0, -0.0, 1e-40, -2.5e-39, 3.0e38, -1.0, 0.1, 7.0], np.float32)
    sc = np.tile(np.repeat(vals, 32)[None, :], (K, 1)).astype(np.float32)
    got = _dequant_ptr(qw, qz, sc, "f32", "f32", K, N, g, _lib.AWQ_ORDER_SEQUENTIAL, dev)
    want = oracle.dequant(qw, qz, sc, g, "seq")
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequantize_native_tensor_refs(dev):
    # Kernel-level entry (dequantize_native) with the integration test's tensors.
    g = load_golden("dequant_seq_128x32_g128")
    out = torch.empty(128, 32, device=dev)
    cube_awq.dequantize_native(torch.from_numpy(g["qweight"].view(np.int32)).to(dev),
                               torch.from_numpy(g["qzeros"].view(np.int32)).to(dev),
                               torch.from_numpy(g["scales"]).to(dev), out, 128)
    torch.cuda.synchronize()
    assert np.array_equal(to_host(out), g["expected"])


def test_linear_forward_matches_cpu_matmul(dev):
    # src/modules/awq_dequantize.rs:239-281: dequantize then matmul, tol 1e-3.
    g = load_golden("dequant_seq_64x32_g2")
    layer = AWQLinear(torch.from_numpy(g["qweight"].view(np.int32)).to(dev),
                      torch.from_numpy(g["qzeros"].view(np.int32)).to(dev),
                      torch.from_numpy(g["scales"]).to(dev))
    x = (torch.arange(2 * 64, dtype=torch.float32) * 0.01).reshape(2, 64)
    y = layer.forward(x.to(dev))
    torch.cuda.synchronize()
    expect = x.double() @ torch.from_numpy(g["expected"]).double()
    assert tuple(y.shape) == (2, 32)
    assert (y.cpu().double() - expect).abs().max().item() <= 1e-3


def _native(qw, qz, sc, out, g, dev):
    cube_awq.dequantize_native(torch.from_numpy(np.ascontiguousarray(qw).view(np.int32)).to(dev),
                               torch.from_numpy(np.ascontiguousarray(qz).view(np.int32)).to(dev),
                               torch.from_numpy(np.ascontiguousarray(sc)).to(dev), out, g)
    torch.cuda.synchronize()
    return to_host(out)


def test_dequantize_native_any_rank(dev):
    # The reference reads every tensor through a linear view
    # (src/kernel/awq_kernel.rs:89-106): a [2, K/2, N/8] q_weight with a
    # [2, K/2, N] output is the same computation as the 2-D one.
    K, N, g = 256, 128, 64
    _, qw, qz, sc, _ = make_problem(1, K, N, g, s_dt="f32", scale_range=(-0.03, 0.03))
    flat = _native(qw, qz, sc, torch.full((K, N), float("nan"), device=dev), g, dev)
    got = _native(qw.reshape(2, K // 2, N // 8), qz.reshape(1, K // g, N // 8), sc.reshape(K // g, 1, N),
                  torch.full((2, K // 2, N), float("nan"), device=dev), g, dev)
    ref = oracle.dequant(qw, qz, sc, g, "seq")
    assert np.array_equal(flat.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(got.reshape(K, N).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("K,g", [(96, 64), (200, 128), (130, 4), (66, 64)])
def test_dequantize_native_partial_last_group(dev, K, g):
    # K % group_size != 0: the reference asserts nothing about it and the last
    # group (row / group_size) is simply shorter.
    N = 64
    groups = -(-K // g)
    rng = np.random.default_rng(K + g)
    qw = rng.integers(0, 2 ** 32, size=(K, N // 8), dtype=np.uint64).astype(np.uint32)
    qz = rng.integers(0, 2 ** 32, size=(groups, N // 8), dtype=np.uint64).astype(np.uint32)
    sc = rng.uniform(-0.03, 0.03, size=(groups, N)).astype(np.float32)
    got = _native(qw, qz, sc, torch.full((K, N), float("nan"), device=dev), g, dev)
    assert np.array_equal(got.view(np.uint32), oracle.dequant(qw, qz, sc, g, "seq").view(np.uint32))


@pytest.mark.parametrize("extra_lines,extra_words", [(1, 0), (3, 0), (2, 3), (0, 2)])
def test_dequantize_native_ragged_q_weight(dev, extra_lines, extra_words):
    # One unit per 4-word line of q_weight (numel / 4, rounded down): extra
    # lines fill the first 32 * extra_lines columns of one more output row;
    # 1..3 trailing words past the last whole line are ignored.
    K, N, g = 64, 256, 32
    rng = np.random.default_rng(11 + extra_lines)
    qw = rng.integers(0, 2 ** 32, size=((K + 1), N // 8), dtype=np.uint64).astype(np.uint32)
    qz = rng.integers(0, 2 ** 32, size=(K // g + 1, N // 8), dtype=np.uint64).astype(np.uint32)
    sc = rng.uniform(-0.03, 0.03, size=(K // g + 1, N)).astype(np.float32)
    words = K * N // 8 + 4 * extra_lines + extra_words
    n_out = K * N + 32 * extra_lines
    # out_width is the output's last dim; row K past the extra lines must stay NaN.
    out = torch.full((K + 1, N), float("nan"), device=dev)
    got = _native(qw.reshape(-1)[:words], qz, sc, out, g, dev).reshape(-1)
    ref = oracle.dequant(qw, qz, sc, g, "seq").reshape(-1)[:n_out]
    assert np.array_equal(got[:n_out].view(np.uint32), ref.view(np.uint32))
    assert np.isnan(got[n_out:]).all()
