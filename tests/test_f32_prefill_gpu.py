"""fp32 activations at prefill sizes (M > 16) on the f16 matrix cores.

The reference's own float type is f32 (its kernel tests and benchmark run
awq_gemm_linear::<R, f32>, src/kernel/awq_kernel_gemm.rs:870-960,
benches/awq_kernel_gemm.rs:303): x is split per row into f16 hi + lo under a
power-of-two row scale, multiplied with the exact integers q - z, and each
quantisation group's sum is scaled by s in fp32, so the result keeps fp32
accuracy: relative L2 <= 1e-5 against the oracle's f64 sum of the reference's
f32 weights (q - z) * s, the fp32 path's tolerance."""
import numpy as np
import pytest
import torch

import awq_oracle as oracle
import cube_awq
from cube_awq import _lib, pack
from helpers import TORCH_OF, host_f32, make_problem, to_device, to_host

pytestmark = pytest.mark.gpu

TOL_FP32 = 1e-5
AWQ_DT = {"f32": _lib.AWQ_F32, "f16": _lib.AWQ_F16, "bf16": _lib.AWQ_BF16}


def _i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(dev)


def gemm(dev, x, qw, qz, sc, b, M, K, N, g, s_dt="f16", y_dt="f32", fn="awq_gemm", order=None):
    d_x, d_sc = to_device(x, "f32", dev), to_device(sc, s_dt, dev)
    d_qw, d_qz = _i32(qw, dev), _i32(qz, dev)
    d_b = to_device(b, "f32", dev) if b is not None else None
    width = N // 2 if fn == "awq_gemm_silu_mul" else N
    y = torch.full((M, width), float("nan"), dtype=TORCH_OF[y_dt], device=dev)
    args = [d_x.data_ptr(), _lib.AWQ_F32, d_qw.data_ptr(), d_qz.data_ptr(), d_sc.data_ptr(), AWQ_DT[s_dt],
            d_b.data_ptr() if d_b is not None else None, _lib.AWQ_F32, y.data_ptr(), AWQ_DT[y_dt], M, K, N, g]
    if order is not None:
        args.append(order)
    _lib.check(getattr(cube_awq.lib(), fn)(*args, None))
    torch.cuda.synchronize()
    return host_f32(to_host(y), y_dt)


def ref64(x, qw, qz, sc, b, g, s_dt="f16", order="awq"):
    return oracle.gemm_f64(x, qw, qz, host_f32(sc, s_dt), g, bias=b, order=order)


# Default routes: 128 x 256 tiles (many tiles), 128 x 128 tiles with K
# splits (few tiles), ragged M and N.
@pytest.mark.parametrize("M,K,N", [(17, 4096, 4096), (64, 4096, 14336), (128, 4096, 4096), (200, 1024, 2080),
                                   (300, 14336, 1024), (512, 4096, 4096), (1000, 2048, 8192)])
def test_f32_prefill_default_routes(dev, M, K, N):
    x, qw, qz, sc, b = make_problem(M, K, N, 128, x_dt="f32", s_dt="f16", bias=True)
    y = gemm(dev, x, qw, qz, sc, b, M, K, N, 128)
    assert oracle.rel_l2(y, ref64(x, qw, qz, sc, b, 128)) <= TOL_FP32


@pytest.mark.parametrize("K,N", [(4096, 14336), (4096, 4096), (14336, 4096)])
def test_f32_prefill_m2048_sampled_rows(dev, K, N):
    M, g = 2048, 128
    x, qw, qz, sc, _ = make_problem(M, K, N, g, x_dt="f32", s_dt="f16")
    y = gemm(dev, x, qw, qz, sc, None, M, K, N, g)
    rows = np.r_[0:16, 1000:1016, 2032:2048]
    assert oracle.rel_l2(y[rows], ref64(x[rows], qw, qz, sc, None, g)) <= TOL_FP32


@pytest.mark.parametrize("tile", ["3", "4"])
@pytest.mark.parametrize("splits", ["1", "2", "3", "8"])
@pytest.mark.parametrize("g", [64, 128, 256])
def test_f32_prefill_every_tile_and_split(dev, monkeypatch, tile, splits, g):
    # Splits that start inside a quantisation group (3 splits of 16 stages,
    # g = 256 -> 4 stages per group) fold their partial group correctly.
    monkeypatch.setenv("AWQ_GEMM_TILE", tile)
    monkeypatch.setenv("AWQ_GEMM_SPLITS", splits)
    M, K, N = 150, 1024, 768
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt="f32", s_dt="f32", bias=True)
    y = gemm(dev, x, qw, qz, sc, b, M, K, N, g, s_dt="f32")
    assert oracle.rel_l2(y, ref64(x, qw, qz, sc, b, g, s_dt="f32")) <= TOL_FP32


@pytest.mark.parametrize("s_dt,y_dt,tol", [("f32", "f32", TOL_FP32), ("bf16", "f32", TOL_FP32),
                                           ("f16", "f16", 1e-3), ("f32", "bf16", 5e-3)])
def test_f32_prefill_scale_and_output_types(dev, s_dt, y_dt, tol):
    M, K, N, g = 96, 2048, 2048, 128
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt="f32", s_dt=s_dt, bias=True)
    y = gemm(dev, x, qw, qz, sc, b, M, K, N, g, s_dt=s_dt, y_dt=y_dt)
    assert oracle.rel_l2(y, ref64(x, qw, qz, sc, b, g, s_dt=s_dt)) <= tol


@pytest.mark.parametrize("row_scales", [(1e30, 1e-30, 7e4, 1e-20), (65504.0, 1e5, 2e-8, 1.0),
                                        (0.0, 3e-38, 1e36, 1.0)])
def test_f32_prefill_activation_magnitudes(dev, row_scales):
    """Rows far outside the f16 range and far below it, and an all-zero row,
    in one call: every output row keeps fp32 accuracy (a zero row gives
    exact zeros)."""
    M, K, N, g = 32, 1024, 1024, 128
    x, qw, qz, sc, _ = make_problem(M, K, N, g, x_dt="f32", s_dt="f16")
    scale = np.resize(np.asarray(row_scales, dtype=np.float64), M)
    x = (x.astype(np.float64) * scale[:, None]).astype(np.float32)
    y = gemm(dev, x, qw, qz, sc, None, M, K, N, g)
    ref = ref64(x, qw, qz, sc, None, g)
    for m in range(M):
        assert np.isfinite(y[m]).all(), m
        if scale[m] == 0:
            assert (y[m] == 0).all()
        else:
            assert oracle.rel_l2(y[m], ref[m]) <= TOL_FP32, (m, scale[m])


def test_f32_prefill_awq_like_statistics(dev):
    # Nibbles near their zero point and positive-mean activations (no
    # cancellation: the q - z operands are exact).
    rng = np.random.default_rng(5)
    M, K, N, g = 64, 4096, 4096, 128
    z = rng.integers(4, 12, size=(K // g, N))
    q = np.clip(np.repeat(z, g, axis=0) + np.rint(rng.normal(0, 1.0, size=(K, N))), 0, 15)
    qw, qz = pack.pack(q.astype(np.uint32), "awq"), pack.pack(z.astype(np.uint32), "awq")
    sc = rng.uniform(0.002, 0.02, size=(K // g, N)).astype(np.float16)
    x = (50.0 * (1.0 + 0.25 * rng.normal(size=(M, K)))).astype(np.float32)
    y = gemm(dev, x, qw, qz, sc, None, M, K, N, g)
    assert oracle.rel_l2(y, ref64(x, qw, qz, sc, None, g)) <= TOL_FP32


def test_f32_prefill_sequential_order(dev):
    # AWQLinear's layout (sequential nibbles, f32 scales: the reference's
    # single F = f32) on the same route.
    M, K, N, g = 130, 2048, 1024, 128
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt="f32", s_dt="f32", bias=True)
    y = gemm(dev, x, qw, qz, sc, b, M, K, N, g, s_dt="f32", fn="awq_gemm_ordered",
             order=_lib.AWQ_ORDER_SEQUENTIAL)
    assert oracle.rel_l2(y, ref64(x, qw, qz, sc, b, g, s_dt="f32", order="seq")) <= TOL_FP32


def test_f32_prefill_silu_mul(dev):
    M, K, N, g = 100, 2048, 2048, 128
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt="f32", s_dt="f16", bias=True)
    y = gemm(dev, x, qw, qz, sc, b, M, K, N, g, fn="awq_gemm_silu_mul")
    r = ref64(x, qw, qz, sc, b, g)
    gate, up = r[:, 0::2], r[:, 1::2]
    assert oracle.rel_l2(y, gate / (1.0 + np.exp(-gate)) * up) <= 2 * TOL_FP32


def test_f32_prefill_repeated_calls_bit_identical(dev):
    M, K, N, g = 256, 4096, 4096, 128
    x, qw, qz, sc, _ = make_problem(M, K, N, g, x_dt="f32", s_dt="f16")
    a = gemm(dev, x, qw, qz, sc, None, M, K, N, g)
    b = gemm(dev, x, qw, qz, sc, None, M, K, N, g)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# The reference's own benchmark cases (benches/awq_kernel_gemm.rs:575-685,
# Qwen2-0.5B projections, f32 everything, group 128), with its input
# generators (:160-215): x = ((i % 31) - 15) / 16; weight nibble
# (row + col + offset) % 15 + 1; zero nibble (group * 3 + col + offset) % 8;
# scale 0.02 + ((group * 17 + col) % 23) * 0.01; nibbles packed with nibble
# `offset` at bits 4 * offset (pack8, :153-157).
def _pack8(nib):
    shifts = (np.arange(8, dtype=np.uint64) * 4)[None, None, :]
    return np.bitwise_or.reduce(nib.astype(np.uint64) << shifts, axis=2).astype(np.uint32)


def reference_bench_case(M, K, N, g=128):
    x = ((np.arange(M * K) % 31).astype(np.float32) - 15.0) * 0.0625
    r, c, o = np.meshgrid(np.arange(K), np.arange(N // 8), np.arange(8), indexing="ij")
    qw = _pack8((r + c + o) % 15 + 1)
    gr, gc, go = np.meshgrid(np.arange(K // g), np.arange(N // 8), np.arange(8), indexing="ij")
    qz = _pack8((gr * 3 + gc + go) % 8)
    sg, sn = np.meshgrid(np.arange(K // g), np.arange(N), indexing="ij")
    sc = (np.float32(0.02) + ((sg * 17 + sn) % 23).astype(np.float32) * np.float32(0.01)).astype(np.float32)
    return x.reshape(M, K), qw, qz, sc


@pytest.mark.parametrize("M", [1, 8, 128, 512])
@pytest.mark.parametrize("K,N", [(896, 896), (896, 4864), (4864, 896)])
def test_reference_benchmark_cases(dev, M, K, N):
    x, qw, qz, sc = reference_bench_case(M, K, N)
    y = gemm(dev, x, qw, qz, sc, None, M, K, N, 128, s_dt="f32")
    assert oracle.rel_l2(y, ref64(x, qw, qz, sc, None, 128, s_dt="f32")) <= TOL_FP32
