"""Decode numerics on AWQ-like statistics, all decode routes.

Real AWQ checkpoints put most nibbles within one or two steps of their zero
point, and transformer activations are not zero-mean. A decode kernel that
factored the zero point out of its sum (s * (sum x q - z sum x)) would
cancel catastrophically there; every route here forms q - z exactly before
the multiply, as the reference's dequantize does ((q - z) * s,
src/kernel/awq_kernel_gemm.rs:553-606), so accuracy does not depend on the
activations' mean, and columns whose weights all equal their zero point come
out exactly zero, as they do in the reference."""
import numpy as np
import pytest
import torch

import awq_oracle as oracle
import cube_awq
from cube_awq import _lib, pack, synth
from helpers import to_device, to_host

pytestmark = pytest.mark.gpu

TOL_FP32 = 1e-5

# (rows, overrides): M = 1 VALU kernel; 2 rows of a small matrix (VALU);
# 4 rows on the 4x4x4 blocks; 8 rows on the 16x16x32 tile; 4 rows forced
# onto the VALU kernel (its many-row variant).
ROUTES = {"valu_m1": (1, {}), "valu_m2": (2, {}), "m4": (4, {}), "mfma16": (8, {}),
          "valu_m4": (4, {"AWQ_DECODE_MFMA": "0"})}


def awq_like_problem(M, K, N, g, sigma, mean, seed):
    rng = np.random.default_rng(seed)
    z = rng.integers(4, 12, size=(K // g, N))
    q = np.clip(np.repeat(z, g, axis=0) + np.rint(rng.normal(0.0, sigma, size=(K, N))), 0, 15)
    zero_cols = np.arange(5, N, 37)
    q[:, zero_cols] = np.repeat(z[:, zero_cols], g, axis=0)  # q == z everywhere in these columns
    qw = pack.pack(q.astype(np.uint32), "awq")
    qz = pack.pack(z.astype(np.uint32), "awq")
    sc = rng.uniform(0.002, 0.02, size=(K // g, N)).astype(np.float16)
    x = (mean * (1.0 + 0.25 * rng.normal(size=(M, K)))).astype(np.float32)
    return x, qw, qz, sc, zero_cols


def run(dev, x, qw, qz, sc, M, K, N, g):
    d_x, d_sc = to_device(x, "f32", dev), to_device(sc, "f16", dev)
    d_qw = torch.from_numpy(qw.view(np.int32)).to(dev)
    d_qz = torch.from_numpy(qz.view(np.int32)).to(dev)
    y = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    _lib.check(cube_awq.lib().awq_gemm(d_x.data_ptr(), _lib.AWQ_F32, d_qw.data_ptr(), d_qz.data_ptr(),
                                       d_sc.data_ptr(), _lib.AWQ_F16, None, _lib.AWQ_F32, y.data_ptr(),
                                       _lib.AWQ_F32, M, K, N, g, None))
    torch.cuda.synchronize()
    return to_host(y)


@pytest.mark.parametrize("route", list(ROUTES))
@pytest.mark.parametrize("mean", [1.0, 5.0, 50.0])
@pytest.mark.parametrize("sigma", [0.7, 1.5])
def test_decode_awq_like_statistics(dev, monkeypatch, route, mean, sigma):
    M, over = ROUTES[route]
    for k, v in over.items():
        monkeypatch.setenv(k, v)
    K, N, g = 4096, 4096, 128
    x, qw, qz, sc, zero_cols = awq_like_problem(M, K, N, g, sigma, mean, seed=int(mean * 10 + sigma * 100))
    y = run(dev, x, qw, qz, sc, M, K, N, g)
    ref = oracle.gemm_f64(x, qw, qz, sc.astype(np.float32), g)
    assert np.isfinite(y).all()
    assert oracle.rel_l2(y, ref) <= TOL_FP32, (route, mean, sigma)
    assert (y[:, zero_cols] == 0).all(), (route, mean, sigma)


def test_decode_m1_gate_up_awq_like(dev):
    # The headline decode shape (4096 -> 14336) with mean-50 activations.
    M, K, N, g = 1, 4096, 14336, 128
    x, qw, qz, sc, zero_cols = awq_like_problem(M, K, N, g, 1.0, 50.0, seed=7)
    y = run(dev, x, qw, qz, sc, M, K, N, g)
    assert oracle.rel_l2(y, oracle.gemm_f64(x, qw, qz, sc.astype(np.float32), g)) <= TOL_FP32
    assert (y[:, zero_cols] == 0).all()


def test_decode_m1_reference_closed_forms_large_k(dev):
    # src/kernel/awq_kernel_gemm.rs:1125-1316 closed forms at a decode shape:
    # x = 1, uniform w and z, s = 1 -> (w - z) * K exactly (all partial sums
    # are small integers, exact in f32).
    K, N, g = 4096, 1024, 128
    for w, z, expect in ((5, 0, 5 * K), (8, 3, 5 * K), (2, 7, -5 * K), (0, 15, -15 * K), (9, 9, 0)):
        qw = np.full((K, N // 8), int(("%x" % w) * 8, 16), dtype=np.uint32)
        qz = np.full((K // g, N // 8), int(("%x" % z) * 8, 16), dtype=np.uint32)
        sc = np.ones((K // g, N), dtype=np.float16)
        x = np.ones((1, K), dtype=np.float32)
        y = run(dev, x, qw, qz, sc, 1, K, N, g)
        assert (y == expect).all(), (w, z)
