"""awq_gemm_noalloc: awq_gemm with its split-K scratch in a static device
array instead of an allocated workspace. On every kernel route that splits
K it must give awq_gemm's bits, on two calls in a row (the second with a
smaller input), and refuse, before launching, a call whose partial sums do
not fit the scratch."""
import numpy as np
import pytest
import torch

import cube_awq
from cube_awq import _lib
from helpers import make_problem, to_device

pytestmark = pytest.mark.gpu

AWQ_DT = {"f32": _lib.AWQ_F32, "f16": _lib.AWQ_F16}
G = 128

# (M, K, N, x dtype, smaller M for the second call): decode VALU with K
# splits, 4x4x4 matrix-core decode, 16x16x32 decode tile, 9..16 rows, the
# skinny kernel with K splits, large tiles with K splits, fp32 16-row slices,
# a large-tile prefill with no split, both matrix-core decode kernels with
# the two-level split sum (28 splits over 8 column chunks), and the skinny
# kernel with it (16 splits).
CASES = [(1, 4096, 4096, "f32", 1), (4, 4096, 14336, "f32", 2), (8, 8192, 8192, "f32", 5),
         (16, 4096, 4096, "f16", 9), (64, 4096, 14336, "f16", 24), (300, 1024, 1024, "f16", 130),
         (40, 4096, 4096, "f32", 17), (512, 4096, 4096, "f16", 256), (8, 14336, 4096, "f32", 6),
         (4, 14336, 4096, "f32", 3), (64, 14336, 4096, "f16", 24)]


def _i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(dev)


def _call(fn, x, xt, qw, qz, sc, b, y, M, K, N):
    return fn(x.data_ptr(), xt, qw.data_ptr(), qz.data_ptr(), sc.data_ptr(), _lib.AWQ_F16,
              b.data_ptr(), _lib.AWQ_F32, y.data_ptr(), _lib.AWQ_F32, M, K, N, G,
              torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("M,K,N,xdt,M2", CASES)
def test_noalloc_matches_awq_gemm(dev, M, K, N, xdt, M2):
    L = cube_awq.lib()
    x, qw, qz, sc, b = make_problem(M, K, N, G, x_dt=xdt, s_dt="f16", bias=True)
    d_x, d_qw, d_qz = to_device(x, xdt, dev), _i32(qw, dev), _i32(qz, dev)
    d_sc, d_b = to_device(sc, "f16", dev), to_device(b, "f32", dev)
    ref1 = torch.full((M, N), float("nan"), device=dev)
    ref2 = torch.full((M2, N), float("nan"), device=dev)
    _lib.check(_call(L.awq_gemm, d_x, AWQ_DT[xdt], d_qw, d_qz, d_sc, d_b, ref1, M, K, N))
    _lib.check(_call(L.awq_gemm, d_x[M - M2:], AWQ_DT[xdt], d_qw, d_qz, d_sc, d_b, ref2, M2, K, N))
    got1 = torch.full((M, N), float("nan"), device=dev)
    got2 = torch.full((M2, N), float("nan"), device=dev)
    # Two calls in a row on one stream, the second smaller: it must not see
    # anything the first left in the shared scratch.
    _lib.check(_call(L.awq_gemm_noalloc, d_x, AWQ_DT[xdt], d_qw, d_qz, d_sc, d_b, got1, M, K, N))
    _lib.check(_call(L.awq_gemm_noalloc, d_x[M - M2:], AWQ_DT[xdt], d_qw, d_qz, d_sc, d_b, got2, M2, K, N))
    torch.cuda.synchronize()
    assert torch.isfinite(ref1).all() and torch.isfinite(ref2).all()
    assert torch.equal(got1.view(torch.int32), ref1.view(torch.int32)), (M, K, N)
    assert torch.equal(got2.view(torch.int32), ref2.view(torch.int32)), (M2, K, N)


def test_noalloc_graph_replays(dev):
    # The callers it is for: capture under a graph (no allocation may happen
    # there), replay several times with eager work in between.
    L = cube_awq.lib()
    M, K, N = 4, 4096, 14336
    x, qw, qz, sc, b = make_problem(M, K, N, G, x_dt="f32", s_dt="f16", bias=True)
    d_x, d_qw, d_qz = to_device(x, "f32", dev), _i32(qw, dev), _i32(qz, dev)
    d_sc, d_b = to_device(sc, "f16", dev), to_device(b, "f32", dev)
    ref = torch.empty((M, N), device=dev)
    y = torch.empty((M, N), device=dev)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        _lib.check(_call(L.awq_gemm, d_x, _lib.AWQ_F32, d_qw, d_qz, d_sc, d_b, ref, M, K, N))
        _lib.check(_call(L.awq_gemm_noalloc, d_x, _lib.AWQ_F32, d_qw, d_qz, d_sc, d_b, y, M, K, N))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        _lib.check(_call(L.awq_gemm_noalloc, d_x, _lib.AWQ_F32, d_qw, d_qz, d_sc, d_b, y, M, K, N))
    for rep in range(3):
        with torch.cuda.stream(stream):
            y.fill_(float("nan"))
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), ref.view(torch.int32)), rep
        with torch.cuda.stream(stream):  # eager noalloc work between replays, same scratch
            _lib.check(_call(L.awq_gemm_noalloc, d_x[:1], _lib.AWQ_F32, d_qw, d_qz, d_sc, d_b, y[:1],
                             1, K, N))
        torch.cuda.synchronize()


def test_noalloc_rejects_more_partials_than_the_scratch(dev, monkeypatch):
    # 128 x 128 tiles with 8 forced K splits at M = 512, N = 8192: 8 x 512 x
    # 8192 x 4 bytes = 128 MiB of partials, past the 63 MiB the scratch holds.
    # Refused before any launch (the output keeps its NaNs); awq_gemm runs it.
    monkeypatch.setenv("AWQ_GEMM_TILE", "4")
    monkeypatch.setenv("AWQ_GEMM_SPLITS", "8")
    L = cube_awq.lib()
    M, K, N = 512, 4096, 8192
    x, qw, qz, sc, b = make_problem(M, K, N, G, x_dt="f16", s_dt="f16", bias=True)
    d_x, d_qw, d_qz = to_device(x, "f16", dev), _i32(qw, dev), _i32(qz, dev)
    d_sc, d_b = to_device(sc, "f16", dev), to_device(b, "f32", dev)
    y = torch.full((M, N), float("nan"), device=dev)
    rc = _call(L.awq_gemm_noalloc, d_x, _lib.AWQ_F16, d_qw, d_qz, d_sc, d_b, y, M, K, N)
    torch.cuda.synchronize()
    assert rc == _lib.AWQ_ERR_INVALID
    msg = L.awq_last_error().decode()
    assert "awq_gemm_noalloc" in msg and "partial sums" in msg and "static scratch" in msg, msg
    assert torch.isnan(y).all()
    _lib.check(_call(L.awq_gemm, d_x, _lib.AWQ_F16, d_qw, d_qz, d_sc, d_b, y, M, K, N))
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
