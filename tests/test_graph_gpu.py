"""Calls captured in a HIP graph and replayed give the eager results, bit for
bit, on every kernel route with split-K handshakes (decode VALU and matrix
core, skinny, large tiles) and the gate/up SiLU epilogue: the arrival
counters are re-armed by the kernels themselves, so replays need no memset
(none may be recorded in a graph). Between replays the outputs are refilled
and other eager work runs on the same stream."""
import numpy as np
import pytest
import torch

import cube_awq
from cube_awq import _lib
from helpers import make_problem, to_device

pytestmark = pytest.mark.gpu

AWQ_DT = {"f32": _lib.AWQ_F32, "f16": _lib.AWQ_F16}

# (M, K, N, x dtype, silu): decode VALU with K splits, matrix-core decode,
# 9..16 rows, skinny with K splits, large tiles with K splits, SiLU epilogue
CASES = [(1, 4096, 4096, "f32", False), (4, 4096, 4096, "f32", False), (16, 2048, 2048, "f16", False),
         (40, 4096, 8192, "f16", False), (300, 1024, 1024, "f16", False), (1, 2048, 2048, "f32", True),
         (64, 2048, 8192, "f16", True)]


def _i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(dev)


def test_graph_replays_match_eager(dev):
    L = cube_awq.lib()
    g_size = 128
    items = []
    for (M, K, N, xdt, silu) in CASES:
        x, qw, qz, sc, b = make_problem(M, K, N, g_size, x_dt=xdt, s_dt="f16", bias=True)
        width = N // 2 if silu else N
        items.append(dict(M=M, K=K, N=N, xt=AWQ_DT[xdt], fn=L.awq_gemm_silu_mul if silu else L.awq_gemm,
                          x=to_device(x, xdt, dev), qw=_i32(qw, dev), qz=_i32(qz, dev),
                          sc=to_device(sc, "f16", dev), b=to_device(b, "f32", dev),
                          y=torch.empty((M, width), dtype=torch.float32, device=dev)))

    def launch(it):
        _lib.check(it["fn"](it["x"].data_ptr(), it["xt"], it["qw"].data_ptr(), it["qz"].data_ptr(),
                            it["sc"].data_ptr(), _lib.AWQ_F16, it["b"].data_ptr(), _lib.AWQ_F32,
                            it["y"].data_ptr(), _lib.AWQ_F32, it["M"], it["K"], it["N"], g_size,
                            torch.cuda.current_stream().cuda_stream))

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):  # eager reference; also sizes the stream's workspace
        for it in items:
            launch(it)
    torch.cuda.synchronize()
    refs = [it["y"].clone() for it in items]

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for it in items:
            launch(it)
    for rep in range(3):
        with torch.cuda.stream(stream):
            for it in items:
                it["y"].fill_(float("nan"))
            graph.replay()
        torch.cuda.synchronize()
        for it, ref in zip(items, refs):
            assert torch.equal(it["y"].view(torch.int32), ref.view(torch.int32)), (rep, it["M"], it["N"])
        with torch.cuda.stream(stream):  # eager work between replays, same kernels and workspace
            launch(items[rep % len(items)])
        torch.cuda.synchronize()


def test_graph_replay_after_workspace_growth(dev):
    """A graph captured with the stream's split-K workspace at one size keeps
    working after a larger eager call on the same stream has replaced that
    workspace: superseded buffers are retired, never freed, so the replay
    still writes memory it owns and reproduces the eager result bit for
    bit. The serving pattern: capture at one batch size, warm up another
    eagerly, replay the first."""
    L = cube_awq.lib()
    g_size = 128

    def problem(M, K, N, xdt):
        x, qw, qz, sc, _ = make_problem(M, K, N, g_size, x_dt=xdt, s_dt="f16")
        return dict(M=M, K=K, N=N, xt=AWQ_DT[xdt], x=to_device(x, xdt, dev), qw=_i32(qw, dev),
                    qz=_i32(qz, dev), sc=to_device(sc, "f16", dev),
                    y=torch.empty((M, N), dtype=torch.float32, device=dev))

    def launch(it):
        _lib.check(L.awq_gemm(it["x"].data_ptr(), it["xt"], it["qw"].data_ptr(), it["qz"].data_ptr(),
                              it["sc"].data_ptr(), _lib.AWQ_F16, None, _lib.AWQ_F32, it["y"].data_ptr(),
                              _lib.AWQ_F32, it["M"], it["K"], it["N"], g_size,
                              torch.cuda.current_stream().cuda_stream))

    # Small: M = 1 decode with K splits (a few hundred KB of partials at
    # most). Large: 8 rows, 8192 -> 28672 (several MB of partials) and a
    # 64-row skinny split-K call, each larger than anything before it.
    small = problem(1, 4096, 4096, "f32")
    larger = [problem(8, 8192, 28672, "f32"), problem(64, 8192, 28672, "f16")]
    stream = torch.cuda.Stream()  # a fresh stream: its workspace starts empty
    with torch.cuda.stream(stream):
        launch(small)
    torch.cuda.synchronize()
    ref_small = small["y"].clone()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        launch(small)

    refs_large = []
    for big in larger:
        with torch.cuda.stream(stream):  # grows the workspace the graph captured
            launch(big)
        torch.cuda.synchronize()
        refs_large.append(big["y"].clone())
        for rep in range(2):
            with torch.cuda.stream(stream):
                small["y"].fill_(float("nan"))
                graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(small["y"].view(torch.int32), ref_small.view(torch.int32)), (big["M"], rep)

    # The larger calls still compute their own results on the new buffers,
    # interleaved with replays.
    for big, ref in zip(larger, refs_large):
        with torch.cuda.stream(stream):
            big["y"].fill_(float("nan"))
            launch(big)
            graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(big["y"].view(torch.int32), ref.view(torch.int32)), big["M"]
        assert torch.equal(small["y"].view(torch.int32), ref_small.view(torch.int32))
