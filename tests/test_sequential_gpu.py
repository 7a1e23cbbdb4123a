"""Sequential nibble order through the fused kernels: awq_gemm_ordered and
AWQLinear.forward (the reference's AWQLinear dequantizes in this order and
then multiplies, src/modules/awq_dequantize.rs:74-108).

Checked two ways: against the f64 oracle summing the sequentially unpacked
weights (same tolerances as the AutoAWQ-order tests), and bit for bit against
awq_gemm on the same logical weights packed in AutoAWQ order: the kernels
give every output column the same arithmetic in the same order whichever
packed lane holds it, so the two outputs must be identical."""
import numpy as np
import pytest
import torch

import awq_oracle as oracle
import cube_awq
from cube_awq import AWQLinear, _lib, pack
from helpers import TORCH_OF, host_f32, make_problem, to_device, to_host

pytestmark = pytest.mark.gpu

TOL_FP32 = 1e-5
TOL_MFMA = 2e-3
AWQ_DT = {"f32": _lib.AWQ_F32, "f16": _lib.AWQ_F16, "bf16": _lib.AWQ_BF16}


def _i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(dev)


def _to_seq(words):
    """Repack AutoAWQ-order words as sequential-order words (same logical nibbles)."""
    return pack.pack(pack.unpack(words, "awq"), "seq")


def _run(dev, x, qw, qz, sc, b, M, K, N, g, dt, order, y_dt=None):
    y_dt = y_dt or dt
    d_x, d_sc = to_device(x, dt, dev), to_device(sc, dt, dev)
    d_qw, d_qz = _i32(qw, dev), _i32(qz, dev)
    d_b = to_device(b, "f32", dev) if b is not None else None
    y = torch.full((M, N), float("nan"), dtype=TORCH_OF[y_dt], device=dev)
    _lib.check(cube_awq.lib().awq_gemm_ordered(
        d_x.data_ptr(), AWQ_DT[dt], d_qw.data_ptr(), d_qz.data_ptr(), d_sc.data_ptr(), AWQ_DT[dt],
        d_b.data_ptr() if d_b is not None else None, _lib.AWQ_F32, y.data_ptr(), AWQ_DT[y_dt],
        M, K, N, g, order, None))
    torch.cuda.synchronize()
    return to_host(y)


@pytest.mark.parametrize("M", [1, 2, 3, 5, 8, 9, 64, 300])
@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_sequential_matches_oracle_and_autoawq_bits(dev, M, dt):
    K, N, g = 1024, 1056, 64
    x, qw_awq, qz_awq, sc, b = make_problem(M, K, N, g, x_dt=dt, s_dt=dt, bias=True)
    qw_seq, qz_seq = _to_seq(qw_awq), _to_seq(qz_awq)
    y_seq = _run(dev, x, qw_seq, qz_seq, sc, b, M, K, N, g, dt, _lib.AWQ_ORDER_SEQUENTIAL, "f32")
    y_awq = _run(dev, x, qw_awq, qz_awq, sc, b, M, K, N, g, dt, _lib.AWQ_ORDER_AUTOAWQ, "f32")
    assert np.array_equal(y_seq.view(np.uint32), y_awq.view(np.uint32))
    ref = oracle.gemm_f64(host_f32(x, dt), qw_seq, qz_seq, host_f32(sc, dt), g, bias=b, order="seq")
    tol = TOL_FP32 if (dt == "f32" or M <= 8) else TOL_MFMA
    assert oracle.rel_l2(y_seq, ref) <= tol


@pytest.mark.parametrize("M,dt", [(1, "f32"), (4, "f32"), (8, "f16"), (12, "f32")])
def test_sequential_deep_k_split_sums(dev, monkeypatch, M, dt):
    """Deep K on the decode kernels (36..72 K splits): the grouped one-row sum
    and, forced here, the two-level sum of the matrix-core kernels, in
    sequential order against AutoAWQ order (same bits) and the oracle."""
    monkeypatch.setenv("AWQ_DECODE_TREE", "1")
    K, N, g = 9216, 1056, 128
    x, qw_awq, qz_awq, sc, b = make_problem(M, K, N, g, x_dt=dt, s_dt=dt, bias=True)
    qw_seq, qz_seq = _to_seq(qw_awq), _to_seq(qz_awq)
    y_seq = _run(dev, x, qw_seq, qz_seq, sc, b, M, K, N, g, dt, _lib.AWQ_ORDER_SEQUENTIAL, "f32")
    y_awq = _run(dev, x, qw_awq, qz_awq, sc, b, M, K, N, g, dt, _lib.AWQ_ORDER_AUTOAWQ, "f32")
    assert np.array_equal(y_seq.view(np.uint32), y_awq.view(np.uint32))
    ref = oracle.gemm_f64(host_f32(x, dt), qw_seq, qz_seq, host_f32(sc, dt), g, bias=b, order="seq")
    assert oracle.rel_l2(y_seq, ref) <= TOL_FP32


@pytest.mark.parametrize("tile", [1, 2, 3, 4, 6, 7, 8, 9, 10, 11, 12])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_sequential_every_tile_configuration(dev, monkeypatch, tile, dt):
    monkeypatch.setenv("AWQ_GEMM_TILE", str(tile))
    M, K, N, g = 300, 512, 672, 128
    x, qw_awq, qz_awq, sc, _ = make_problem(M, K, N, g, x_dt=dt, s_dt=dt)
    qw_seq, qz_seq = _to_seq(qw_awq), _to_seq(qz_awq)
    y_seq = _run(dev, x, qw_seq, qz_seq, sc, None, M, K, N, g, dt, _lib.AWQ_ORDER_SEQUENTIAL, "f32")
    y_awq = _run(dev, x, qw_awq, qz_awq, sc, None, M, K, N, g, dt, _lib.AWQ_ORDER_AUTOAWQ, "f32")
    assert np.array_equal(y_seq.view(np.uint32), y_awq.view(np.uint32))
    ref = oracle.gemm_f64(host_f32(x, dt), qw_seq, qz_seq, host_f32(sc, dt), g, order="seq")
    assert oracle.rel_l2(y_seq, ref) <= TOL_MFMA


@pytest.mark.parametrize("M", [17, 64, 128])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("chunk", [{}, {"AWQ_SKINNY_COLS": "256"}])
def test_sequential_skinny_kernel(dev, monkeypatch, M, dt, chunk):
    """17..128 rows of f16 or bf16 on the skinny kernel, forced on at a narrow N."""
    monkeypatch.setenv("AWQ_SKINNY", "1")
    for k, v in chunk.items():
        monkeypatch.setenv(k, v)
    K, N, g = 2048, 2080, 128
    x, qw_awq, qz_awq, sc, b = make_problem(M, K, N, g, x_dt=dt, s_dt=dt, bias=True)
    qw_seq, qz_seq = _to_seq(qw_awq), _to_seq(qz_awq)
    y_seq = _run(dev, x, qw_seq, qz_seq, sc, b, M, K, N, g, dt, _lib.AWQ_ORDER_SEQUENTIAL, "f32")
    y_awq = _run(dev, x, qw_awq, qz_awq, sc, b, M, K, N, g, dt, _lib.AWQ_ORDER_AUTOAWQ, "f32")
    assert np.array_equal(y_seq.view(np.uint32), y_awq.view(np.uint32))
    ref = oracle.gemm_f64(host_f32(x, dt), qw_seq, qz_seq, host_f32(sc, dt), g, bias=b, order="seq")
    assert oracle.rel_l2(y_seq, ref) <= TOL_MFMA


def test_sequential_rejects_mixed_scale_dtype(dev):
    L = cube_awq.lib()
    rc = L.awq_gemm_ordered(None, _lib.AWQ_F16, None, None, None, _lib.AWQ_F32, None, 0, None,
                            _lib.AWQ_F16, 16, 64, 32, 64, _lib.AWQ_ORDER_SEQUENTIAL, None)
    assert rc == _lib.AWQ_ERR_INVALID
    assert "sequential-order GEMM needs scales in the input dtype" in L.awq_last_error().decode()
    rc = L.awq_gemm_ordered(None, _lib.AWQ_F16, None, None, None, _lib.AWQ_F16, None, 0, None,
                            _lib.AWQ_F16, 16, 64, 32, 64, 7, None)
    assert rc == _lib.AWQ_ERR_INVALID and "order must be" in L.awq_last_error().decode()


@pytest.mark.parametrize("M", [1, 4, 130])
@pytest.mark.parametrize("dt", ["f32", "f16"])
def test_linear_forward_fused_matches_dequantize_matmul(dev, M, dt):
    """AWQLinear.forward (fused, sequential order) against the reference's
    two steps: its own bit-exact dequantize() and a float64 matmul."""
    K, N, g = 4096, 1024, 128
    x, qw_awq, qz_awq, sc, _ = make_problem(M, K, N, g, x_dt=dt, s_dt=dt)
    layer = AWQLinear(_i32(_to_seq(qw_awq), dev), _i32(_to_seq(qz_awq), dev), to_device(sc, dt, dev))
    xd = to_device(x, dt, dev)
    assert layer._fusable(xd, M, K, N)
    y = layer.forward(xd)
    w = layer.dequantize()
    torch.cuda.synchronize()
    assert y.dtype == xd.dtype and tuple(y.shape) == (M, N)
    ref = host_f32(x, dt).astype(np.float64) @ w.float().cpu().numpy().astype(np.float64)
    got = y.float().cpu().numpy()
    tol = TOL_FP32 if dt == "f32" else 1e-3  # f16 output: one rounding of ~2^-11
    assert oracle.rel_l2(got, ref) <= tol


def test_linear_forward_unfusable_shape_uses_dequantize_matmul(dev):
    """The reference's g = 2 test layer is below the fused kernels' g >= 64:
    forward takes dequantize() + matmul and still meets the reference's
    1e-3 (src/modules/awq_dequantize.rs:239-281)."""
    from conftest import load_golden
    gd = load_golden("dequant_seq_64x32_g2")
    layer = AWQLinear(_i32(gd["qweight"], dev), _i32(gd["qzeros"], dev), torch.from_numpy(gd["scales"]).to(dev))
    x = (torch.arange(2 * 64, dtype=torch.float32) * 0.01).reshape(2, 64).to(dev)
    assert not layer._fusable(x, 2, 64, 32)
    y = layer.forward(x)
    torch.cuda.synchronize()
    expect = x.cpu().double() @ torch.from_numpy(gd["expected"]).double()
    assert (y.cpu().double() - expect).abs().max().item() <= 1e-3
