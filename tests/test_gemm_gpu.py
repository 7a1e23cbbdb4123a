"""Fused AWQ dequant-GEMM on the GPU vs the oracle.

Tolerances (relative L2 against the oracle's f64 sum of the reference's f32
dequantised weights):
  fp32 path (f32 activations, decode GEMV and fp32-MFMA prefill): 1e-5
  fp16/bf16-MFMA prefill path:                                     2e-3
Plus the reference's own absolute tolerances on its own cases
(src/kernel/awq_kernel_gemm.rs:1125-1391, src/modules/awq_gemm.rs:408-604)."""
import numpy as np
import pytest
import torch

import awq_oracle as oracle
import cube_awq
from cube_awq import AWQGEMMLinear, ShapeConfig, _lib, synth
from conftest import load_golden
from helpers import TORCH_OF, host_f32, make_problem, round_to, to_device, to_host

pytestmark = pytest.mark.gpu

TOL_FP32 = 1e-5
TOL_MFMA = 2e-3
AWQ_DT = {"f32": _lib.AWQ_F32, "f16": _lib.AWQ_F16, "bf16": _lib.AWQ_BF16}


def _i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(dev)


def run_kernel(dev, x, qw, qz, sc, m, k, n, gs, tile_m=32):
    """The reference's run_kernel (src/kernel/awq_kernel_gemm.rs:870-960):
    ShapeConfig(rows, n, k, 32, tile_n, inner_k) through awq_gemm_linear, f32."""
    inner_k = 64 if (k >= 64 and k % 64 == 0 and gs >= 64 and gs % 64 == 0) else 32
    tile_n = 128 if (n >= 128 and n % 128 == 0) else 64 if (n >= 64 and n % 64 == 0) else 32
    shape = ShapeConfig.new(m, n, k, tile_m, tile_n, inner_k)
    out = torch.full((m, n), float("nan"), device=dev)
    cube_awq.awq_gemm_linear(torch.from_numpy(x).to(dev), _i32(qw, dev), _i32(qz, dev),
                             torch.from_numpy(sc).to(dev), out, shape, gs)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def uniform_word(v):
    return int(("%x" % v) * 8, 16)


@pytest.mark.parametrize("m,k,n,gs,w,z,s,xv,tol", [
    (32, 32, 32, 32, 7, 0, 1.0, 0.0, 1e-5),    # kernel_zero_input_yields_zero_output
    (32, 32, 32, 32, 5, 5, 2.0, 1.0, 1e-5),    # kernel_zero_weight_yields_zero_output
    (32, 32, 32, 32, 15, 0, 0.0, 1.0, 1e-5),   # kernel_zero_scale_yields_zero_output
    (32, 32, 32, 32, 5, 0, 1.0, 1.0, 1e-3),    # kernel_ones_input_uniform_weight_single_tile
    (32, 32, 32, 32, 8, 3, 2.0, 1.0, 1e-3),    # kernel_uniform_with_nonzero_zero_point
    (32, 32, 32, 32, 2, 7, 1.0, 1.0, 1e-3),    # kernel_negative_effective_weight
    (32, 32, 32, 32, 15, 0, 1.0, 1.0, 1e-3),   # kernel_weight_nibble_at_max_15
    (32, 32, 32, 32, 0, 15, 1.0, 1.0, 1e-3),   # kernel_weight_nibble_zero_zeropoint_fifteen
    (32, 64, 32, 64, 4, 1, 1.0, 1.0, 1e-2),    # kernel_two_k_tiles
    (32, 128, 32, 128, 6, 2, 0.25, 0.5, 1e-2), # kernel_four_k_tiles
    (32, 64, 32, 32, 5, 1, 1.0, 1.0, 1e-2),    # kernel_two_groups_uniform_scale
    (64, 32, 32, 32, 5, 0, 1.0, 1.0, 1e-3),    # kernel_m_double_n_single_tile
    (1, 32, 32, 32, 5, 0, 1.0, 1.0, 1e-3),     # kernel_m_one_partial_tile
    (32, 32, 64, 32, 3, 1, 2.0, 1.0, 1e-3),    # kernel_n_double_m_single_tile
])
def test_reference_kernel_uniform_cases(dev, m, k, n, gs, w, z, s, xv, tol):
    qw = np.full((k, n // 8), uniform_word(w), np.uint32)
    qz = np.full((k // gs, n // 8), uniform_word(z), np.uint32)
    sc = np.full((k // gs, n), s, np.float32)
    x = np.full((m, k), xv, np.float32)
    out = run_kernel(dev, x, qw, qz, sc, m, k, n, gs)
    expect = oracle.gemm_f32(x, qw, qz, sc, gs)
    assert np.abs(out - expect).max() <= tol
    assert np.array_equal(out, np.full((m, n), k * xv * (w - z) * s, np.float32))


def test_reference_kernel_two_groups_different_scales(dev):
    m, k, n, gs = 32, 64, 32, 32
    qw = np.full((k, n // 8), uniform_word(6), np.uint32)
    qz = np.full((k // gs, n // 8), uniform_word(2), np.uint32)
    sc = np.concatenate([np.full((1, n), 1.0), np.full((1, n), 0.5)]).astype(np.float32)
    out = run_kernel(dev, np.ones((m, k), np.float32), qw, qz, sc, m, k, n, gs)
    assert np.abs(out - oracle.gemm_f32(np.ones((m, k), np.float32), qw, qz, sc, gs)).max() <= 1e-2


def test_reference_kernel_four_groups(dev):
    m, k, n, gs = 32, 128, 32, 32
    qw = np.full((k, n // 8), uniform_word(7), np.uint32)
    qz = np.full((k // gs, n // 8), uniform_word(3), np.uint32)
    sc = np.repeat((np.arange(1, 5, dtype=np.float32) * 0.25)[:, None], n, 1)
    x = np.ones((m, k), np.float32)
    assert np.abs(run_kernel(dev, x, qw, qz, sc, m, k, n, gs) - oracle.gemm_f32(x, qw, qz, sc, gs)).max() <= 1e-1


def test_reference_kernel_large_m_large_n(dev):
    g = load_golden("gemm_large_m_large_n")
    out = run_kernel(dev, g["x"], g["qweight"], g["qzeros"], g["scales"], 128, 32, 128, 32)
    assert np.abs(out - g["expected"]).max() <= 1e-1
    assert oracle.rel_l2(out, g["expected"]) <= TOL_FP32


def test_reference_kernel_two_batches(dev):
    # kernel_two_batches_match_cpu_ref: b=2 flattened into 64 rows.
    m, k, n, gs = 64, 32, 32, 32
    x = np.concatenate([np.ones((32, k)), np.full((32, k), 2.0)]).astype(np.float32)
    qw = np.full((k, n // 8), uniform_word(5), np.uint32)
    qz = np.full((k // gs, n // 8), uniform_word(1), np.uint32)
    sc = np.full((k // gs, n), 0.5, np.float32)
    out = run_kernel(dev, x, qw, qz, sc, m, k, n, gs)
    assert np.abs(out - oracle.gemm_f32(x, qw, qz, sc, gs)).max() <= 1e-3


@pytest.mark.parametrize("name", ["gemm_fwd_b2m32_k64n32_g32", "gemm_fwd_bias_b2m32_k64n32_g32",
                                  "gemm_fwd_4d_1x16x14_k64n32_g32"])
def test_module_golden_cases_through_kernel_level(dev, name):
    # The reference module would panic on group_size 32 (it fixes INNER_K = 64);
    # the same numbers through the kernel-level launcher with inner_k = 32.
    g = load_golden(name)
    x = g["x"]
    rows, k = x.shape
    out = run_kernel(dev, x, g["qweight"], g["qzeros"], g["scales"], rows, k, 32, 32)
    if "bias" in g:
        out = out + g["bias"][None, :]
    assert np.abs(out - g["expected"]).max() <= 1e-2
    assert oracle.rel_l2(out, g["expected"]) <= TOL_FP32


def test_module_forward_decode_golden(dev):
    # test_forward_decode_shape_matches_cpu_reference (src/modules/awq_gemm.rs:517-559).
    g = load_golden("gemm_decode_b2m1_k64n32_g64")
    layer = AWQGEMMLinear(_i32(g["qweight"], dev), _i32(g["qzeros"], dev),
                          torch.from_numpy(g["scales"]).to(dev))
    y = layer.forward(torch.from_numpy(g["x"]).reshape(2, 1, 64).to(dev))
    torch.cuda.synchronize()
    assert tuple(y.shape) == (2, 1, 32)
    out = y.reshape(2, 32).cpu().numpy()
    assert np.abs(out - g["expected"]).max() <= 1e-2
    assert oracle.rel_l2(out, g["expected"]) <= TOL_FP32


def _gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, x_dt, s_dt, y_dt="f32", b_dt="f32", y_init=None):
    # Keep every device tensor referenced until the launch is queued: a temporary
    # freed before the call could be recycled by the caching allocator.
    d_x = to_device(x, x_dt, dev)
    d_sc = to_device(sc, s_dt, dev)
    d_qw, d_qz = _i32(qw, dev), _i32(qz, dev)
    d_b = to_device(b, b_dt, dev) if b is not None else None
    y = torch.full((M, N), float("nan") if y_init is None else y_init, dtype=TORCH_OF[y_dt],
                   device=dev)
    _lib.check(cube_awq.lib().awq_gemm(
        d_x.data_ptr(), AWQ_DT[x_dt], d_qw.data_ptr(), d_qz.data_ptr(),
        d_sc.data_ptr(), AWQ_DT[s_dt], d_b.data_ptr() if d_b is not None else None, AWQ_DT[b_dt],
        y.data_ptr(), AWQ_DT[y_dt], M, K, N, g, None))
    torch.cuda.synchronize()
    return y


def _ref64(x, qw, qz, sc, b, g, x_dt, s_dt):
    return oracle.gemm_f64(host_f32(x, x_dt), qw, qz, host_f32(sc, s_dt), g, bias=b)


SHAPES_8B = [(4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096)]


@pytest.mark.parametrize("K,N", SHAPES_8B)
@pytest.mark.parametrize("M", [1, 4, 8])
def test_decode_sweep_fp32(dev, M, K, N):
    # Decode sweep: f32 activations ~N(0,1), f16 scales U[0.002, 0.02], g128.
    x, qw, qz, sc, _ = make_problem(M, K, N, 128, x_dt="f32", s_dt="f16")
    y = _gemm_ptr(dev, x, qw, qz, sc, None, M, K, N, 128, "f32", "f16")
    assert oracle.rel_l2(to_host(y), _ref64(x, qw, qz, sc, None, 128, "f32", "f16")) <= TOL_FP32


@pytest.mark.parametrize("M", [1, 2, 3, 5, 6, 7])
def test_decode_all_row_counts(dev, M):
    K, N, g = 1024, 2080, 64  # N not a multiple of 512: partial column chunk
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt="f32", s_dt="f32", bias=True)
    y = _gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, "f32", "f32")
    assert oracle.rel_l2(to_host(y), _ref64(x, qw, qz, sc, b, g, "f32", "f32")) <= TOL_FP32


def test_decode_config1_f32_scales(dev):
    # M=1, 4096 -> 4096, g128, f32 activations and f32 scales (the CPU-baseline case).
    x, qw, qz, sc, _ = make_problem(1, 4096, 4096, 128, x_dt="f32", s_dt="f32")
    y = _gemm_ptr(dev, x, qw, qz, sc, None, 1, 4096, 4096, 128, "f32", "f32")
    assert oracle.rel_l2(to_host(y), _ref64(x, qw, qz, sc, None, 128, "f32", "f32")) <= TOL_FP32


@pytest.mark.parametrize("x_dt,s_dt,y_dt", [("f16", "f16", "f16"), ("bf16", "bf16", "bf16"),
                                             ("f16", "f32", "f32"), ("bf16", "f16", "f32")])
def test_decode_low_precision_io(dev, x_dt, s_dt, y_dt):
    # Decode computes in fp32 whatever the I/O types; only the output cast rounds.
    M, K, N, g = 3, 4096, 1024, 128
    x, qw, qz, sc, _ = make_problem(M, K, N, g, x_dt=x_dt, s_dt=s_dt)
    y = _gemm_ptr(dev, x, qw, qz, sc, None, M, K, N, g, x_dt, s_dt, y_dt)
    tol = TOL_FP32 if y_dt == "f32" else (1e-3 if y_dt == "f16" else 5e-3)
    got = host_f32(to_host(y), y_dt)
    assert oracle.rel_l2(got, _ref64(x, qw, qz, sc, None, g, x_dt, s_dt)) <= tol


@pytest.mark.parametrize("K,N", [(4096, 4096), (4096, 14336), (14336, 4096)])
@pytest.mark.parametrize("M", [64, 512])
def test_prefill_sweep_f16(dev, M, K, N):
    x, qw, qz, sc, _ = make_problem(M, K, N, 128, x_dt="f16", s_dt="f16")
    y = _gemm_ptr(dev, x, qw, qz, sc, None, M, K, N, 128, "f16", "f16", "f16")
    got = host_f32(to_host(y), "f16")
    assert oracle.rel_l2(got, _ref64(x, qw, qz, sc, None, 128, "f16", "f16")) <= TOL_MFMA


@pytest.mark.parametrize("K,N", [(4096, 14336), (4096, 4096), (14336, 4096)])
def test_prefill_m2048_sampled_rows(dev, K, N):
    # Full-size prefill at M=2048 on the three Llama-3-8B shapes (256 x 224
    # ping-pong tiles for 4096 -> 14336, 128 x 256 tiles with K up to 14336
    # for the others): checked on 48 sampled rows.
    M, g = 2048, 128
    x, qw, qz, sc, _ = make_problem(M, K, N, g, x_dt="f16", s_dt="f16")
    y = _gemm_ptr(dev, x, qw, qz, sc, None, M, K, N, g, "f16", "f16", "f16")
    rows = np.r_[0:16, 1000:1016, 2032:2048]
    got = host_f32(to_host(y)[rows], "f16")
    assert oracle.rel_l2(got, _ref64(x[rows], qw, qz, sc, None, g, "f16", "f16")) <= TOL_MFMA


@pytest.mark.parametrize("M,K,N,x_dt", [(768, 4096, 14336, "f16"), (768, 28672, 8192, "f16"),
                                         (768, 4096, 14336, "bf16"), (300, 4096, 14336, "f16"),
                                         (1024, 28672, 8192, "f16")])
def test_prefill_mid_range_routes_sampled_rows(dev, M, K, N, x_dt):
    # 257..1024 rows with few 256-row tiles: the launcher's default choice
    # (256 x 224 tiles, with 2 K splits at 28672 -> 8192 and M = 768),
    # checked on 24 sampled rows including the last.
    g = 128
    x, qw, qz, sc, _ = make_problem(M, K, N, g, x_dt=x_dt, s_dt=x_dt)
    y = to_host(_gemm_ptr(dev, x, qw, qz, sc, None, M, K, N, g, x_dt, x_dt, "f32"))
    rows = np.r_[0:8, M // 2:M // 2 + 8, M - 8:M]
    assert oracle.rel_l2(y[rows], _ref64(x[rows], qw, qz, sc, None, g, x_dt, x_dt)) <= TOL_MFMA


# Llama-3-70B projections (8192 -> 8192, 8192 -> 1024, 8192 -> 28672,
# 28672 -> 8192), g128, fp16 activations N(0,1) and f16 scales, f16 output,
# from decode (M = 1, 8) to prefill (M = 128 .. 4096). Outputs are checked on
# all rows for M <= 8 and on 8 sampled rows otherwise (the f64 oracle costs
# K*N per row).
_SHAPES_70B = [(8192, 8192), (8192, 1024), (8192, 28672), (28672, 8192)]
_CASES_70B = [(K, N, M) for (K, N) in _SHAPES_70B for M in (1, 8, 128, 1024, 4096)]
_weights_70b = {}


def _weights_for(K, N, g):
    if (K, N) not in _weights_70b:
        _weights_70b.clear()  # one shape's weights held at a time
        _, qw, qz, sc, _ = make_problem(1, K, N, g, x_dt="f16", s_dt="f16")
        _weights_70b[(K, N)] = (qw, qz, sc)
    return _weights_70b[(K, N)]


@pytest.mark.parametrize("K,N,M", _CASES_70B)
def test_llama70b_projection_shapes(dev, K, N, M):
    g = 128
    qw, qz, sc = _weights_for(K, N, g)
    x = synth.normal(synth.TID_X, (M, K), np.float16)
    y = to_host(_gemm_ptr(dev, x, qw, qz, sc, None, M, K, N, g, "f16", "f16", "f16"))
    rows = np.arange(M) if M <= 8 else np.r_[0:3, M // 2:M // 2 + 2, M - 3:M]
    got = host_f32(y[rows], "f16")
    assert np.isfinite(got).all()
    ref = _ref64(x[rows], qw, qz, sc, None, g, "f16", "f16")
    # f16 output: one rounding of a value of relative size ~2^-11.
    assert oracle.rel_l2(got, ref) <= (1e-3 if M <= 8 else TOL_MFMA)


@pytest.mark.parametrize("M,K,N,g", [(9, 256, 96, 64), (100, 512, 224, 128), (130, 4096, 1024, 128),
                                     (37, 96, 64, 32), (64, 36, 32, 4)])
@pytest.mark.parametrize("x_dt", ["f16", "bf16", "f32"])
def test_prefill_odd_shapes(dev, M, K, N, g, x_dt):
    s_dt = "f32" if x_dt == "f32" else x_dt
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt=x_dt, s_dt=s_dt, bias=True)
    y = _gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, x_dt, s_dt, "f32") if K % 64 == 0 and g % 64 == 0 \
        else None
    if y is None:  # K or g below the module's INNER_K: kernel-level launcher, inner_k 4/32
        inner_k = 32 if (K % 32 == 0 and g % 32 == 0) else 4
        shape = ShapeConfig.new(M, N, K, 32, 32, inner_k)
        y = torch.full((M, N), float("nan"), device=dev)
        cube_awq.awq_gemm_linear(to_device(x, x_dt, dev), _i32(qw, dev), _i32(qz, dev),
                                 to_device(sc, s_dt, dev), y, shape, g)
        torch.cuda.synchronize()
        ref = _ref64(x, qw, qz, sc, None, g, x_dt, s_dt)
    else:
        ref = _ref64(x, qw, qz, sc, b, g, x_dt, s_dt)
    tol = TOL_FP32 if x_dt == "f32" else TOL_MFMA
    assert oracle.rel_l2(to_host(y), ref) <= tol


def test_m_valid_rows_untouched(dev):
    # Rows >= m_valid are neither computed nor written (src/kernel/awq_kernel_gemm.rs:225-226).
    for M, mv in ((40, 17), (6, 2)):
        K, N, g = 256, 64, 64
        x, qw, qz, sc, _ = make_problem(M, K, N, g, x_dt="f32", s_dt="f32")
        y = torch.full((M, N), 123.0, device=dev)
        shape = ShapeConfig.new_with_valid_m(M, N, K, 32, 64, 64, mv)
        cube_awq.awq_gemm_linear(torch.from_numpy(x).to(dev), _i32(qw, dev), _i32(qz, dev),
                                 torch.from_numpy(sc).to(dev), y, shape, g)
        torch.cuda.synchronize()
        out = y.cpu().numpy()
        assert np.all(out[mv:] == 123.0)
        assert oracle.rel_l2(out[:mv], _ref64(x[:mv], qw, qz, sc, None, g, "f32", "f32")) <= TOL_FP32


def test_m_valid_batched_rule(dev):
    # shape.m = 2, input flattened to 6 rows, m_valid == m -> all 6 rows valid (:675-690).
    K, N, g = 128, 32, 64
    x, qw, qz, sc, _ = make_problem(6, K, N, g, x_dt="f32", s_dt="f32")
    y = torch.full((3, 2, N), 7.0, device=dev)
    shape = ShapeConfig.new(2, N, K, 8, 32, 64)
    cube_awq.awq_gemm_linear(torch.from_numpy(x).reshape(3, 2, K).to(dev), _i32(qw, dev),
                             _i32(qz, dev), torch.from_numpy(sc).to(dev), y, shape, g)
    torch.cuda.synchronize()
    out = y.reshape(6, N).cpu().numpy()
    assert oracle.rel_l2(out, _ref64(x, qw, qz, sc, None, g, "f32", "f32")) <= TOL_FP32


@pytest.mark.parametrize("M", [1, 8, 256])
def test_repeated_calls_bit_identical(dev, M):
    # Deterministic reductions (no atomics in the sums), split-K counters reset.
    K, N, g = 4096, 4096, 128
    x, qw, qz, sc, _ = make_problem(M, K, N, g, x_dt="f16" if M > 8 else "f32", s_dt="f16")
    x_dt = "f16" if M > 8 else "f32"
    a = to_host(_gemm_ptr(dev, x, qw, qz, sc, None, M, K, N, g, x_dt, "f16"))
    for _ in range(3):
        b = to_host(_gemm_ptr(dev, x, qw, qz, sc, None, M, K, N, g, x_dt, "f16"))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("tile", [1, 2, 3, 4, 6, 7, 8, 9, 10, 11, 12])
@pytest.mark.parametrize("splits", [1, 3, 8])
@pytest.mark.parametrize("x_dt", ["f16", "bf16"])
def test_prefill_every_tile_configuration(dev, monkeypatch, tile, splits, x_dt):
    """Every prefill kernel configuration (tile shape, MFMA shape, split-K),
    forced through the tuning overrides, on a shape ragged in M and N for all
    of them, with bias."""
    monkeypatch.setenv("AWQ_GEMM_TILE", str(tile))
    monkeypatch.setenv("AWQ_GEMM_SPLITS", str(splits))
    M, K, N, g = 300, 512, 672, 128
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt=x_dt, s_dt="f16", bias=True)
    y = _gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, x_dt, "f16", "f32")
    got = to_host(y)
    assert np.isfinite(got).all()
    assert oracle.rel_l2(got, _ref64(x, qw, qz, sc, b, g, x_dt, "f16")) <= TOL_MFMA


@pytest.mark.parametrize("tiles", [(9, 10), (12, 11)])
@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("x_dt,s_dt", [("f16", "f16"), ("bf16", "bf16"), ("f16", "f32")])
def test_prefill_ping_pong_matches_single_phase_bits(dev, monkeypatch, tiles, splits, x_dt, s_dt):
    """The 256 x 224 and 128 x 256 tiles with the two halves of their waves a
    phase apart (tiles 10, 11) perform each accumulator's MFMAs in the same
    order as the single-phase schedule (tiles 9, 12), so the outputs are
    bit-identical; checked on a shape ragged in M and N, 12 stages, with and
    without K splits."""
    monkeypatch.setenv("AWQ_GEMM_SPLITS", str(splits))
    M, K, N, g = 520, 768, 1120, 64
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt=x_dt, s_dt=s_dt, bias=True)
    outs = []
    for tile in tiles:
        monkeypatch.setenv("AWQ_GEMM_TILE", str(tile))
        outs.append(to_host(_gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, x_dt, s_dt, "f32")))
    assert np.isfinite(outs[1]).all()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert oracle.rel_l2(outs[1], _ref64(x, qw, qz, sc, b, g, x_dt, s_dt)) <= TOL_MFMA


@pytest.mark.parametrize("group_m", [1, 2, 3, 5])
def test_prefill_tile_raster_groups(dev, monkeypatch, group_m):
    """The grouped tile order of the large-tile kernel covers every output
    tile once, including a last group with fewer row tiles than the others
    (7 row tiles of 128) and tiles past the XCD-mapped multiple of 8."""
    monkeypatch.setenv("AWQ_GEMM_TILE", "4")
    monkeypatch.setenv("AWQ_GEMM_GROUP_M", str(group_m))
    M, K, N, g = 800, 256, 1152, 64
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt="f16", s_dt="f16", bias=True)
    y = _gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, "f16", "f16", "f32")
    got = to_host(y)
    assert np.isfinite(got).all()
    assert oracle.rel_l2(got, _ref64(x, qw, qz, sc, b, g, "f16", "f16")) <= TOL_MFMA


# Decode rows 2..8 run on the matrix cores by default (2..4 rows on 4x4x4
# blocks, 5..8 on the 16-row tile); AWQ_DECODE_M4=0 sends 2..4 rows to the
# 16-row tile and AWQ_DECODE_MFMA=0 selects the VALU kernel. All three are
# checked, and every launch configuration below.
DECODE_KERNELS = {"m4": {"AWQ_DECODE_MFMA": "1", "AWQ_DECODE_M4": "1"},
                  "mfma16": {"AWQ_DECODE_MFMA": "1", "AWQ_DECODE_M4": "0"},
                  "valu": {"AWQ_DECODE_MFMA": "0"}}


@pytest.mark.parametrize("kernel", ["m4", "mfma16", "valu"])
@pytest.mark.parametrize("M", [2, 3, 4, 7, 8])
@pytest.mark.parametrize("x_dt", ["f32", "f16", "bf16"])
def test_decode_rows_both_kernels(dev, monkeypatch, kernel, M, x_dt):
    for k, v in DECODE_KERNELS[kernel].items():
        monkeypatch.setenv(k, v)
    K, N, g = 2048, 2080, 128  # N not a multiple of 512: partial column chunk
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt=x_dt, s_dt="f16", bias=True)
    y = _gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, x_dt, "f16", "f32")
    ref = _ref64(x, qw, qz, sc, b, g, x_dt, "f16")
    assert oracle.rel_l2(to_host(y), ref) <= TOL_FP32


@pytest.mark.parametrize("kernel,M,x_dt,y_dt,K", [
    ("valu", 1, "f32", "f32", 9216),   # 8 waves x 32 rows: 36 splits, 4 thread groups
    ("valu", 1, "f16", "f16", 14336),  # 16 waves x 32 rows: 28 splits, 8 thread groups
    ("valu", 1, "bf16", "bf16", 9216),
    ("valu", 2, "f32", "f32", 4096),   # 16 waves x 8 rows: 32 splits
    ("m4", 3, "f16", "f32", 8192),     # 16 waves x 32 rows: 16 splits, 2 thread groups
    ("m4", 4, "f16", "f16", 4608),     # 9 splits
])
def test_decode_deep_k_split_sum(dev, monkeypatch, kernel, M, x_dt, y_dt, K):
    """More than 8 K splits: the last workgroup's sum over the splits is
    shared by thread groups (contiguous split ranges, then the groups in a
    fixed order). Partial column chunk, bias, each output type; two calls
    give the same bits."""
    for k, v in DECODE_KERNELS[kernel].items():
        monkeypatch.setenv(k, v)
    N, g = 2080, 128
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt=x_dt, s_dt="f16", bias=True)
    y1 = _gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, x_dt, "f16", y_dt)
    y2 = _gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, x_dt, "f16", y_dt)
    assert torch.equal(y1, y2)
    got = host_f32(to_host(y1), y_dt)
    assert np.isfinite(got).all()
    tol = TOL_FP32 if y_dt == "f32" else (1e-3 if y_dt == "f16" else 5e-3)
    assert oracle.rel_l2(got, _ref64(x, qw, qz, sc, b, g, x_dt, "f16")) <= tol


@pytest.mark.parametrize("kernel,M,x_dt,K,g", [
    ("m4", 2, "f32", 8192, 128),      # 8 waves x 32 rows: 32 splits, groups of 6 (the last of 2)
    ("m4", 4, "f16", 14336, 128),     # 56 splits, groups of 8
    ("m4", 3, "bf16", 4160, 64),      # 17 splits, the last wave of the last past K
    ("mfma16", 3, "f32", 9216, 128),  # 4-row tile: 36 splits, groups of 6
    ("mfma16", 8, "f16", 14336, 128), # 8 x 32 rows: 56 splits, groups of 8
    ("mfma16", 6, "bf16", 6144, 64),  # 24 splits, groups of 5 (the last of 4)
])
@pytest.mark.parametrize("tree", ["0", "1"])
def test_decode_split_sum_levels(dev, monkeypatch, kernel, M, x_dt, K, g, tree):
    """The matrix-core decode kernels' split-K sum in one level (the last
    workgroup sums every split) and in two (groups of splits, then the
    groups), each against the oracle, with bias and a partial column chunk;
    two calls give the same bits."""
    for k, v in DECODE_KERNELS[kernel].items():
        monkeypatch.setenv(k, v)
    monkeypatch.setenv("AWQ_DECODE_TREE", tree)
    N = 2080
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt=x_dt, s_dt="f16", bias=True)
    y1 = _gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, x_dt, "f16", "f32")
    y2 = _gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, x_dt, "f16", "f32")
    assert torch.equal(y1, y2)
    got = to_host(y1)
    assert np.isfinite(got).all()
    assert oracle.rel_l2(got, _ref64(x, qw, qz, sc, b, g, x_dt, "f16")) <= TOL_FP32


@pytest.mark.parametrize("M,x_dt", [(12, "f32"), (16, "f32")])
def test_small_m_split_sum_two_levels(dev, monkeypatch, M, x_dt):
    """9..16 rows on the 16-row decode tile with the two-level split sum."""
    monkeypatch.setenv("AWQ_DECODE_TREE", "1")
    K, N, g = 8192, 1056, 128
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt=x_dt, s_dt="f16", bias=True)
    y = to_host(_gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, x_dt, "f16", "f32"))
    assert np.isfinite(y).all()
    assert oracle.rel_l2(y, _ref64(x, qw, qz, sc, b, g, x_dt, "f16")) <= TOL_FP32


@pytest.mark.parametrize("waves,rpw", [(8, 64), (8, 32), (4, 64), (4, 32)])
@pytest.mark.parametrize("s_dt", ["f32", "f16", "bf16"])
def test_decode_mfma_every_configuration(dev, monkeypatch, waves, rpw, s_dt):
    # 5 rows: the 16-row matrix-core tile (2..4 rows take the 4x4x4 blocks)
    monkeypatch.setenv("AWQ_MFMA_WAVES", str(waves))
    monkeypatch.setenv("AWQ_MFMA_RPW", str(rpw))
    M, K, N, g = 5, 4096, 1536, 64
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt="f32", s_dt=s_dt, bias=True)
    y = _gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, "f32", s_dt, "f32")
    ref = _ref64(x, qw, qz, sc, b, g, "f32", s_dt)
    assert oracle.rel_l2(to_host(y), ref) <= TOL_FP32


@pytest.mark.parametrize("waves,rpw", [(16, 32), (8, 64), (8, 32)])
@pytest.mark.parametrize("x_dt,s_dt", [("f32", "f16"), ("f16", "f16"), ("bf16", "bf16"), ("f32", "f32")])
@pytest.mark.parametrize("M", [2, 3, 4])
def test_decode_m4_every_configuration(dev, monkeypatch, waves, rpw, x_dt, s_dt, M):
    """The 4x4x4 decode kernel in each launch configuration (16 waves only
    with f16 activations; others fall back to 8), with bias, K splits and a
    partial column chunk."""
    monkeypatch.setenv("AWQ_DECODE_MFMA", "1")
    monkeypatch.setenv("AWQ_M4_WAVES", str(waves))
    monkeypatch.setenv("AWQ_M4_RPW", str(rpw))
    K, N, g = 4096, 1536, 64
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt=x_dt, s_dt=s_dt, bias=True)
    y = _gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, x_dt, s_dt, "f32")
    ref = _ref64(x, qw, qz, sc, b, g, x_dt, s_dt)
    assert oracle.rel_l2(to_host(y), ref) <= TOL_FP32


@pytest.mark.parametrize("K,N,g", [(64, 32, 64), (192, 64, 64), (4160, 544, 64), (320, 4096, 64),
                                   (30720, 544, 128), (128, 28672, 128)])
@pytest.mark.parametrize("x_dt", ["f32", "f16", "bf16"])
def test_decode_one_row_edge_shapes(dev, K, N, g, x_dt):
    """One row through the launch-shape rule at its edges: one 32-column
    chunk (most lanes clamped), waves whose rows start past K, the shortest
    runs (16 waves x 8 rows), deep K over few chunks (16 waves x 16 rows,
    120 splits: the grouped sum) and one split over many chunks."""
    x, qw, qz, sc, b = make_problem(1, K, N, g, x_dt=x_dt, s_dt="f16", bias=True)
    y = to_host(_gemm_ptr(dev, x, qw, qz, sc, b, 1, K, N, g, x_dt, "f16", "f32"))
    assert np.isfinite(y).all()
    assert oracle.rel_l2(y, _ref64(x, qw, qz, sc, b, g, x_dt, "f16")) <= TOL_FP32


@pytest.mark.parametrize("K,N,g", [(64, 32, 64), (192, 64, 64), (4160, 544, 64), (320, 4096, 64)])
@pytest.mark.parametrize("x_dt", ["f32", "f16"])
@pytest.mark.parametrize("M", [2, 3, 4])
def test_decode_m4_edge_shapes(dev, monkeypatch, K, N, g, x_dt, M):
    """4x4x4 decode edge cases: one pack chunk with most lanes clamped
    (N = 32), waves whose rows start past K (K not a multiple of a
    workgroup's rows), one K split or many (g = 64: the reference's module
    rule, group >= 64)."""
    monkeypatch.setenv("AWQ_DECODE_MFMA", "1")
    monkeypatch.setenv("AWQ_DECODE_M4", "1")
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt=x_dt, s_dt="f16", bias=True)
    y = to_host(_gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, x_dt, "f16", "f32"))
    assert np.isfinite(y).all()
    assert oracle.rel_l2(y, _ref64(x, qw, qz, sc, b, g, x_dt, "f16")) <= TOL_FP32


@pytest.mark.parametrize("row_scales", [(1e6, 1e-6, 1.0, 3e4), (1e30, 1e-30, 7e4, 1e-20), (65504.0, 1e5, 2e-8, 1.0)])
@pytest.mark.parametrize("kernel", ["m4", "mfma16", "valu", "valu_m1"])
def test_decode_mfma_activation_magnitudes(dev, monkeypatch, row_scales, kernel):
    """fp32 activations far outside the f16 range, and far below it, in
    different rows of one call (valu_m1: one M = 1 call per row, the
    headline decode kernel): each output row keeps fp32 accuracy."""
    for k, v in DECODE_KERNELS.get(kernel, {}).items():
        monkeypatch.setenv(k, v)
    M, K, N, g = 4, 1024, 1024, 128
    x, qw, qz, sc, _ = make_problem(M, K, N, g, x_dt="f32", s_dt="f16")
    x = (x * np.asarray(row_scales, dtype=np.float64)[:, None]).astype(np.float32)
    if kernel == "valu_m1":
        y = np.concatenate([to_host(_gemm_ptr(dev, x[m:m + 1], qw, qz, sc, None, 1, K, N, g, "f32", "f16",
                                              "f32")) for m in range(M)])
    else:
        y = to_host(_gemm_ptr(dev, x, qw, qz, sc, None, M, K, N, g, "f32", "f16", "f32"))
    ref = _ref64(x, qw, qz, sc, None, g, "f32", "f16")
    for m in range(M):
        assert np.isfinite(y[m]).all()
        assert oracle.rel_l2(y[m], ref[m]) <= TOL_FP32, (m, row_scales[m])


# 9..16 rows: f16/bf16 activations on the skinny kernel by default, fp32 on
# the matrix-core decode kernel's 16-row tile (two-round LDS reduction, exact
# q - z operands: fp32-level accuracy for every activation type);
# AWQ_SKINNY=0 puts f16/bf16 on that tile too, and with AWQ_SMALLM_MFMA=0 as
# well they go to the large-tile prefill kernels. All three are checked.
SMALL_M_PATHS = {"default": {}, "tile16": {"AWQ_SKINNY": "0"},
                 "tiles": {"AWQ_SMALLM_MFMA": "0", "AWQ_SKINNY": "0"}}


@pytest.mark.parametrize("path", ["default", "tile16", "tiles"])
@pytest.mark.parametrize("M", [9, 12, 16])
@pytest.mark.parametrize("x_dt", ["f32", "f16", "bf16"])
def test_small_m_both_paths(dev, monkeypatch, path, M, x_dt):
    for k, v in SMALL_M_PATHS[path].items():
        monkeypatch.setenv(k, v)
    K, N, g = 2048, 2080, 64
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt=x_dt, s_dt="f16", bias=True)
    y = _gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, x_dt, "f16", "f32")
    ref = _ref64(x, qw, qz, sc, b, g, x_dt, "f16")
    tol = TOL_FP32 if (path == "tile16" or x_dt == "f32") else TOL_MFMA
    assert oracle.rel_l2(to_host(y), ref) <= tol


# fp32 activations past 16 rows: by default the f16 matrix cores with x split
# into hi + lo (test_f32_prefill_gpu.py covers that route in depth);
# AWQ_F32_SLICES=2 runs 16-row slices of the decode kernels' 16-row tile, and
# AWQ_GEMM_TILE=1 with AWQ_F32_SLICES=0 the generic fp32-MFMA kernel. All
# three, with a ragged last slice (1..15 rows, so also the smaller decode
# kernels), bias and every output dtype.
F32_PATHS = {"default": {}, "slices": {"AWQ_F32_SLICES": "2"},
             "generic": {"AWQ_F32_SLICES": "0", "AWQ_GEMM_TILE": "1"}}


@pytest.mark.parametrize("path", list(F32_PATHS))
@pytest.mark.parametrize("M,y_dt", [(17, "f32"), (33, "f16"), (100, "bf16"), (256, "f32"), (300, "f32")])
def test_f32_rows_slices_and_prefill_kernel(dev, monkeypatch, path, M, y_dt):
    for k, v in F32_PATHS[path].items():
        monkeypatch.setenv(k, v)
    K, N, g = 1024, 1056, 64
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt="f32", s_dt="f16", bias=True)
    y = to_host(_gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, "f32", "f16", y_dt))
    ref = _ref64(x, qw, qz, sc, b, g, "f32", "f16")
    # f16 / bf16 outputs: one rounding of relative size 2^-11 / 2^-8.
    tol = {"f32": TOL_FP32, "f16": 1e-3, "bf16": 4e-3}[y_dt]
    assert oracle.rel_l2(host_f32(y, y_dt), ref) <= tol


@pytest.mark.parametrize("rpw", [32, 64])
def test_small_m_every_configuration(dev, monkeypatch, rpw):
    monkeypatch.setenv("AWQ_MFMA_RPW", str(rpw))
    M, K, N, g = 16, 4096, 1536, 128
    x, qw, qz, sc, _ = make_problem(M, K, N, g, x_dt="f32", s_dt="f32")
    y = _gemm_ptr(dev, x, qw, qz, sc, None, M, K, N, g, "f32", "f32", "f32")
    assert oracle.rel_l2(to_host(y), _ref64(x, qw, qz, sc, None, g, "f32", "f32")) <= TOL_FP32


# 9..128 rows of f16 or bf16 activations (16-bit scales) run on the skinny
# kernel (awq_skinny.hip), in 64-column chunks (4 waves) or 256-column chunks
# (8 waves); AWQ_SKINNY=0 sends them to the large-tile kernels (17..128 rows)
# or the 16-row decode tile (9..16).
SKINNY_PATHS = {"c64": {"AWQ_SKINNY": "1", "AWQ_SKINNY_COLS": "64"},
                "c256": {"AWQ_SKINNY": "1", "AWQ_SKINNY_COLS": "256"}, "off": {"AWQ_SKINNY": "0"}}
SKINNY_COLS = {"64": SKINNY_PATHS["c64"], "256": SKINNY_PATHS["c256"]}


def _skinny_cols(monkeypatch, cols):
    for k, v in SKINNY_COLS[cols].items():
        monkeypatch.setenv(k, v)


@pytest.mark.parametrize("path", list(SKINNY_PATHS))
@pytest.mark.parametrize("M", [9, 16, 17, 33, 48, 64, 80, 96, 100, 128])
@pytest.mark.parametrize("x_dt", ["f16", "bf16"])
def test_skinny_both_paths(dev, monkeypatch, path, M, x_dt):
    for k, v in SKINNY_PATHS[path].items():
        monkeypatch.setenv(k, v)
    K, N, g = 2048, 2080, 128  # N % 256 != 0: ragged last chunk
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt=x_dt, s_dt=x_dt, bias=True)
    y = _gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, x_dt, x_dt, "f32")
    assert oracle.rel_l2(to_host(y), _ref64(x, qw, qz, sc, b, g, x_dt, x_dt)) <= TOL_MFMA


@pytest.mark.parametrize("cols", list(SKINNY_COLS))
@pytest.mark.parametrize("splits", [1, 3, 8, 64])
@pytest.mark.parametrize("x_dt,s_dt,g", [("f16", "f16", 64), ("f16", "f32", 128), ("f16", "bf16", 256),
                                         ("bf16", "bf16", 64), ("bf16", "f16", 128)])
def test_skinny_every_split(dev, monkeypatch, cols, splits, x_dt, s_dt, g):
    _skinny_cols(monkeypatch, cols)
    monkeypatch.setenv("AWQ_SKINNY_SPLITS", str(splits))
    M, K, N = 48, 4096, 768
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt=x_dt, s_dt=s_dt, bias=True)
    # bf16 output would add a rounding of relative size ~2^-9 to the bf16
    # weights' own; f16 output is also covered here.
    y_dt = "f16" if x_dt == "f16" else "f32"
    y = to_host(_gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, x_dt, s_dt, y_dt))
    assert oracle.rel_l2(host_f32(y, y_dt), _ref64(x, qw, qz, sc, b, g, x_dt, s_dt)) <= TOL_MFMA


@pytest.mark.parametrize("cols", list(SKINNY_COLS))
@pytest.mark.parametrize("splits", [3, 7, 16, 64])
@pytest.mark.parametrize("M,x_dt", [(17, "f16"), (100, "bf16"), (9, "f16")])
def test_skinny_split_sum_two_levels(dev, monkeypatch, cols, splits, M, x_dt):
    """The skinny kernel's two-level split-K sum (groups of splits, then the
    groups), forced: against the oracle with bias and a ragged last chunk;
    two calls give the same bits."""
    _skinny_cols(monkeypatch, cols)
    monkeypatch.setenv("AWQ_SKINNY", "1")
    monkeypatch.setenv("AWQ_SKINNY_SPLITS", str(splits))
    monkeypatch.setenv("AWQ_SKINNY_TREE", "1")
    K, N, g = 4096, 2080, 64
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt=x_dt, s_dt=x_dt, bias=True)
    y1 = _gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, x_dt, x_dt, "f32")
    y2 = _gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, x_dt, x_dt, "f32")
    assert torch.equal(y1, y2)
    assert oracle.rel_l2(to_host(y1), _ref64(x, qw, qz, sc, b, g, x_dt, x_dt)) <= TOL_MFMA


@pytest.mark.parametrize("cols", list(SKINNY_COLS))
@pytest.mark.parametrize("M", [12, 48, 128])
@pytest.mark.parametrize("splits", ["1", "3"])
@pytest.mark.parametrize("x_dt,s_dt", [("f16", "f16"), ("bf16", "bf16"), ("bf16", "f16"), ("f16", "bf16")])
def test_skinny_weights_exact(dev, monkeypatch, cols, M, splits, x_dt, s_dt):
    """Each row of X selects one k (a single 1), so row m of Y is row k_m of
    the weights as the kernel dequantised them, with nothing else added:
    bit-exact against (q - z) * s rounded once to the activation type (the
    reference's F-typed dequant, src/kernel/awq_kernel_gemm.rs:181-439)."""
    _skinny_cols(monkeypatch, cols)
    monkeypatch.setenv("AWQ_SKINNY_SPLITS", splits)
    K, N, g = 2048, 768, 128
    _, qw, qz, sc, _ = make_problem(M, K, N, g, x_dt=x_dt, s_dt=s_dt)
    ks = (np.arange(M) * 37 + 5) % K  # distinct rows, in every split's range
    x32 = np.zeros((M, K), dtype=np.float32)
    x32[np.arange(M), ks] = 1.0
    x = round_to(x32, x_dt)
    y = to_host(_gemm_ptr(dev, x, qw, qz, sc, None, M, K, N, g, x_dt, s_dt, "f32"))
    w32 = oracle.dequant(qw, qz, host_f32(sc, s_dt), g, order="awq")  # exact for 16-bit scales
    want = host_f32(round_to(w32[ks], x_dt), x_dt)
    assert np.array_equal(y, want)


@pytest.mark.parametrize("M,K,N", [(64, 4096, 4096), (17, 4096, 14336), (100, 2048, 2048), (40, 14336, 4096)])
@pytest.mark.parametrize("splits", ["0", "1", "3"])
def test_skinny_narrow_chunks_xcd_mapped(dev, monkeypatch, M, K, N, splits):
    # 64-column chunks on outputs whose chunk count lets each XCD run a
    # contiguous run of them (N % 2048 == 0), with and without K splits.
    monkeypatch.setenv("AWQ_SKINNY", "1")
    monkeypatch.setenv("AWQ_SKINNY_COLS", "64")
    if splits != "0":
        monkeypatch.setenv("AWQ_SKINNY_SPLITS", splits)
    g = 128
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt="f16", s_dt="f16", bias=True)
    y = _gemm_ptr(dev, x, qw, qz, sc, b, M, K, N, g, "f16", "f16", "f32")
    assert oracle.rel_l2(to_host(y), _ref64(x, qw, qz, sc, b, g, "f16", "f16")) <= TOL_MFMA
