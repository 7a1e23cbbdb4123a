"""Gate/up projections with SiLU in the GEMM epilogue (awq_gemm_silu_mul,
AWQGateUpSiLU) on the GPU.

The weights interleave the two projections by column (2j = gate j, 2j + 1 =
up j), so each kernel's epilogue has both values of an output. Checked on
every kernel route (decode VALU and matrix-core, skinny direct and split-K,
large-tile direct and split-K, generic tiles) two ways:
  * against the oracle: the f64 GEMM of the interleaved weights, then
    SiLU(g) * u in f64 (tolerances of the GEMM paths, doubled: the product
    carries the relative errors of both factors);
  * against awq_gemm on the same weights with SiLU(g) * u applied on the host
    to its fp32 output: the GEMM sums are the same bits, so only the
    epilogue's exp and division differ (2e-6)."""
import numpy as np
import pytest
import torch

import awq_oracle as oracle
import cube_awq
from cube_awq import AWQGateUpSiLU, AWQGEMMLinear, _lib, pack
from helpers import TORCH_OF, host_f32, make_problem, to_device, to_host

pytestmark = pytest.mark.gpu

AWQ_DT = {"f32": _lib.AWQ_F32, "f16": _lib.AWQ_F16, "bf16": _lib.AWQ_BF16}


def _i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(dev)


def silu_mul64(h):
    h = np.asarray(h, dtype=np.float64)
    g, u = h[:, 0::2], h[:, 1::2]
    return g / (1.0 + np.exp(-g)) * u


def _launch(fn, dev, x, qw, qz, sc, b, M, K, N, g, x_dt, s_dt, width):
    d_x, d_sc = to_device(x, x_dt, dev), to_device(sc, s_dt, dev)
    d_qw, d_qz = _i32(qw, dev), _i32(qz, dev)
    d_b = to_device(b, "f32", dev) if b is not None else None
    y = torch.full((M, width), float("nan"), dtype=torch.float32, device=dev)
    _lib.check(fn(d_x.data_ptr(), AWQ_DT[x_dt], d_qw.data_ptr(), d_qz.data_ptr(), d_sc.data_ptr(),
                  AWQ_DT[s_dt], d_b.data_ptr() if d_b is not None else None, _lib.AWQ_F32,
                  y.data_ptr(), _lib.AWQ_F32, M, K, N, g, None))
    torch.cuda.synchronize()
    return to_host(y)


# (M, x dtype, environment): one case per kernel route.
ROUTES = [
    (1, "f32", {}),                                   # decode GEMV (VALU)
    (3, "f32", {}),
    (8, "f32", {}),
    (4, "f16", {}),                                   # decode on 4x4x4 matrix-core blocks
    (3, "bf16", {"AWQ_DECODE_M4": "0"}),              # decode on the 16-row matrix-core tile
    (8, "bf16", {}),
    (12, "f32", {}),                                  # 9..16 rows, matrix cores
    (16, "f16", {}),                                  # 9..16 rows of f16: skinny
    (16, "f16", {"AWQ_SKINNY": "0"}),                 # 9..16 rows on the 16-row tile
    (17, "f16", {}),                                  # skinny, split-K
    (64, "f16", {"AWQ_SKINNY_SPLITS": "1"}),          # skinny, direct store
    (100, "f16", {}),
    (24, "bf16", {}),                                 # skinny bf16, split-K
    (96, "bf16", {"AWQ_SKINNY": "1", "AWQ_SKINNY_SPLITS": "1"}),  # skinny bf16, direct store
    (64, "f16", {"AWQ_SKINNY": "0"}),                 # large tiles, split-K
    (300, "f16", {}),                                 # large tiles, direct store
    (300, "bf16", {}),
    (300, "f16", {"AWQ_GEMM_TILE": "1"}),             # generic tiles
    (300, "f16", {"AWQ_GEMM_TILE": "10"}),            # 256 x 224 tiles, ping-pong halves
    (40, "f32", {}),                                  # fp32 prefill: x split hi + lo, matrix cores
    (200, "f32", {"AWQ_GEMM_TILE": "4"}),             # the same on 128 x 128 tiles
    (20, "f32", {}),                                  # fp32, 16-row slices
    (64, "f16", {"AWQ_SKINNY_COLS": "256", "AWQ_SKINNY_SPLITS": "1"}),  # 256-column skinny, direct store
    (64, "f16", {"AWQ_SKINNY_COLS": "256"}),          # 256-column skinny, split-K
    (48, "bf16", {"AWQ_SKINNY_COLS": "256", "AWQ_SKINNY_SPLITS": "1"}),  # 256-column bf16, direct store
    (96, "bf16", {"AWQ_SKINNY": "1", "AWQ_SKINNY_COLS": "256", "AWQ_SKINNY_SPLITS": "1"}),
]


@pytest.mark.parametrize("M,x_dt,env", ROUTES)
def test_silu_mul_every_route(dev, monkeypatch, M, x_dt, env):
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    K, N, g = 1024, 1024, 128
    s_dt = "f16" if x_dt == "f32" else x_dt
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt=x_dt, s_dt=s_dt, bias=True)
    L = cube_awq.lib()
    y = _launch(L.awq_gemm_silu_mul, dev, x, qw, qz, sc, b, M, K, N, g, x_dt, s_dt, N // 2)
    assert np.isfinite(y).all()
    h = oracle.gemm_f64(host_f32(x, x_dt), qw, qz, host_f32(sc, s_dt), g, bias=b)
    tol = 2e-5 if (x_dt == "f32" or M <= 8) else 4e-3
    assert oracle.rel_l2(y, silu_mul64(h)) <= tol
    full = _launch(L.awq_gemm, dev, x, qw, qz, sc, b, M, K, N, g, x_dt, s_dt, N)
    assert oracle.rel_l2(y, silu_mul64(full)) <= 2e-6


@pytest.mark.parametrize("M,x_dt,K,env", [
    (1, "f32", 9216, {}),                        # decode VALU, 36 K splits
    (1, "f16", 14336, {}),                       # 28 K splits
    (2, "f32", 4096, {"AWQ_DECODE_MFMA": "0"}),  # 2 rows, 32 K splits
    (3, "f16", 8192, {}),                        # 4x4x4 blocks, 16 waves, 16 K splits
    (4, "f32", 14336, {"AWQ_DECODE_TREE": "1"}),   # 4x4x4 blocks, two-level split sum
    (8, "f16", 14336, {"AWQ_DECODE_TREE": "1"}),   # 16-row tile, two-level split sum
    (64, "f16", 14336, {"AWQ_SKINNY_TREE": "1", "AWQ_SKINNY_SPLITS": "16"}),  # skinny, two levels
])
def test_silu_mul_decode_deep_k(dev, monkeypatch, M, x_dt, K, env):
    """SiLU epilogue after a split-K sum over more than 8 splits (shared by
    thread groups, or in two levels), with a partial column chunk and bias."""
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    N, g = 2112, 128  # a multiple of 64 (the gate/up rule), not of 512
    s_dt = "f16"
    x, qw, qz, sc, b = make_problem(M, K, N, g, x_dt=x_dt, s_dt=s_dt, bias=True)
    L = cube_awq.lib()
    y = _launch(L.awq_gemm_silu_mul, dev, x, qw, qz, sc, b, M, K, N, g, x_dt, s_dt, N // 2)
    assert np.isfinite(y).all()
    h = oracle.gemm_f64(host_f32(x, x_dt), qw, qz, host_f32(sc, s_dt), g, bias=b)
    tol = 2e-5 if (x_dt == "f32" or M <= 8) else 4e-3  # the skinny route builds f16 weights
    assert oracle.rel_l2(y, silu_mul64(h)) <= tol
    full = _launch(L.awq_gemm, dev, x, qw, qz, sc, b, M, K, N, g, x_dt, s_dt, N)
    assert oracle.rel_l2(y, silu_mul64(full)) <= 2e-6


@pytest.mark.parametrize("M", [1, 5, 40, 200])
def test_gate_up_module_matches_separate_layers(dev, M):
    """AWQGateUpSiLU.from_gate_up(gate, up)(x) == SiLU(gate(x)) * up(x)."""
    K, I, g = 2048, 1536, 128
    x, qw, qz, sc, b = make_problem(M, K, 2 * I, g, x_dt="f16", s_dt="f16", bias=True)
    half = I // 8
    gate = AWQGEMMLinear(_i32(qw[:, :half], dev), _i32(qz[:, :half], dev),
                         torch.from_numpy(np.ascontiguousarray(sc[:, :I])).to(dev),
                         torch.from_numpy(b[:I]).to(dev).half())
    up = AWQGEMMLinear(_i32(qw[:, half:], dev), _i32(qz[:, half:], dev),
                       torch.from_numpy(np.ascontiguousarray(sc[:, I:])).to(dev), None)
    layer = AWQGateUpSiLU.from_gate_up(gate, up)
    xd = to_device(x, "f16", dev)
    y = layer(xd)
    assert y.dtype == torch.float16 and tuple(y.shape) == (M, I)
    gy, uy = gate(xd).double(), up(xd).double()
    ref = (gy / (1 + torch.exp(-gy)) * uy).cpu().numpy()
    assert oracle.rel_l2(y.double().cpu().numpy(), ref) <= 2e-3  # two f16 output roundings apart


def test_interleave_on_device_matches_host(dev):
    rng = np.random.default_rng(7)
    a = pack.pack(rng.integers(0, 16, (64, 256)), "awq")
    b = pack.pack(rng.integers(0, 16, (64, 256)), "awq")
    on_dev = pack.interleave_packed(_i32(a, dev), _i32(b, dev))
    assert np.array_equal(on_dev.cpu().numpy().view(np.uint32), pack.interleave_packed(a, b))
