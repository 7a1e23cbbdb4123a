"""Pins the CPU oracle (oracle/awq_oracle.c) before anything is checked against it.

Each oracle function is checked against something it does not compute itself:
the reference tests' golden vectors (tests/golden, written by make_golden.py
from the reference's own closed forms), exhaustive brute force, exact
rational arithmetic, and closed forms. Planted mistakes (wrong nibble order,
dropped zero point, transposed operand) must fail these checks.
"""
import itertools

import numpy as np
import pytest

import awq_oracle as oracle
from conftest import load_golden
from cube_awq import pack


def test_nibble_orders_known_answers():
    # Sequential: column c is bits 4c..4c+3 (src/kernel/awq_kernel.rs:8-19).
    w = 0x76543210
    assert [oracle.nibble_seq(w, c) for c in range(8)] == list(range(8))
    # AutoAWQ: packed lane p holds column [0,2,4,6,1,3,5,7][p]
    # (src/kernel/awq_kernel_gemm.rs:10-30 shifts {0,16,4,20} then {8,24,12,28}).
    assert [oracle.nibble_awq(w, c) for c in range(8)] == [0, 4, 1, 5, 2, 6, 3, 7]
    # The reference's pack_i4 (src/modules/awq_gemm.rs:270-277) round trip.
    vals = [3, 14, 1, 15, 9, 2, 6, 5]
    word = int(pack.pack(np.array([vals]), "awq")[0, 0])
    assert [oracle.nibble_awq(word, c) for c in range(8)] == vals
    # Unpacking at the reference's explicit shifts.
    shifts = [0, 16, 4, 20, 8, 24, 12, 28]
    assert [(word >> s) & 0xF for s in shifts] == vals


@pytest.mark.parametrize("name", ["dequant_seq_64x32_g2", "dequant_seq_128x32_g128"])
def test_dequant_matches_reference_golden(name):
    g = load_golden(name)
    out = oracle.dequant(g["qweight"], g["qzeros"], g["scales"], int(g["group_size"]), "seq")
    assert np.array_equal(out.view(np.uint32), g["expected"].view(np.uint32))


def test_dequant_golden_rejects_planted_mistakes():
    g = load_golden("dequant_seq_64x32_g2")
    gs = int(g["group_size"])
    wrong_order = oracle.dequant(g["qweight"], g["qzeros"], g["scales"], gs, "awq")
    assert not np.array_equal(wrong_order, g["expected"])
    no_zero = oracle.dequant(g["qweight"], np.zeros_like(g["qzeros"]), g["scales"], gs, "seq")
    assert not np.array_equal(no_zero, g["expected"])
    wrong_group = oracle.dequant(g["qweight"], np.repeat(g["qzeros"][::2], 2, 0),
                                 np.repeat(g["scales"][::2], 2, 0), gs, "seq")
    assert not np.array_equal(wrong_group, g["expected"])


def test_dequant_exhaustive_pairs_bit_exact():
    # All 256 (q, z) pairs x a sweep of scales, including signed zeros,
    # subnormals, a power of two and non-representable decimals.
    scales = np.array([1.0, -1.0, 0.0, -0.0, 0.1, 1e-40, -3.3e-39, 2.0 ** -126, 65504.0,
                       0.002, 0.0199, 7.25], np.float32)
    K, N = 256, 32 * len(scales)
    q = np.zeros((K, N), np.uint8)
    z = np.zeros((K, N), np.uint8)
    for r, (qq, zz) in enumerate(itertools.product(range(16), range(16))):
        q[r, :] = qq
        z[r, :] = zz
    # group size 1 so every row has its own zero row
    qw = pack.pack(q, "seq")
    qz = pack.pack(z, "seq")
    sc = np.tile(np.repeat(scales, 32)[None, :], (K, 1)).astype(np.float32)
    out = oracle.dequant(qw, qz, sc, 1, "seq")
    expect = ((q.astype(np.float32) - z.astype(np.float32)) * sc).astype(np.float32)
    assert np.array_equal(out.view(np.uint32), expect.view(np.uint32))
    # the q == z entries are +0.0 times s: sign follows s
    eq = q == z
    assert np.array_equal(np.signbit(out[eq]), np.signbit(sc[eq]))


def test_dequant_awq_order_matches_pack_helper():
    rng = np.random.default_rng(1)
    K, N, g = 64, 64, 16
    qn = rng.integers(0, 16, (K, N))
    zn = rng.integers(0, 16, (K // g, N))
    s = rng.uniform(-1, 1, (K // g, N)).astype(np.float32)
    out = oracle.dequant(pack.pack(qn, "awq"), pack.pack(zn, "awq"), s, g, "awq")
    expect = (qn.astype(np.float32) - np.repeat(zn, g, 0).astype(np.float32)) * np.repeat(s, g, 0)
    assert np.array_equal(out, expect.astype(np.float32))


@pytest.mark.parametrize("name", ["gemm_decode_b2m1_k64n32_g64", "gemm_fwd_b2m32_k64n32_g32",
                                  "gemm_fwd_bias_b2m32_k64n32_g32", "gemm_fwd_4d_1x16x14_k64n32_g32",
                                  "gemm_large_m_large_n"])
def test_gemm_f32_matches_reference_golden(name):
    g = load_golden(name)
    y = oracle.gemm_f32(g["x"], g["qweight"], g["qzeros"], g["scales"], int(g["group_size"]),
                        bias=g.get("bias"))
    # Same loop order and roundings as the reference's cpu_reference: bit-exact.
    assert np.array_equal(y.view(np.uint32), g["expected"].view(np.uint32))


def test_gemm_golden_rejects_planted_mistakes():
    g = load_golden("gemm_fwd_b2m32_k64n32_g32")
    gs = int(g["group_size"])
    ref = g["expected"]
    seq = oracle.gemm_f32(g["x"], g["qweight"], g["qzeros"], g["scales"], gs, order="seq")
    assert np.abs(seq - ref).max() > 1e-2
    xt = np.ascontiguousarray(g["x"][:, ::-1])  # permuted K
    assert np.abs(oracle.gemm_f32(xt, g["qweight"], g["qzeros"], g["scales"], gs) - ref).max() > 1e-2
    neg = oracle.gemm_f32(g["x"], g["qweight"], g["qzeros"], -g["scales"], gs)
    assert np.abs(neg - ref).max() > 1e-2


def test_gemm_f64_exact_rational():
    g = load_golden("gemm_exact_m3k64n32_g32")
    y = oracle.gemm_f64(g["x"], g["qweight"], g["qzeros"], g["scales"], int(g["group_size"]))
    np.testing.assert_allclose(y, g["expected"], rtol=1e-13, atol=1e-15)
    y32 = oracle.gemm_f32(g["x"], g["qweight"], g["qzeros"], g["scales"], int(g["group_size"]))
    assert oracle.rel_l2(y32, g["expected"]) < 1e-6


@pytest.mark.parametrize("w,z,s,x,expect_per_k", [
    (5, 0, 1.0, 1.0, 5.0),     # kernel_ones_input_uniform_weight_single_tile
    (8, 3, 2.0, 1.0, 10.0),    # kernel_uniform_with_nonzero_zero_point
    (2, 7, 1.0, 1.0, -5.0),    # kernel_negative_effective_weight
    (15, 0, 1.0, 1.0, 15.0),   # kernel_weight_nibble_at_max_15
    (0, 15, 1.0, 1.0, -15.0),  # kernel_weight_nibble_zero_zeropoint_fifteen
    (7, 0, 1.0, 0.0, 0.0),     # kernel_zero_input_yields_zero_output
    (5, 5, 2.0, 1.0, 0.0),     # kernel_zero_weight_yields_zero_output
    (15, 0, 0.0, 1.0, 0.0),    # kernel_zero_scale_yields_zero_output
    (6, 2, 0.25, 0.5, 0.5),    # kernel_four_k_tiles
])
def test_gemm_closed_forms(w, z, s, x, expect_per_k):
    # src/kernel/awq_kernel_gemm.rs:1125-1264: uniform nibbles give K * x * (w - z) * s.
    M, K, N, g = 4, 128, 32, 32
    qw = np.full((K, N // 8), int("%x" % w * 8, 16), np.uint32)
    qz = np.full((K // g, N // 8), int("%x" % z * 8, 16), np.uint32)
    sc = np.full((K // g, N), s, np.float32)
    xx = np.full((M, K), x, np.float32)
    y = oracle.gemm_f32(xx, qw, qz, sc, g)
    assert np.array_equal(y, np.full((M, N), K * expect_per_k, np.float32))


def test_gemm_per_group_scales_closed_form():
    # kernel_four_groups (src/kernel/awq_kernel_gemm.rs:1293-1316): scales 0.25*(g+1).
    M, K, N, g = 2, 128, 32, 32
    qw = np.full((K, N // 8), 0x77777777, np.uint32)
    qz = np.full((K // g, N // 8), 0x33333333, np.uint32)
    sc = np.repeat(np.array([0.25, 0.5, 0.75, 1.0], np.float32)[:, None], N, 1)
    y = oracle.gemm_f32(np.ones((M, K), np.float32), qw, qz, sc, g)
    assert np.all(y == 32 * 4 * (0.25 + 0.5 + 0.75 + 1.0))


def test_gemm_m_valid_leaves_rows():
    g = load_golden("gemm_fwd_b2m32_k64n32_g32")
    y = oracle.gemm_f32(g["x"], g["qweight"], g["qzeros"], g["scales"], int(g["group_size"]),
                        m_valid=10)
    assert np.array_equal(y[:10], g["expected"][:10])
    assert np.isnan(y[10:]).all()


def test_gemm_f64_vs_bruteforce_dequant():
    # The f64 GEMM equals (dequantised weight matrix) @ x in f64 on random data.
    rng = np.random.default_rng(7)
    M, K, N, g = 5, 256, 64, 64
    qw = rng.integers(0, 2 ** 32, (K, N // 8), dtype=np.uint64).astype(np.uint32)
    qz = rng.integers(0, 2 ** 32, (K // g, N // 8), dtype=np.uint64).astype(np.uint32)
    sc = rng.uniform(0.002, 0.02, (K // g, N)).astype(np.float32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = oracle.dequant(qw, qz, sc, g, "awq").astype(np.float64)
    y = oracle.gemm_f64(x, qw, qz, sc, g)
    np.testing.assert_allclose(y, x.astype(np.float64) @ w, rtol=1e-12, atol=1e-12)
