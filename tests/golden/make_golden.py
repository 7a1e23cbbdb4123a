"""Writes the golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

Every fixture restates one of the reference's own test cases: the same input
formulas, packing helper and CPU expectation loop, evaluated here with numpy
float32 arithmetic (each operation rounded to f32, never fused, matching the
Rust f32 expressions) or exactly with fractions. Nothing here calls the
oracle or the product library, so the fixtures can pin both.

  dequant_seq_64x32_g2      src/modules/awq_dequantize.rs:133-206 (build_test_layer)
  dequant_seq_128x32_g128   tests/awq_test.rs:117-221 (test_awq_kernel)
  gemm_decode_b2m1_k64n32_g64   src/modules/awq_gemm.rs:279-342, 517-559
  gemm_fwd_b2m32_k64n32_g32     src/modules/awq_gemm.rs:408-450
  gemm_fwd_bias_b2m32_k64n32_g32 src/modules/awq_gemm.rs:452-503
  gemm_fwd_4d_1x16x14_k64n32_g32 src/modules/awq_gemm.rs:561-604
  gemm_large_m_large_n      src/kernel/awq_kernel_gemm.rs:1348-1361 (input (i % 7) * 0.1)
  gemm_exact_m3k64n32_g32   seeded random tiny case, exact rational sum (f64 golden)
"""
import os
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
F = np.float32

AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)
AWQ_REVERSE_ORDER = (0, 4, 1, 5, 2, 6, 3, 7)


def pack_seq(vals):
    """pack_i4 of src/modules/awq_dequantize.rs:121-127 / pack_u32_cpu of tests/awq_test.rs:104-112."""
    p = 0
    for i, v in enumerate(vals):
        p |= (int(v) & 0xF) << (4 * i)
    return p


def pack_awq(vals):
    """pack_i4 of src/modules/awq_gemm.rs:270-277: packed lane p <- logical AWQ_ORDER[p]."""
    p = 0
    for packed_lane, logical in enumerate(AWQ_ORDER):
        p |= (int(vals[logical]) & 0xF) << (4 * packed_lane)
    return p


def unpack_awq(packed, logical_lane):
    """unpack_i4 of src/modules/awq_gemm.rs:279-282."""
    return (packed >> (AWQ_REVERSE_ORDER[logical_lane] * 4)) & 0xF


def unpack_seq(packed, idx):
    return (packed >> (idx * 4)) & 0xF


def dequant_seq_64x32_g2():
    height, out_width = 64, 32
    pw = out_width // 8
    g = height // out_width
    ng = height // g
    qw = np.zeros((height, pw), np.uint32)
    qz = np.zeros((ng, pw), np.uint32)
    sc = np.zeros((ng, out_width), np.float32)
    for r in range(height):
        for cb in range(pw):
            qw[r, cb] = pack_seq([(r + cb + i) % 16 for i in range(8)])
    for gi in range(ng):
        for cb in range(pw):
            qz[gi, cb] = pack_seq([(gi + cb + i) % 8 for i in range(8)])
        for c in range(out_width):
            sc[gi, c] = F(0.5) + F(gi) * F(0.01) + F(c) * F(0.001)
    exp = np.zeros((height, out_width), np.float32)
    for r in range(height):
        gi = r // g
        for c in range(out_width):
            w = F(unpack_seq(int(qw[r, c // 8]), c % 8))
            z = F(unpack_seq(int(qz[gi, c // 8]), c % 8))
            exp[r, c] = (w - z) * sc[gi, c]
    return dict(qweight=qw, qzeros=qz, scales=sc, expected=exp, group_size=np.int64(g))


def dequant_seq_128x32_g128():
    height, out_width, g = 128, 32, 128
    pw = out_width // 8
    qw = np.zeros((height, pw), np.uint32)
    qz = np.zeros((height // g, pw), np.uint32)
    sc = np.zeros((height // g, out_width), np.float32)
    exp = np.zeros((height, out_width), np.float32)
    for r in range(height):
        for cb in range(pw):
            w_vals = [(r + cb + i) % 15 for i in range(8)]
            z_vals = [(i + 1) % 8 for i in range(8)]
            qw[r, cb] = pack_seq(w_vals)
            if r == 0:
                qz[0, cb] = pack_seq(z_vals)
            for i in range(8):
                col = cb * 8 + i
                s = F(0.5) + F(col) * F(0.1)
                if r == 0:
                    sc[0, col] = s
                exp[r, col] = (F(w_vals[i]) - F(z_vals[i])) * s
    return dict(qweight=qw, qzeros=qz, scales=sc, expected=exp, group_size=np.int64(g))


def build_layer(k, n, g):
    """build_layer of src/modules/awq_gemm.rs:284-342 (AWQ-ordered packs)."""
    npk = n // 8
    ng = k // g
    qw = np.zeros((k, npk), np.uint32)
    qz = np.zeros((ng, npk), np.uint32)
    sc = np.zeros((ng, n), np.float32)
    for row in range(k):
        for col in range(npk):
            qw[row, col] = pack_awq([(row + col + lane) % 16 for lane in range(8)])
    for gi in range(ng):
        for col in range(npk):
            qz[gi, col] = pack_awq([(gi + col + lane) % 8 for lane in range(8)])
        for col in range(n):
            sc[gi, col] = F(0.05) + F(gi) * F(0.01) + F(col) * F(0.002)
    return qw, qz, sc


def awq_weights_f32(qw, qz, sc, g):
    """(w - z) * scale per element, f32, AWQ order (cpu_reference's inner term)."""
    k, npk = qw.shape
    n = npk * 8
    w = np.zeros((k, n), np.float32)
    for kk in range(k):
        gi = kk // g
        for col in range(n):
            wv = F(unpack_awq(int(qw[kk, col // 8]), col % 8))
            zv = F(unpack_awq(int(qz[gi, col // 8]), col % 8))
            w[kk, col] = (wv - zv) * sc[gi, col]
    return w


def cpu_reference(x, w, bias=None):
    """cpu_reference of src/modules/awq_gemm.rs:322-341: one f32 accumulator per
    output, k ascending, acc += x * w (two roundings), bias added last."""
    m, k = x.shape
    acc = np.zeros((m, w.shape[1]), np.float32)
    for kk in range(k):
        prod = x[:, kk:kk + 1] * w[kk:kk + 1, :]  # f32 multiply
        acc = acc + prod                           # f32 add
    if bias is not None:
        acc = acc + bias[None, :]
    return acc


def gemm_case(batch, m, k, n, g, input_fn, bias=None, dims=None):
    qw, qz, sc = build_layer(k, n, g)
    rows = batch * m
    x = np.array([input_fn(i) for i in range(rows * k)], np.float32).reshape(rows, k)
    w = awq_weights_f32(qw, qz, sc, g)
    exp = cpu_reference(x, w, bias)
    out = dict(qweight=qw, qzeros=qz, scales=sc, x=x, expected=exp, group_size=np.int64(g),
               dims=np.array(dims if dims else (batch, m, k), np.int64))
    if bias is not None:
        out["bias"] = bias
    return out


def gemm_large_m_large_n():
    # kernel_large_m_large_n: M=128, K=32, N=128, g=32, uniform w=4, z=2, s=0.5,
    # input (i % 7) * 0.1; expected via cpu_ref (src/kernel/awq_kernel_gemm.rs:793-829).
    m, k, n, g = 128, 32, 128, 32
    qw = np.full((k, n // 8), 0x44444444, np.uint32)
    qz = np.full((k // g, n // 8), 0x22222222, np.uint32)
    sc = np.full((k // g, n), 0.5, np.float32)
    x = np.array([F(i % 7) * F(0.1) for i in range(m * k)], np.float32).reshape(m, k)
    w = awq_weights_f32(qw, qz, sc, g)
    return dict(qweight=qw, qzeros=qz, scales=sc, x=x, expected=cpu_reference(x, w),
                group_size=np.int64(g), dims=np.array((1, m, k), np.int64))


def gemm_exact_m3k64n32_g32():
    """Random nibbles and scales (fixed numpy seed); expected is the exact
    rational sum_k x * ((q - z) * s)_f32, rounded once to f64."""
    rng = np.random.default_rng(20251201)
    m, k, n, g = 3, 64, 32, 32
    qn = rng.integers(0, 16, size=(k, n))
    zn = rng.integers(0, 16, size=(k // g, n))
    sc = rng.uniform(0.002, 0.02, size=(k // g, n)).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    qw = np.zeros((k, n // 8), np.uint32)
    qz = np.zeros((k // g, n // 8), np.uint32)
    for r in range(k):
        for p in range(n // 8):
            qw[r, p] = pack_awq(qn[r, p * 8:(p + 1) * 8])
    for r in range(k // g):
        for p in range(n // 8):
            qz[r, p] = pack_awq(zn[r, p * 8:(p + 1) * 8])
    exp = np.zeros((m, n), np.float64)
    for i in range(m):
        for j in range(n):
            acc = Fraction(0)
            for kk in range(k):
                wq = F(F(int(qn[kk, j])) - F(int(zn[kk // g, j]))) * sc[kk // g, j]  # f32 weight
                acc += Fraction(float(x[i, kk])) * Fraction(float(wq))
            exp[i, j] = float(acc)
    return dict(qweight=qw, qzeros=qz, scales=sc, x=x, expected=exp, group_size=np.int64(g),
                qn=qn.astype(np.uint8), zn=zn.astype(np.uint8))


def main():
    cases = {
        "dequant_seq_64x32_g2": dequant_seq_64x32_g2(),
        "dequant_seq_128x32_g128": dequant_seq_128x32_g128(),
        "gemm_decode_b2m1_k64n32_g64": gemm_case(2, 1, 64, 32, 64, lambda i: (F(i % 11) - F(5.0)) * F(0.09)),
        "gemm_fwd_b2m32_k64n32_g32": gemm_case(2, 32, 64, 32, 32, lambda i: (F(i % 17) - F(8.0)) * F(0.1)),
        "gemm_fwd_bias_b2m32_k64n32_g32": gemm_case(
            2, 32, 64, 32, 32, lambda i: (F(i % 13) - F(6.0)) * F(0.07),
            bias=np.array([F(-0.2) + F(i) * F(0.01) for i in range(32)], np.float32)),
        "gemm_fwd_4d_1x16x14_k64n32_g32": gemm_case(
            1, 16 * 14, 64, 32, 32, lambda i: (F(i % 23) - F(11.0)) * F(0.03), dims=(1, 16, 14, 64)),
        "gemm_large_m_large_n": gemm_large_m_large_n(),
        "gemm_exact_m3k64n32_g32": gemm_exact_m3k64n32_g32(),
    }
    for name, arrays in cases.items():
        np.savez(os.path.join(HERE, name + ".npz"), **arrays)
        print("wrote", name, {k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    main()
