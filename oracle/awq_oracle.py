"""Python front of the CPU parity oracle (oracle/awq_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker. Nothing in the product
(cube-awq_amd/) imports it.

All inputs are numpy arrays. Activations, scales and bias may be float32,
float16 or bfloat16 bit patterns (uint16, pass `bf16=True`); they are widened
to float32 exactly before the C restatement runs, so the oracle is the
reference's F = f32 computation on the exactly-upcast values.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle_awq.so")
ORDER = {"awq": 0, "seq": 1}

_lib = None


def build():
    subprocess.run(["make", "-B", "-C", _HERE], check=True, stdout=subprocess.DEVNULL)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        h = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        I = ctypes.c_int64
        h.awqo_nibble_seq.restype = ctypes.c_uint32
        h.awqo_nibble_seq.argtypes = [ctypes.c_uint32, ctypes.c_int]
        h.awqo_nibble_awq.restype = ctypes.c_uint32
        h.awqo_nibble_awq.argtypes = [ctypes.c_uint32, ctypes.c_int]
        h.awqo_dequant_f32.restype = None
        h.awqo_dequant_f32.argtypes = [P, P, P, P, I, I, I, ctypes.c_int]
        h.awqo_gemm_f32.restype = None
        h.awqo_gemm_f32.argtypes = [P, P, P, P, P, P, I, I, I, I, I, ctypes.c_int]
        h.awqo_gemm_f64.restype = None
        h.awqo_gemm_f64.argtypes = [P, P, P, P, P, P, I, I, I, I, ctypes.c_int]
        h.awqo_num_threads.restype = ctypes.c_int
        h.awqo_num_threads.argtypes = []
        _lib = h
    return _lib


def to_f32(a, bf16=False):
    """Exact widening to contiguous float32."""
    a = np.asarray(a)
    if bf16:
        return np.ascontiguousarray((a.astype(np.uint16).astype(np.uint32) << 16).view(np.float32))
    return np.ascontiguousarray(a.astype(np.float32))


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def nibble_seq(word, col):
    return lib().awqo_nibble_seq(word, col)


def nibble_awq(word, col):
    return lib().awqo_nibble_awq(word, col)


def dequant(qweight, qzeros, scales, group_size, order="seq", scales_bf16=False):
    """[K, N] float32 = (q - z) * s."""
    qw = np.ascontiguousarray(np.asarray(qweight).view(np.uint32))
    qz = np.ascontiguousarray(np.asarray(qzeros).view(np.uint32))
    s = to_f32(scales, scales_bf16)
    K, N = qw.shape[0], qw.shape[1] * 8
    out = np.empty((K, N), dtype=np.float32)
    lib().awqo_dequant_f32(_p(qw), _p(qz), _p(s), _p(out), K, N, group_size, ORDER[order])
    return out


def _gemm_args(x, qweight, qzeros, scales, bias, x_bf16, s_bf16, b_bf16):
    qw = np.ascontiguousarray(np.asarray(qweight).view(np.uint32))
    qz = np.ascontiguousarray(np.asarray(qzeros).view(np.uint32))
    xf = to_f32(x, x_bf16)
    sf = to_f32(scales, s_bf16)
    bf = to_f32(bias, b_bf16) if bias is not None else None
    return xf, qw, qz, sf, bf


def gemm_f32(x, qweight, qzeros, scales, group_size, bias=None, order="awq", m_valid=None,
             x_bf16=False, s_bf16=False, b_bf16=False):
    """[M, N] float32, the reference's sequential-k f32 loop (rows >= m_valid
    left as NaN)."""
    xf, qw, qz, sf, bf = _gemm_args(x, qweight, qzeros, scales, bias, x_bf16, s_bf16, b_bf16)
    M, K = xf.shape
    N = qw.shape[1] * 8
    y = np.full((M, N), np.nan, dtype=np.float32)
    lib().awqo_gemm_f32(_p(xf), _p(qw), _p(qz), _p(sf), _p(bf), _p(y), M, K, N, group_size,
                        M if m_valid is None else m_valid, ORDER[order])
    return y


def gemm_f64(x, qweight, qzeros, scales, group_size, bias=None, order="awq",
             x_bf16=False, s_bf16=False, b_bf16=False):
    """[M, N] float64 sum of the same f32-dequantised weights."""
    xf, qw, qz, sf, bf = _gemm_args(x, qweight, qzeros, scales, bias, x_bf16, s_bf16, b_bf16)
    M, K = xf.shape
    N = qw.shape[1] * 8
    y = np.empty((M, N), dtype=np.float64)
    lib().awqo_gemm_f64(_p(xf), _p(qw), _p(qz), _p(sf), _p(bf), _p(y), M, K, N, group_size,
                        ORDER[order])
    return y


def num_threads():
    return lib().awqo_num_threads()


def rel_l2(actual, expected):
    """||a - e||_2 / ||e||_2 in f64 (0 if both are zero)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    den = np.linalg.norm(e)
    num = np.linalg.norm(a - e)
    return float(num / den) if den > 0 else float(num)
