"""Seeded synthetic AWQ tensors (portable, bit-reproducible on any host).

Generator: SplitMix64, one stream per tensor with seed 0xA77A0000 + tensor_id;
draw i (i = 0, 1, ...) is mix(seed + (i + 1) * 0x9E3779B97F4A7C15).
  * nibble U{0..15}: top 4 bits of one draw; 8 consecutive draws fill one
    packed word, draw j going to bits 4j..4j+3 (the packed lane; which logical
    column a lane is depends on the nibble order of the consumer).
  * U[a, b): a + (b - a) * (draw >> 40) / 2**24, in f64, then rounded once to
    the target dtype.
  * N(0, 1): Box-Muller in f64 over draw pairs (u1 = ((d0 >> 11) + 1) / 2**53,
    u2 = (d1 >> 11) / 2**53, r = sqrt(-2 ln u1), cos then sin), rounded once.
Tensor ids used by the tests and the benchmark: 0 activations, 1 qweight,
2 qzeros, 3 scales, 4 bias.
"""
import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
SEED_BASE = 0xA77A0000

TID_X, TID_QWEIGHT, TID_QZEROS, TID_SCALES, TID_BIAS = range(5)


_BLOCK = 1 << 17  # draws per block: keeps the uint64 temporaries in cache


def _draws(seed, start, count):
    """Draws start .. start+count-1 (0-based) of the stream seeded with `seed`."""
    with np.errstate(over="ignore"):
        z = np.arange(start + 1, start + count + 1, dtype=np.uint64)
        z *= _GOLDEN
        z += np.uint64(seed)
        t = z >> np.uint64(30)
        z ^= t
        z *= _M1
        np.right_shift(z, np.uint64(27), out=t)
        z ^= t
        z *= _M2
        np.right_shift(z, np.uint64(31), out=t)
        z ^= t
        return z


def splitmix64(seed, n):
    """First n draws of SplitMix64 seeded with `seed`, as uint64."""
    out = np.empty(n, dtype=np.uint64)
    for s in range(0, n, _BLOCK):
        out[s:s + _BLOCK] = _draws(seed, s, min(_BLOCK, n - s))
    return out


def packed_nibbles(tensor_id, rows, words_per_row):
    """uint32 [rows, words_per_row] of uniform 4-bit nibbles."""
    n = rows * words_per_row
    out = np.empty(n, dtype=np.uint32)
    wb = _BLOCK // 8
    for s in range(0, n, wb):
        e = min(n, s + wb)
        z = _draws(SEED_BASE + tensor_id, 8 * s, 8 * (e - s))
        z >>= np.uint64(60)
        nib = z.astype(np.uint32).reshape(-1, 8)
        w = nib[:, 0].copy()
        for j in range(1, 8):
            w |= nib[:, j] << np.uint32(4 * j)
        out[s:e] = w
    return out.reshape(rows, words_per_row)


def uniform(tensor_id, shape, a, b, dtype=np.float32):
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.uint16 if dtype == "bfloat16" else dtype)
    for s in range(0, n, _BLOCK):
        c = min(_BLOCK, n - s)
        u = (_draws(SEED_BASE + tensor_id, s, c) >> np.uint64(40)).astype(np.float64) / float(1 << 24)
        out[s:s + c] = _round_to(a + (b - a) * u, dtype)
    return out.reshape(shape)


def normal(tensor_id, shape, dtype=np.float32):
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.uint16 if dtype == "bfloat16" else dtype)
    pb = _BLOCK // 2
    for s in range(0, n, 2 * pb):  # s: first value of the block (even)
        c = min(2 * pb, n - s)
        pairs = (c + 1) // 2
        d = _draws(SEED_BASE + tensor_id, s, 2 * pairs).reshape(pairs, 2)
        u1 = ((d[:, 0] >> np.uint64(11)).astype(np.float64) + 1.0) / float(1 << 53)
        u2 = (d[:, 1] >> np.uint64(11)).astype(np.float64) / float(1 << 53)
        r = np.sqrt(-2.0 * np.log(u1))
        t = 2 * np.pi * u2
        z = np.stack([r * np.cos(t), r * np.sin(t)], axis=1).reshape(-1)[:c]
        out[s:s + c] = _round_to(z, dtype)
    return out.reshape(shape)


def _round_to(v64, dtype):
    """Round f64 values once to float32/float16, or to bfloat16 (returned as
    the uint16 bit patterns, round to nearest even)."""
    if dtype == "bfloat16":
        return _f64_to_bf16_bits(v64)
    return v64.astype(dtype)


def _f64_to_bf16_bits(v64):
    """Round f64 -> bf16 once (nearest, ties to even), as uint16 bits. Valid for
    finite values in the normal bf16 range, which is all the generators make."""
    v64 = np.asarray(v64, dtype=np.float64)
    sign = ((v64.view(np.uint64) >> np.uint64(63)).astype(np.uint16) << np.uint16(15))
    m, e = np.frexp(np.abs(v64))      # |v| = m * 2**e, m in [0.5, 1)
    q = np.rint(np.ldexp(m, 8))       # 8 significant bits, RNE (np.rint ties to even)
    r = np.ldexp(q, e - 8).astype(np.float32)  # exact: r has <= 8 significant bits
    return ((r.view(np.uint32) >> np.uint32(16)).astype(np.uint16)) | sign


def bf16_bits_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)
