"""Nibble packing between logical 4-bit matrices [R, N] and packed words [R, N/8].

AutoAWQ order (what the fused GEMM reads): packed lane p (bits 4p..4p+3) holds
logical column AWQ_ORDER[p] of its 8-column pack, i.e. logical column c sits
in lane AWQ_REVERSE_ORDER[c] (reference src/modules/awq_gemm.rs:248-277,
src/kernel/awq_kernel_gemm.rs:7-30).
Sequential order (what the standalone dequantize reads): column c is lane c
(reference src/kernel/awq_kernel.rs:8-19).
"""
import numpy as np

AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)
AWQ_REVERSE_ORDER = (0, 4, 1, 5, 2, 6, 3, 7)


def _lanes(order):
    if order == "awq":
        return np.array(AWQ_REVERSE_ORDER, dtype=np.uint32)  # lane of logical column c
    if order == "seq":
        return np.arange(8, dtype=np.uint32)
    raise ValueError(f"order must be 'awq' or 'seq', got {order!r}")


def pack(nibbles, order):
    """uint values in [0, 16) of shape [R, N] (N % 8 == 0) -> uint32 [R, N/8]."""
    a = np.asarray(nibbles)
    r, n = a.shape
    assert n % 8 == 0, "N must be a multiple of 8"
    cols = (a.astype(np.uint32) & np.uint32(0xF)).reshape(r, n // 8, 8)
    shifts = (_lanes(order) * np.uint32(4))[None, None, :]
    return np.bitwise_or.reduce(cols << shifts, axis=2).astype(np.uint32)


def unpack(words, order):
    """uint32 [R, N/8] -> uint8 [R, N] of logical nibbles."""
    w = np.asarray(words).astype(np.uint32)
    r, np_ = w.shape
    shifts = (_lanes(order) * np.uint32(4))[None, None, :]
    return ((w[:, :, None] >> shifts) & np.uint32(0xF)).astype(np.uint8).reshape(r, np_ * 8)


def interleave_columns(a, b):
    """[R, N] and [R, N] -> [R, 2N] with column 2j = a[:, j], 2j + 1 = b[:, j]
    (numpy or torch). The gate/up layout of the fused SiLU epilogue."""
    if hasattr(a, "dim"):  # torch
        import torch
        return torch.stack([a, b], dim=-1).reshape(a.shape[0], 2 * a.shape[1])
    return np.stack([np.asarray(a), np.asarray(b)], axis=-1).reshape(a.shape[0], 2 * a.shape[1])


def interleave_packed(a_words, b_words):
    """Two AutoAWQ-order packed tensors [R, N/8] -> one [R, 2N/8] whose
    logical column 2j is column j of a and 2j + 1 column j of b (int32 or
    uint32 torch tensors on any device, or numpy; same kind and dtype out)."""
    if not hasattr(a_words, "dim"):
        return pack(interleave_columns(unpack(a_words, "awq"), unpack(b_words, "awq")), "awq")
    import torch
    lanes = torch.tensor(AWQ_REVERSE_ORDER, dtype=torch.int64, device=a_words.device) * 4

    def logical(w):  # int64 nibbles [R, N]
        w64 = w.to(torch.int64) & 0xFFFFFFFF
        return ((w64[:, :, None] >> lanes) & 0xF).reshape(w.shape[0], -1)

    nib = interleave_columns(logical(a_words), logical(b_words))
    words = (nib.reshape(nib.shape[0], -1, 8) << lanes).sum(dim=-1)  # disjoint bits: sum == or
    words = torch.where(words >= 2 ** 31, words - 2 ** 32, words).to(torch.int32)
    return words if a_words.dtype == torch.int32 else words.view(a_words.dtype)


def as_int32(words):
    """Reinterpret packed uint32 words as int32 (AutoAWQ checkpoints store int32)."""
    return np.asarray(words, dtype=np.uint32).view(np.int32)
