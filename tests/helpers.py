"""Shared helpers of the GPU parity tests: seeded inputs (cube_awq.synth) in
numpy, their device copies, and conversions that keep the exact bits."""
import numpy as np
import torch

from cube_awq import synth

NP_OF = {"f32": np.float32, "f16": np.float16}
TORCH_OF = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def to_device(a, dt, dev):
    """numpy array (bf16 given as uint16 bits) -> torch tensor of dtype dt on dev."""
    if dt == "bf16":
        return torch.from_numpy(np.ascontiguousarray(a.astype(np.uint16)).view(np.int16)).to(dev).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def to_host(t):
    """torch tensor -> numpy (bf16 returned as uint16 bits)."""
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.uint32:
        return t.view(torch.int32).numpy().view(np.uint32)
    return t.numpy()


def host_f32(a, dt):
    """Exact float32 view of a host array of logical dtype dt."""
    if dt == "bf16":
        return synth.bf16_bits_to_f32(a)
    return a.astype(np.float32)


def round_to(a32, dt):
    """Round float32 values once to dt (RNE), returned as host array of that dt."""
    a32 = np.asarray(a32, dtype=np.float32)
    if dt == "f32":
        return a32
    if dt == "f16":
        return a32.astype(np.float16)
    b = a32.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(a32)
    r[nan] = ((b[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def make_problem(M, K, N, g, x_dt="f32", s_dt="f16", scale_range=(0.002, 0.02), bias=False):
    """Seeded AWQ problem in host arrays: x [M, K], qweight, qzeros, scales, bias."""
    x = synth.normal(synth.TID_X, (M, K), "bfloat16" if x_dt == "bf16" else NP_OF[x_dt])
    qw = synth.packed_nibbles(synth.TID_QWEIGHT, K, N // 8)
    qz = synth.packed_nibbles(synth.TID_QZEROS, K // g, N // 8)
    sc = synth.uniform(synth.TID_SCALES, (K // g, N), *scale_range,
                       dtype="bfloat16" if s_dt == "bf16" else NP_OF[s_dt])
    b = synth.uniform(synth.TID_BIAS, (N,), -1.0, 1.0, dtype=np.float32) if bias else None
    return x, qw, qz, sc, b
