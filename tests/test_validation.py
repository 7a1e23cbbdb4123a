"""Host-side behaviour that needs no GPU: the reference's launch validation
suite (src/kernel/awq_kernel_gemm.rs:965-1117), tile selection known answers
(src/modules/awq_gemm.rs:251-268), module build asserts, and every rejection
path of the launchers, all through the C ABI with the reference's messages."""
import re

import numpy as np
import pytest
import torch

import cube_awq
from cube_awq import (AWQGEMMLinear, AWQGEMMLinearConfig, AWQLinear, AWQLinearConfig, Panic,
                      ShapeConfig, validate_decode_launch_params, validate_launch_params)
from cube_awq import _lib

# ---- suite A: validate_launch_params -------------------------------------------------


def test_validate_accepts_minimal_valid_config():
    validate_launch_params(ShapeConfig.new(32, 32, 32, 32, 32, 32), 32)


def test_validate_accepts_large_multi_tile_config():
    validate_launch_params(ShapeConfig.new(128, 256, 512, 32, 32, 32), 128)


def test_validate_rejects_line_size_zero():
    s = ShapeConfig.new(32, 32, 32, 32, 32, 32)
    s.line_size = 0
    with pytest.raises(Panic, match="line_size must be > 0"):
        validate_launch_params(s, 32)


@pytest.mark.parametrize("args,gs,msg", [
    ((32, 32, 32, 0, 32, 32), 32, "m_tile_size must be > 0"),
    ((32, 32, 32, 32, 0, 32), 32, "n_tile_size must be > 0"),
    ((32, 32, 32, 32, 32, 0), 32, "inner_k_size must be > 0"),
    ((32, 32, 32, 32, 32, 32), 0, "group_size must be > 0"),
    ((32, 32, 6, 32, 32, 4), 2, "k must be divisible by line_size"),
    ((32, 6, 32, 32, 32, 32), 32, "n must be divisible by line_size"),
    ((32, 32, 32, 32, 32, 6), 32, "inner_k_size must be divisible by line_size"),
    ((32, 48, 32, 32, 32, 32), 32, "n must be divisible by n_tile_size"),
    ((32, 32, 48, 32, 32, 32), 16, "k must be divisible by inner_k_size"),
    ((32, 16, 32, 32, 16, 32), 32, "n_tile_size must be divisible by line_size\\*8"),
    ((32, 32, 32, 32, 32, 32), 24, "k must be divisible by group_size"),
    ((0, 32, 32, 32, 32, 32), 32, "m must be > 0"),
    ((32, 32, 32, 32, 32, 32), 1, "fast path requires group_size"),
    ((32, 32, 96, 32, 32, 32), 48, "fast path requires group_size"),
])
def test_validate_rejections(args, gs, msg):
    with pytest.raises(Panic, match=msg):
        validate_launch_params(ShapeConfig.new(*args), gs)


def test_validate_accepts_m_not_multiple_of_m_tile():
    validate_launch_params(ShapeConfig.new(48, 32, 32, 32, 32, 32), 32)


def test_validate_rejects_m_valid_larger_than_padded_m():
    with pytest.raises(Panic, match="m_valid must be <= m"):
        validate_launch_params(ShapeConfig.new_with_valid_m(32, 32, 32, 32, 32, 32, 33), 32)


def test_validate_exact_boundary_all_equal():
    validate_launch_params(ShapeConfig.new(32, 32, 32, 32, 32, 32), 32)


def test_validate_group_size_equals_k():
    validate_launch_params(ShapeConfig.new(32, 32, 64, 32, 32, 32), 64)


def test_validate_thread_mapping_rules_differ_between_paths():
    # Prefill maps 2 rows per thread, decode 1 (ROWS_PER_THREAD{,_DECODE}).
    s = ShapeConfig.new(8, 32, 64, 7, 32, 64)
    with pytest.raises(Panic, match="m_tile_size must be divisible by ROWS_PER_THREAD"):
        validate_launch_params(s, 64)
    validate_decode_launch_params(s, 64)


def test_validate_first_failing_check_wins():
    # Same order as the reference: group_size 0 is reported before k % line_size.
    with pytest.raises(Panic, match="group_size must be > 0"):
        validate_launch_params(ShapeConfig.new(32, 32, 6, 32, 32, 32), 0)


# ---- tile selection ---------------------------------------------------------------------


def test_select_tile_m_uses_small_tiles_for_decode_like_shapes():
    L = cube_awq.lib()
    assert [L.awq_select_tile_m(m) for m in (1, 8, 16, 17)] == [8, 8, 16, 32]


def test_select_tile_n_uses_large_tile_when_possible():
    L = cube_awq.lib()
    got = [L.awq_select_tile_n(n) for n in (32, 48, 64, 128, 192, 1536, 5632)]
    assert got == [32, 32, 64, 128, 64, 128, 128]


def test_decode_threshold():
    assert cube_awq.lib().awq_decode_m_threshold() == cube_awq.DECODE_M_THRESHOLD == 8


# ---- module build -----------------------------------------------------------------------


def test_config_build_shapes_without_bias():
    layer = AWQGEMMLinearConfig.new(64, 32, 32).build("cpu")
    assert tuple(layer.qweight.shape) == (64, 4)
    assert tuple(layer.qzeros.shape) == (2, 4)
    assert tuple(layer.scales.shape) == (2, 32)
    assert layer.group_size() == 32
    assert layer.bias is None


def test_config_build_shapes_with_bias():
    layer = AWQGEMMLinearConfig.new(64, 32, 32).with_bias(True).build("cpu")
    assert tuple(layer.bias.shape) == (32,)
    assert torch.all(layer.bias == 0)


@pytest.mark.parametrize("cfg,msg", [
    ((64, 32, 0), "group_size must be > 0"),
    ((64, 36, 4), "d_output must be divisible by 8"),
    ((64, 40, 64), re.escape("d_output must be divisible by TILE_N (32)")),
    ((96, 32, 32), re.escape("d_input must be divisible by INNER_K (64)")),
    ((128, 32, 96), "d_input must be divisible by group_size"),
])
def test_gemm_config_build_rejections(cfg, msg):
    with pytest.raises(Panic, match=msg):
        AWQGEMMLinearConfig.new(*cfg).build("cpu")


@pytest.mark.parametrize("cfg,msg", [
    ((64, 36, 2), re.escape("self.d_output % 8 == 0")),
    ((64, 32, 3), re.escape("self.d_input % self.group_size == 0")),
    ((64, 40, 2), re.escape("self.d_output % 32 == 0")),
])
def test_linear_config_build_rejections(cfg, msg):
    with pytest.raises(Panic, match=msg):
        AWQLinearConfig.new(*cfg).build("cpu")


def test_linear_group_size():
    # build_test_layer: 64 rows, 32 scale rows -> group size 2 (no %64 rule here).
    layer = AWQLinearConfig.new(64, 32, 2).build("cpu")
    assert layer.group_size() == 2


# ---- forward / launcher rejections (fail before any GPU work) --------------------------


def _layer(k=64, n=32, g=64, dtype=torch.float32):
    lay = AWQGEMMLinearConfig.new(k, n, g).build("cpu", dtype)
    lay.qweight.zero_()
    lay.qzeros.zero_()
    lay.scales.fill_(1.0)
    return lay


def test_forward_rejects_rank1():
    with pytest.raises(Panic, match=re.escape("input tensor must have at least 2 dims: [..., K]")):
        _layer().forward(torch.zeros(64))


def test_forward_rejects_k_zero():
    with pytest.raises(Panic, match=re.escape("input last dim (K) must be > 0")):
        _layer().forward(torch.zeros(2, 0))


def test_forward_rejects_k_mismatch():
    with pytest.raises(Panic, match=re.escape("input last dim (K) must match qweight rows")):
        _layer().forward(torch.zeros(1, 1, 128))


def test_forward_rejects_non_int_qweight():
    lay = _layer()
    lay.qweight = lay.qweight.to(torch.float32)
    with pytest.raises(Panic, match="qweight must have i32/u32 dtype"):
        lay.forward(torch.zeros(1, 64))


def test_forward_rejects_non_int_qzeros():
    lay = _layer()
    lay.qzeros = lay.qzeros.to(torch.int64)
    with pytest.raises(Panic, match="qzeros must have i32/u32 dtype"):
        lay.forward(torch.zeros(1, 64))


def test_module_forward_with_group32_panics_like_reference():
    # The module always validates with INNER_K = 64 (src/modules/awq_gemm.rs:207), so
    # group_size 32 fails "fast path requires ..." exactly as the reference would.
    lay = AWQGEMMLinear(torch.zeros(64, 4, dtype=torch.int32), torch.zeros(2, 4, dtype=torch.int32),
                        torch.ones(2, 32))
    with pytest.raises(Panic, match="fast path requires group_size >= inner_k_size"):
        lay.forward(torch.zeros(2, 32, 64))


def _gemm_linear(x, qw, qz, sc, out, shape, gs):
    cube_awq.awq_gemm_linear(x, qw, qz, sc, out, shape, gs)


@pytest.mark.parametrize("mut,msg", [
    (lambda t: t.update(x=torch.zeros(64)), re.escape("input must have shape [.., M, K] or [M, K]")),
    (lambda t: t.update(qw=torch.zeros(256, dtype=torch.int32)), re.escape("qweight must have shape [K, N/8]")),
    (lambda t: t.update(qz=torch.zeros(4, dtype=torch.int32)), re.escape("qzeros must have shape [K/G, N/8]")),
    (lambda t: t.update(sc=torch.zeros(32)), re.escape("scales must have shape [K/G, N]")),
    (lambda t: t.update(out=torch.zeros(32)), re.escape("output must have shape [.., M, N] or [M, N]")),
    (lambda t: t.update(x=torch.zeros(4, 0)), re.escape("input K must be > 0")),
    (lambda t: t.update(x=torch.zeros(4, 128)), "input K must match shape.k"),
    (lambda t: t.update(out=torch.zeros(4, 64)), "output N must match shape.n"),
    (lambda t: t.update(out=torch.zeros(5, 32)), "output rows must match flattened input rows"),
    (lambda t: t.update(qw=torch.zeros(128, 4, dtype=torch.int32)), "qweight K must match shape.k"),
    (lambda t: t.update(qw=torch.zeros(64, 8, dtype=torch.int32)), "qweight packed N must be N/8"),
    (lambda t: t.update(qz=torch.zeros(2, 4, dtype=torch.int32)), "qzeros rows must be K/group_size"),
    (lambda t: t.update(qz=torch.zeros(1, 8, dtype=torch.int32)), "qzeros packed N must be N/8"),
    (lambda t: t.update(sc=torch.zeros(2, 32)), "scales rows must be K/group_size"),
    (lambda t: t.update(sc=torch.zeros(1, 64)), "scales N must match shape.n"),
    (lambda t: t.update(qw=torch.zeros(64, 4)), "qweight must have i32/u32 dtype"),
    (lambda t: t.update(qz=torch.zeros(1, 4, dtype=torch.int64)), "qzeros must have i32/u32 dtype"),
])
def test_awq_gemm_linear_rejections(mut, msg):
    t = dict(x=torch.zeros(4, 64), qw=torch.zeros(64, 4, dtype=torch.int32),
             qz=torch.zeros(1, 4, dtype=torch.int32), sc=torch.zeros(1, 32), out=torch.zeros(4, 32))
    mut(t)
    shape = ShapeConfig.new(4, 32, 64, 8, 32, 64)
    with pytest.raises(Panic, match=msg):
        _gemm_linear(t["x"], t["qw"], t["qz"], t["sc"], t["out"], shape, 64)


def test_assert_eq_message_format():
    # assert_eq! panics print "assertion `left == right` failed: msg\n  left: ..\n right: ..".
    shape = ShapeConfig.new(4, 32, 64, 8, 32, 64)
    with pytest.raises(Panic) as e:
        _gemm_linear(torch.zeros(4, 128), torch.zeros(64, 4, dtype=torch.int32),
                     torch.zeros(1, 4, dtype=torch.int32), torch.zeros(1, 32), torch.zeros(4, 32),
                     shape, 64)
    assert str(e.value) == "assertion `left == right` failed: input K must match shape.k\n  left: 128\n right: 64"


@pytest.mark.parametrize("bad,which", [(torch.int16, "q_weight"), (torch.int64, "q_weight"),
                                       (torch.int16, "q_zeros"), (torch.int64, "q_zeros")])
def test_dequantize_rejects_non_32bit_packed(bad, which):
    # tests/awq_test.rs:223-377.
    qw = torch.zeros(32, 4, dtype=bad if which == "q_weight" else torch.int32)
    qz = torch.zeros(1, 4, dtype=bad if which == "q_zeros" else torch.int32)
    size = torch.tensor([], dtype=bad).element_size()
    with pytest.raises(Panic, match=re.escape(
            f"AWQ packed {which} must use 32-bit elements (i32/u32), got elem_size={size}.")):
        cube_awq.dequantize_native(qw, qz, torch.ones(1, 32), torch.zeros(32, 32), 32)


def test_dequantize_panics_on_invalid_out_width():
    # src/modules/awq_dequantize.rs:302-336.
    lay = AWQLinear(torch.zeros(64, 2, dtype=torch.int32), torch.zeros(16, 2, dtype=torch.int32),
                    torch.ones(16, 16))
    with pytest.raises(Panic, match=re.escape("out_width % 32 == 0")):
        lay.dequantize()


def test_linear_forward_rank3_panics_on_rank_mismatch():
    # src/modules/awq_dequantize.rs:283-300 (checked before the matmul runs)
    lay = AWQLinear(torch.zeros(64, 4, dtype=torch.int32), torch.zeros(32, 4, dtype=torch.int32),
                    torch.ones(32, 32))
    with pytest.raises(Panic, match="RankMismatch"):
        lay.forward(torch.zeros(2, 3, 64))


def test_pointer_abi_rejections():
    L = cube_awq.lib()
    rc = L.awq_gemm(None, _lib.AWQ_F32, None, None, None, _lib.AWQ_F32, None, 0, None,
                    _lib.AWQ_F32, 1, 96, 32, 64, None)
    assert rc == _lib.AWQ_ERR_INVALID
    assert L.awq_last_error().decode() == "k must be divisible by inner_k_size"
    rc = L.awq_dequantize(None, None, None, _lib.AWQ_F32, None, _lib.AWQ_F32, 64, 48, 2,
                          _lib.AWQ_ORDER_SEQUENTIAL, None)
    assert rc == _lib.AWQ_ERR_INVALID
    assert "out_width % 32 == 0" in L.awq_last_error().decode()
    rc = L.awq_gemm(None, 7, None, None, None, _lib.AWQ_F32, None, 0, None, _lib.AWQ_F32, 1, 64,
                    32, 64, None)
    assert rc == _lib.AWQ_ERR_INVALID and "input must have f32/f16/bf16 dtype" in L.awq_last_error().decode()


def test_misaligned_pointer_rejected():
    L = cube_awq.lib()
    rc = L.awq_gemm(8, _lib.AWQ_F32, 16, 16, 16, _lib.AWQ_F32, None, 0, 16, _lib.AWQ_F32, 1, 64,
                    32, 64, None)
    assert rc == _lib.AWQ_ERR_INVALID and "input must be 16-byte aligned" in L.awq_last_error().decode()


def test_last_error_cleared_on_success():
    L = cube_awq.lib()
    assert L.awq_validate_launch_params(None, 1) == _lib.AWQ_ERR_INVALID
    s = ShapeConfig.new(32, 32, 32, 32, 32, 32)._c()
    import ctypes
    assert L.awq_validate_launch_params(ctypes.byref(s), 32) == 0
    assert L.awq_last_error().decode() == ""


@pytest.mark.parametrize("M,K,N,g", [(1, 96, 32, 64), (1, 64, 48, 64), (1, 128, 32, 32), (1, 192, 32, 128),
                                     (64, 96, 32, 64), (64, 64, 48, 64), (64, 128, 32, 0), (9, 64, 40, 64),
                                     (0, 64, 32, 64), (8, 4096, 14336, 96)])
def test_validate_gemm_matches_awq_gemm(M, K, N, g):
    """awq_validate_gemm runs awq_gemm's shape checks alone: same result code
    and message, with no device pointer needed."""
    L = cube_awq.lib()
    rc_v = L.awq_validate_gemm(M, K, N, g)
    msg_v = L.awq_last_error().decode()
    rc_g = L.awq_gemm(None, _lib.AWQ_F32, None, None, None, _lib.AWQ_F32, None, 0, None,
                      _lib.AWQ_F32, M, K, N, g, None)
    msg_g = L.awq_last_error().decode()
    assert rc_v == rc_g == _lib.AWQ_ERR_INVALID
    assert msg_v == msg_g and msg_v


@pytest.mark.parametrize("M,K,N,g", [(1, 4096, 14336, 128), (8, 4096, 4096, 128), (2048, 4096, 14336, 128),
                                     (4096, 28672, 8192, 64), (9, 64, 32, 64)])
def test_validate_gemm_accepts_module_shapes(M, K, N, g):
    L = cube_awq.lib()
    assert L.awq_validate_gemm(M, K, N, g) == 0
    assert L.awq_last_error().decode() == ""


def test_silu_mul_rejects_width_not_multiple_of_64():
    L = cube_awq.lib()
    rc = L.awq_gemm_silu_mul(None, _lib.AWQ_F32, None, None, None, _lib.AWQ_F16, None, 0, None,
                             _lib.AWQ_F32, 1, 64, 96, 64, None)
    assert rc == _lib.AWQ_ERR_INVALID
    assert "N (gate and up interleaved) must be a multiple of 64" in L.awq_last_error().decode()


def test_interleave_packed_round_trip():
    import numpy as np
    import torch
    from cube_awq import pack
    rng = np.random.default_rng(3)
    a, b = rng.integers(0, 16, (9, 64)), rng.integers(0, 16, (9, 64))
    w = pack.interleave_packed(pack.pack(a, "awq"), pack.pack(b, "awq"))
    nib = pack.unpack(w, "awq")
    assert np.array_equal(nib[:, 0::2], a) and np.array_equal(nib[:, 1::2], b)
    t = pack.interleave_packed(torch.from_numpy(pack.pack(a, "awq").view(np.int32)),
                               torch.from_numpy(pack.pack(b, "awq").view(np.int32)))
    assert t.dtype == torch.int32 and np.array_equal(t.numpy().view(np.uint32), w)


@pytest.mark.parametrize("qz_rows,sc_rows,out_rows,msg", [
    (1, 2, 96, "q_zeros is too small"), (2, 1, 96, "q_scales is too small"),
    (2, 2, 95, "output is too small")])
def test_dequantize_native_rejects_out_of_bounds(qz_rows, sc_rows, out_rows, msg):
    # K = 96 rows, g = 64 -> groups 0 and 1. The reference reads these through
    # unchecked linear views; here a buffer too small to hold what the lines of
    # q_weight touch is rejected before any launch.
    with pytest.raises(Panic, match=msg):
        cube_awq.dequantize_native(torch.zeros(96, 4, dtype=torch.int32),
                                   torch.zeros(qz_rows, 4, dtype=torch.int32),
                                   torch.ones(sc_rows, 32), torch.zeros(out_rows, 32), 64)


def test_dequantize_native_rejects_division_by_zero():
    with pytest.raises(Panic, match="group_size must be > 0"):
        cube_awq.dequantize_native(torch.zeros(8, 4, dtype=torch.int32), torch.zeros(1, 4, dtype=torch.int32),
                                   torch.ones(1, 32), torch.zeros(8, 32), 0)
    with pytest.raises(Panic, match="out_width must be > 0"):
        cube_awq.dequantize_native(torch.zeros(8, 4, dtype=torch.int32), torch.zeros(1, 4, dtype=torch.int32),
                                   torch.ones(1, 32), torch.zeros(8, 0), 64)


def test_dequantize_native_empty_q_weight_is_a_no_op():
    # No lines, no work: accepted whatever the other sizes (as in the reference).
    cube_awq.dequantize_native(torch.zeros(0, 4, dtype=torch.int32), torch.zeros(0, 4, dtype=torch.int32),
                               torch.ones(0, 32), torch.zeros(0, 32), 0)


# AWQ_GEMM_FORCE_TILE_M is read the way the reference reads it
# (src/modules/awq_gemm.rs:20-28): std::env::var (absent or not Unicode ->
# no override), raw.trim() (Unicode White_Space), parse::<usize>() (optional
# '+', ASCII digits, no 64-bit overflow), kept if 8, 16 or 32. Read once per
# process (a OnceLock there), so each case runs in its own process.
_FORCE_CASES = [
    (b"16", 16), (b"+16", 16), (b"0000016", 16), (b"  32\t", 32), (b"\n8\r\n", 8),
    ("\u300016\u00a0".encode(), 16), ("16\u2028".encode(), 16), ("\u0085\u2003" "8\u3000".encode(), 8),
    (b"00000000000000000000000000000032", 32),
    (b"++16", None), (b"1 6", None), (b"\x1c16", None), (b"-16", None), (b"64", None), (b"", None),
    (b"+", None), (b"0x10", None), (b"18446744073709551616", None), (b"\xff16", None), (b"16.0", None),
    ("\u200b16".encode(), None)]


@pytest.mark.parametrize("raw,forced", _FORCE_CASES)
def test_forced_tile_m_parses_like_rust(raw, forced):
    import os
    import subprocess
    import sys
    from cube_awq import _lib as lib_mod
    code = ("import ctypes, sys; L = ctypes.CDLL(sys.argv[1]); "
            "L.awq_select_tile_m.restype = ctypes.c_int64; "
            "L.awq_select_tile_m.argtypes = [ctypes.c_int64]; print(L.awq_select_tile_m(100))")
    env = {k: v for k, v in os.environb.items() if k != b"AWQ_GEMM_FORCE_TILE_M"}
    env[b"AWQ_GEMM_FORCE_TILE_M"] = raw
    out = subprocess.run([sys.executable, "-c", code, lib_mod.LIB_PATH], env=env, check=True,
                         capture_output=True).stdout
    assert int(out) == (forced if forced is not None else 32), raw
