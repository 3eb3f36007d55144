"""C-ABI checks that run without a GPU: the library loads, exports every symbol
include/xrmm.h declares, and rejects invalid geometry before touching a device."""
import ctypes

import pytest

from xrgpu_amd import _native as nat


def test_library_exports_every_declared_symbol():
    lib = nat.lib()
    declared = nat.declared_symbols()
    assert len(declared) >= 7
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing


def test_version():
    assert b"gfx950" in nat.lib().xrmm_version()


@pytest.mark.parametrize("kw,msg", [
    (dict(bits=3), "bits"),
    (dict(block_size=0), "block_size"),
    (dict(K=0), "K must be positive"),
    (dict(N=0), "N required"),
    (dict(dtype=nat.I32), "T1"),
    (dict(zp_dtype=nat.I32), "zero points"),
])
def test_invalid_geometry_is_einval(kw, msg):
    args = dict(M=0, K=64, N=8, bits=4, block_size=32, dtype=nat.F16, zp_dtype=nat.UNSPECIFIED)
    args.update(kw)
    rc = nat.lib().xrmm_matmul_nbits(None, None, None, None, args["zp_dtype"], None, None, args["M"], args["K"],
                                     args["N"], args["bits"], args["block_size"], args["dtype"], None)
    assert rc == nat.XRMM_EINVAL
    assert msg in nat.last_error()


@pytest.mark.parametrize("K,msg", [(100, "multiple of 128"), (16384 + 128, "K up to 16384")])
def test_int8a_rejects_unsupported_k(K, msg):
    """The int8-activation GEMV holds a column's codes in one wave (at most
    16384 codes): a longer K is an error, not a silently truncated sum."""
    rc = nat.lib().xrmm_matmul_nbits_int8a(None, None, None, None, nat.UNSPECIFIED, None, None, None, 0, 1, K, 8,
                                           4, 32, nat.F16, None)
    assert rc == nat.XRMM_EINVAL and msg in nat.last_error()
    assert nat.lib().xrmm_matmul_nbits_int8a_workspace_bytes(1, K) == -1


def test_big_gemm_tile_threshold_override(monkeypatch):
    """XRMM_GEMM_BIG_MIN_TILES moves the 256 x 256 GEMM's tile threshold
    (read at every selection); malformed values keep the default."""
    sel = lambda: nat.lib().xrmm_select_kernel(0, 256, 1024, 256, 4, 128, nat.F16, nat.U8).decode()
    assert sel() == "gemm_q4_mfma"
    monkeypatch.setenv("XRMM_GEMM_BIG_MIN_TILES", "0")
    assert sel() == "gemm_q4_big"
    monkeypatch.setenv("XRMM_GEMM_BIG_MIN_TILES", "-3")
    assert sel() == "gemm_q4_mfma"
    monkeypatch.setenv("XRMM_GEMM_BIG_MIN_TILES", "12x")
    assert sel() == "gemm_q4_mfma"


def test_empty_m_is_a_no_op_without_device():
    # M = 0 (fixture empty_zero_dim): nothing to launch, returns OK
    rc = nat.lib().xrmm_matmul_nbits(None, None, None, None, nat.UNSPECIFIED, None, None, 0, 32, 4, 4, 32,
                                     nat.F32, None)
    assert rc == nat.XRMM_OK and nat.last_error() == ""


def test_qkv_requires_norm_scale():
    rc = nat.lib().xrmm_matmul_nbits_qkv(*([None] * 12), nat.UNSPECIFIED, None, None, None, None, 0, 64, 8, 8, 4, 32,
                                         ctypes.c_float(1e-6), nat.F16, None)
    assert rc == nat.XRMM_EINVAL and "normScaleT" in nat.last_error()


@pytest.mark.parametrize("op,M,K,N,bs,dtype,zp,expect", [
    (0, 1, 4096, 14336, 32, nat.F16, nat.UNSPECIFIED, "gemv_q4_dot"),
    (0, 4, 4096, 14336, 64, nat.F16, nat.U8, "gemv_q4_splitk"),
    (0, 2, 4096, 14336, 64, nat.F16, nat.U8, "gemv_q4_dot"),
    (2, 1, 4096, 14336, 32, nat.F16, nat.UNSPECIFIED, "gemv_q4_splitk"),
    (0, 8, 4096, 14336, 32, nat.F16, nat.UNSPECIFIED, "gemv_q4_splitk"),
    (0, 5, 2048, 14336, 64, nat.F16, nat.F16, "gemv_q4_splitk"),
    (0, 16, 1024, 14336, 32, nat.F16, nat.UNSPECIFIED, "gemv_q4_mfma"),   # 32 chunks: no even split
    (0, 16, 4096, 14336, 16, nat.F16, nat.UNSPECIFIED, "gemv_q4_mfma"),   # bs = 16
    (0, 2048, 4096, 14336, 128, nat.F16, nat.U8, "gemm_q4_big"),      # 448 tiles of 256 x 256
    (0, 2048, 14336, 4096, 128, nat.F16, nat.U8, "gemm_q4_big"),      # 128 tiles: half the CUs
    (0, 1024, 14336, 4096, 128, nat.F16, nat.U8, "gemm_q4_mfma"),     # 64 tiles: the 128 x 128 GEMM
    (0, 256, 4096, 14336, 128, nat.F16, nat.UNSPECIFIED, "gemm_q4_mfma"),
    (0, 128, 4096, 14336, 32, nat.F16, nat.F16, "gemm_q4_mfma"),      # float zero points: the same tile rule
    (0, 2048, 4096, 14336, 32, nat.F16, nat.F32, "gemm_q4_big"),
    (0, 127, 4096, 14336, 32, nat.F16, nat.U8, "gemm_q4_mfma"),
    (0, 64, 4096, 14336, 32, nat.F16, nat.F16, "gemv_q4_splitk"),    # four row chunks of 16
    (0, 65, 4096, 14336, 32, nat.F16, nat.F16, "gemm_q4_mfma"),
    (0, 64, 14336, 4096, 32, nat.F16, nat.U8, "gemm_q4_thin"),       # the down projection at 64 rows
    (0, 17, 512, 96, 16, nat.F16, nat.F16, "gemm_q4_thin"),          # no split-K GEMV shape for K = 512
    (1, 4, 4096, 4096, 64, nat.F16, nat.U8, "gemv_q4_mq"),
    (1, 4, 4096, 4096, 64, nat.F16, nat.F16, "gemv_q4_dot"),      # float zero points
    (1, 2, 8192, 4096, 32, nat.F16, nat.UNSPECIFIED, "gemv_q4_dot"),  # K beyond the MFMA GEMV's 4096
    (1, 4, 4096, 4096, 16, nat.F16, nat.U8, "gemv_q4_dot"),       # bs = 16
    (1, 8, 4096, 4096, 64, nat.F16, nat.U8, "gemv_q4_splitk"),
    (2, 16, 4096, 14336, 32, nat.F16, nat.UNSPECIFIED, "gemv_q4_splitk"),
    (2, 16, 3072, 8192, 32, nat.F16, nat.UNSPECIFIED, "gemv_q4_mfma"),
    (2, 17, 3072, 8192, 32, nat.F16, nat.UNSPECIFIED, "gemm_q4_thin"),    # Mlp prefill, 17..64 rows
    (2, 65, 3072, 8192, 32, nat.F16, nat.UNSPECIFIED, "gemm_q4_fused"),   # Mlp prefill past 64 rows
    (2, 2048, 4096, 14336, 64, nat.F16, nat.U8, "gemm_q4_big_fused"),  # 896 tiles of 256 staged columns
    (2, 256, 4096, 14336, 64, nat.F16, nat.U8, "gemm_q4_fused"),      # 112 tiles: the 128 x 128 GEMM
    (1, 2048, 4096, 4096, 64, nat.F16, nat.U8, "gemm_q4_big_fused"),  # Qkv prefill, one grid for Q, K, V
    (1, 128, 4096, 4096, 64, nat.F16, nat.U8, "gemm_q4_fused"),
    (1, 64, 2048, 512, 32, nat.F16, nat.U8, "gemv_q4_splitk"),          # Qkv, four row chunks
    (1, 65, 2048, 512, 32, nat.F16, nat.U8, "gemm_q4_fused"),           # Qkv prefill
    (1, 17, 4096, 4096, 16, nat.F16, nat.F16, "gemm_q4_fused"),
    (1, 32, 96, 16, 32, nat.F32, nat.UNSPECIFIED, "f32_proj"),          # float32 Qkv: prologue + float32 MatMulNBits
    (0, 1, 2048, 2048, 32, nat.F32, nat.U8, "gemv_q4_f32"),       # the CPU-oracle workload, float32
    (0, 4, 4096, 14336, 64, nat.F32, nat.F32, "gemv_q4_f32"),
    (0, 5, 2048, 2048, 32, nat.F32, nat.U8, "gemv_q4_f32"),         # float32 beyond four rows: chunks of four
    (0, 64, 4096, 4096, 32, nat.F32, nat.UNSPECIFIED, "gemm_f32_mfma"),  # float32, more than 16 rows: MFMA
    (0, 16, 4096, 4096, 32, nat.F32, nat.UNSPECIFIED, "gemm_f32_mfma"),  # 2^24 codes: MFMA from 12 rows
    (0, 11, 4096, 4096, 32, nat.F32, nat.UNSPECIFIED, "gemv_q4_f32"),
    (0, 5, 4096, 14336, 32, nat.F32, nat.UNSPECIFIED, "gemm_f32_mfma"),  # 2^25 codes or more: from 5 rows
    (0, 4, 4096, 14336, 32, nat.F32, nat.UNSPECIFIED, "gemv_q4_f32"),
    (0, 16, 2048, 5632, 32, nat.F32, nat.UNSPECIFIED, "gemv_q4_f32"),    # fewer codes: the GEMV up to 16 rows
    (0, 64, 4000, 4096, 32, nat.F32, nat.UNSPECIFIED, "gemm_f32_mfma"),  # padded K not a multiple of 64
    (0, 64, 4096, 4096, 16, nat.F32, nat.UNSPECIFIED, "gemv_q4_f32"),    # blocks of 16
    (0, 64, 4096, 4096, 32, nat.F32, nat.F32, "gemv_q4_f32"),            # float zero points, blocks of 32
    (0, 64, 4096, 4096, 64, nat.F32, nat.F32, "gemm_f32_mfma"),          # float zero points, blocks of 64
    (1, 8, 256, 64, 32, nat.F32, nat.UNSPECIFIED, "f32_proj"),        # float32 Qkv
    (2, 1, 2048, 5632, 32, nat.F32, nat.UNSPECIFIED, "f32_proj"),     # upstream mlp-q4-decode-k2048-n5632 (float32)
    (2, 64, 2048, 5632, 32, nat.F32, nat.UNSPECIFIED, "f32_proj"),    # upstream mlp-q4-prefill-m64-k2048-n5632
    (1, 8, 4096, 4096, 32, nat.F32, nat.UNSPECIFIED, "f32_proj"),     # upstream qkv-q4-llama-spec8
    (1, 4, 96, 64, 48, nat.F32, nat.UNSPECIFIED, "generic"),          # non-power-of-two blocks: the generic kernel
    (0, 1, 2048, 2048, 32, nat.F32, nat.U8, "gemv_q4_f32"),
    (0, 4, 16384, 14336, 16, nat.F16, nat.UNSPECIFIED, "generic"),  # dot staging would exceed 160 KB of LDS
    (0, 1, 33, 8, 32, nat.F16, nat.UNSPECIFIED, "generic"),
    (0, 4, 64, 8, 8, nat.F16, nat.UNSPECIFIED, "generic"),
])
def test_kernel_selection(op, M, K, N, bs, dtype, zp, expect):
    r = nat.lib().xrmm_select_kernel(op, M, K, N, 4, bs, dtype, zp)
    assert r.decode() == expect


def test_prepack_sizes_and_validation_without_device():
    lib = nat.lib()
    assert lib.xrmm_prepacked_bytes(14336, 4096, 4, 128) == 14336 * 4096 // 2
    assert lib.xrmm_prepacked_bytes(100, 96, 4, 32) == 2 * 100 * 32      # a K step and a half: the half is padded
    assert lib.xrmm_prepacked_bytes(100, 20, 4, 16) == 100 * 32          # one chunk of 32 codes
    assert lib.xrmm_prepacked_bytes(8, 64, 8, 32) == 0                   # 8-bit codes have no packed layout
    assert lib.xrmm_prepacked_bytes(8, 40, 4, 8) == 0                    # 40-code columns are not whole 32-code chunks
    rc = lib.xrmm_prepack_weights(None, None, 8, 64, 8, 32, None)
    assert rc == nat.XRMM_EINVAL and "4-bit" in nat.last_error()
    rc = lib.xrmm_prepack_weights(None, None, 8, 64, 4, 32, None)
    assert rc == nat.XRMM_EINVAL and "null" in nat.last_error()
    rc = lib.xrmm_matmul_nbits_prepacked(None, None, None, None, nat.UNSPECIFIED, None, None, 0, 64, 8, 4, 32,
                                         nat.F16, None)
    assert rc == nat.XRMM_OK  # M = 0: nothing to do


def test_fuzz_reaches_every_kernel_family():
    """The seeded GPU fuzz draws (tests/test_gpu_fuzz.py) must dispatch to every
    MatMulNBits-family kernel, so every family meets shapes nobody picked
    (checked here, without a device, through the dispatcher)."""
    import torch
    from tests import test_gpu_fuzz as F
    from xrgpu_amd import ops
    kind = {"none": None, "packed": "packed", "float_int": "float", "float": "float"}
    seen = set()
    for M, K, N, bits, bs, zp, _, dt in F.MM + F.MMF32 + F.MMF32P:
        seen.add(ops.select_kernel("MatMulNBits", M, K, N, bits, bs, torch.float16 if dt == "f16" else torch.float32,
                                   kind[zp]))
    for M, K, Nq, _, bs, zp, _ in F.QKV + F.QKV2:
        seen.add(ops.select_kernel("MatMulNBitsQkv", M, K, Nq, 4, bs, torch.float16, kind[zp]))
    for M, K, N, bs, *_ in F.MLP + F.MLP2:
        seen.add(ops.select_kernel("MatMulNBitsMlp", M, K, N, 4, bs, torch.float16))
    want = {"gemv_q4_dot", "gemv_q4_mq", "gemv_q4_splitk", "gemv_q4_mfma", "gemv_q4_f32", "gemm_f32_mfma", "gemm_q4_mfma",
            "gemm_q4_thin", "gemm_q4_fused", "generic"}
    assert want <= seen, f"not reached: {sorted(want - seen)}"


@pytest.mark.parametrize("op,M,K,N,bits,bs,dtype,zp,expect", [
    (0, 1, 2560, 4096, 8, 32, nat.F32, nat.UNSPECIFIED, "gemv_q4_f32"),  # the upstream q8 decode case, float32
    (0, 512, 2560, 4096, 8, 32, nat.F32, nat.U8, "gemm_f32_mfma"),       # the upstream q8 prefill case, float32: MFMA
    (0, 1, 2560, 4096, 8, 32, nat.F16, nat.UNSPECIFIED, "gemv_q4_f32"),  # float16 8-bit codes: float32 arithmetic
    (0, 512, 2560, 4096, 8, 64, nat.F16, nat.U8, "gemm_f32_mfma"),       # float16 8-bit prefill rows: MFMA
    (0, 512, 2560, 4096, 8, 16, nat.F16, nat.U8, "gemv_q4_f32"),         # blocks of 16: the GEMV
    (0, 512, 2560, 4096, 8, 64, nat.F16, nat.F16, "gemm_f32_mfma"),      # float zero points, blocks of 64: MFMA
    (0, 512, 2560, 4096, 8, 32, nat.F16, nat.F16, "gemv_q4_f32"),        # float zero points, blocks of 32: the GEMV
    (0, 512, 2560, 4096, 4, 64, nat.F32, nat.F16, "gemv_q4_f32"),        # zero points of another type: the GEMV
    (0, 512, 2560, 4096, 4, 64, nat.F32, nat.F32, "gemm_f32_mfma"),      # upstream qwen3 prefill zero-bias case
    (0, 48, 2561, 1021, 8, 32, nat.F32, nat.UNSPECIFIED, "gemm_f32_mfma"),  # upstream tail case (K % 4 != 0)
    (0, 128, 5120, 17408, 2, 128, nat.F16, nat.F16, "gemm_f32_mfma"),    # upstream bonsai2 case, float16 zero points
    (0, 1, 2048, 2048, 2, 32, nat.F32, nat.UNSPECIFIED, "gemv_q4_f32"),  # 2-bit codes, one row: the float32 GEMV
    (0, 2, 5120, 17408, 2, 128, nat.F16, nat.F16, "gemv_q4_f32"),        # 2-bit float16 decode (bonsai2 geometry)
    (0, 4, 5120, 17408, 2, 128, nat.F16, nat.F16, "gemv_q4_f32"),        # four rows of two chunks per lane: chunks of two rows
    (0, 16, 8192, 512, 2, 32, nat.F32, nat.UNSPECIFIED, "gemv_q4_f32"),  # 2-bit, 16 rows of K 8192: chunks of two rows
    (0, 128, 5120, 17408, 2, 128, nat.F16, nat.UNSPECIFIED, "gemm_f32_mfma"),  # upstream bonsai2 2-bit prefill
    (0, 64, 2048, 2048, 2, 32, nat.F32, nat.U8, "gemm_f32_mfma"),        # 2-bit, float32
    (0, 64, 2048, 2048, 4, 32, nat.F16, nat.UNSPECIFIED, "gemv_q4_splitk"),  # 4-bit float16: the binary16 kernels
])
def test_kernel_selection_bits(op, M, K, N, bits, bs, dtype, zp, expect):
    assert nat.lib().xrmm_select_kernel(op, M, K, N, bits, bs, dtype, zp).decode() == expect


@pytest.mark.parametrize("T,H,E,F1,k,bits,bs,act,fusion,expect", [
    (256, 4096, 4, 12800, 2, 4, 0, nat.ACT["swiglu"], 1, "qmoe_grouped"),   # many tokens, 4-bit row scales
    (16, 2048, 64, 1536, 2, 4, 0, nat.ACT["swiglu"], 1, "qmoe_grouped"),    # 32 (token, slot) pairs
    (15, 2048, 64, 1536, 2, 4, 0, nat.ACT["swiglu"], 1, "qmoe_rows"),       # 30 pairs: one pass per pair
    (256, 4096, 4, 12800, 2, 4, 64, nat.ACT["swiglu"], 1, "qmoe_grouped"),  # block scales
    (256, 4096, 4, 12800, 2, 8, 0, nat.ACT["swiglu"], 1, "qmoe_grouped"),   # 8-bit codes
    (256, 4096, 4, 12800, 2, 4, 16, nat.ACT["swiglu"], 1, "qmoe_rows"),     # blocks of 16: one pass per pair
    (256, 4000, 4, 12800, 2, 4, 0, nat.ACT["swiglu"], 1, "qmoe_rows"),      # H not a multiple of 64
    (64, 256, 4097, 256, 1, 4, 0, nat.ACT["relu"], 0, "qmoe_scalar"),       # more experts than either fast path counts
])
def test_qmoe_kernel_selection(T, H, E, F1, k, bits, bs, act, fusion, expect):
    """The grouped-expert path takes 4- or 8-bit experts with row scales or
    power-of-two blocks dividing H and I, and at least 32 pairs; the
    workspace holds its lists (two offsets per expert up to 4096 experts, two
    words per pair, one per token)."""
    lib = nat.lib()
    assert lib.xrmm_qmoe_kernel(T, H, E, F1, k, bits, bs, act, fusion).decode() == expect
    I = F1 // 2 if fusion else F1
    need_lists = 4 * (2 * 4097 + 2 * T * k + T)
    assert lib.xrmm_qmoe_workspace_bytes(T, k, H, I) >= 2 * 4 * T * k + 4 * T * k * I + 4 * T * k * H + need_lists
