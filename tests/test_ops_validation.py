"""CPU: the torch front end rejects shapes and dtypes the kernels would read or
write past, before any device work (the kernels take raw pointers and derive
byte ranges from M, K and N)."""
import pytest

torch = pytest.importorskip("torch")

from xrgpu_amd import _native as nat  # noqa: E402
from xrgpu_amd import ops  # noqa: E402


def u8(*shape):
    return torch.zeros(shape, dtype=torch.uint8)


def f16(*shape):
    return torch.zeros(shape, dtype=torch.float16)


def f32(*shape):
    return torch.zeros(shape, dtype=torch.float32)


M, K, N, BS = 2, 64, 8, 32
KB = K // BS


def mnb_args():
    return f16(M, K), u8(N, KB, BS // 2), f16(N, KB)


def test_valid_call_reaches_the_device_check():
    with pytest.raises(nat.XrmmInvalid, match="on the GPU"):
        ops.matmul_nbits(*mnb_args(), block_size=BS)


@pytest.mark.parametrize("out", [f16(M, N + 1), f32(M, N), f16(M * N)])
def test_matmul_nbits_rejects_mismatched_out(out):
    with pytest.raises(nat.XrmmInvalid, match="out must be"):
        ops.matmul_nbits(*mnb_args(), block_size=BS, out=out)


def test_mlp_rejects_mixed_zero_point_dtypes():
    A, B, S = mnb_args()
    with pytest.raises(nat.XrmmInvalid, match="share a dtype"):
        ops.matmul_nbits_mlp(A, B, S, B.clone(), S.clone(), block_size=BS, gate_zero_points=f16(N, KB),
                             up_zero_points=u8(N, 1))


def test_qkv_rejects_mixed_zero_point_dtypes():
    A, B, S = mnb_args()
    with pytest.raises(nat.XrmmInvalid, match="share a dtype"):
        ops.matmul_nbits_qkv(A, B, S, B, S, B, S, norm_scale=f16(K), block_size=BS, q_zero_points=u8(N, 1),
                             k_zero_points=f16(N, KB))


@pytest.mark.parametrize("kw,msg", [
    (dict(skip=f16(M, K - 8)), "skip"),
    (dict(skip=f32(M, K)), "skip"),
    (dict(norm_scale=f32(K)), "norm_scale"),
    (dict(norm_scale=f16(K // 2)), "norm_scale"),
])
def test_qkv_rejects_bad_skip_and_norm_scale(kw, msg):
    A, B, S = mnb_args()
    args = dict(norm_scale=f16(K))
    args.update(kw)
    with pytest.raises(nat.XrmmInvalid, match=msg):
        ops.matmul_nbits_qkv(A, B, S, B, S, B, S, block_size=BS, **args)


def test_qkv_requires_norm_scale():
    A, B, S = mnb_args()
    with pytest.raises(nat.XrmmInvalid, match="normScaleT"):
        ops.matmul_nbits_qkv(A, B, S, B, S, B, S, norm_scale=None, block_size=BS)


@pytest.mark.parametrize("kw,msg", [
    (dict(skip=f16(M + 1, K)), "skip"),
    (dict(norm_scale=f32(K)), "norm_scale"),
    (dict(gate_bias=f16(N + 1)), "gate_bias"),
    (dict(up_bias=f32(N)), "up_bias"),
    (dict(up_bias=f16(1, N)), "up_bias"),
])
def test_mlp_rejects_bad_auxiliary_inputs(kw, msg):
    A, B, S = mnb_args()
    with pytest.raises(nat.XrmmInvalid, match=msg):
        ops.matmul_nbits_mlp(A, B, S, B.clone(), S.clone(), block_size=BS, **kw)


def test_bnb4_rejects_mismatched_out():
    A = f16(M, K)
    with pytest.raises(nat.XrmmInvalid, match="out must be"):
        ops.matmul_bnb4(A, u8(N * K // 2), f16(N * K // 32), K=K, N=N, out=f32(M, N))


def test_int8a_rejects_mismatched_out():
    A = f16(1, 128)
    with pytest.raises(nat.XrmmInvalid, match="out must be"):
        ops.matmul_nbits_int8a(A, u8(N, 4, 16), f16(N, 4), K=128, N=N, out=f16(1, N - 1))


@pytest.mark.parametrize("status", [torch.zeros(1, dtype=torch.int8), torch.zeros(0, dtype=torch.int32),
                                    torch.zeros(1, dtype=torch.float32)])
def test_gather_rejects_bad_status_word(status):
    with pytest.raises(nat.XrmmInvalid, match="status"):
        ops.gather_block_quantized(u8(4, 16), torch.zeros(2, dtype=torch.int32), f32(4, 1), bits=4, block_size=32,
                                   status=status)
