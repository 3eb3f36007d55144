"""Request-level plan() through the C ABI, without a device: contract checks,
attribute defaults, args-over-attrs precedence, output shapes and requested
outputs (kernels/_shared/extended/planner.cpp:67-93, complex_plan.cpp:117-120,
contract_data.h:722-751)."""
import numpy as np
import pytest

from xrgpu_amd import operator as op

MNB, QKV, MLP = "com.microsoft.MatMulNBits", "com.microsoft.MatMulNBitsQkv", "com.microsoft.MatMulNBitsMlp"


def T(name, shape, dtype="float16"):
    return op.Tensor(name, np.zeros(shape, np.dtype(dtype)))


def mnb(K=64, N=8, bs=32, lead=(2, 3), dtype="float16", extra=()):
    kb = (K + bs - 1) // bs
    return [T("aT", lead + (K,), dtype), T("bT", (N, kb, bs // 2), "uint8"), T("scalesT", (N, kb), dtype), *extra]


def test_output_shape_folds_leading_axes():
    outs = op.plan(op.Request(MNB, mnb(), attrs={"N": 8, "block_size": 32}))
    assert [(t.name, t.shape, t.dtype, t.storage_dtype) for t in outs] == [("yT", (2, 3, 8), "float16", "float16")]


def test_K_defaults_to_last_dim_and_block_size_to_32():
    outs = op.plan(op.Request(MNB, mnb(K=64, bs=32), attrs={"N": 8}))
    assert outs[0].shape == (2, 3, 8)


def test_args_override_attrs():
    req = op.Request(MNB, mnb(N=8), attrs={"N": 5, "block_size": 32}, args={"N": 8})
    assert op.plan(req)[0].shape[-1] == 8
    with pytest.raises(op.XrmmInvalid, match="bT must have shape"):
        op.plan(op.Request(MNB, mnb(N=8), attrs={"N": 8, "block_size": 32}, args={"N": 5}))


def test_float_integer_attribute_accepted_and_fraction_rejected():
    assert op.plan(op.Request(MNB, mnb(), attrs={"N": 8.0}))[0].shape[-1] == 8
    with pytest.raises(op.XrmmInvalid, match="Integer attribute required: N"):
        op.plan(op.Request(MNB, mnb(), attrs={"N": 8.5}))


@pytest.mark.parametrize("mutate,msg", [
    (lambda ins: ins[:1], "Missing required frozen-contract input: bT"),
    (lambda ins: ins + [T("gammaT", (64,))], "Unknown input outside frozen contract: gammaT"),
    (lambda ins: [T("aT", (2, 3, 64), "int32")] + ins[1:], "Logical dtype outside frozen contract: aT"),
    (lambda ins: ins[:2] + [T("scalesT", (8, 2), "float32")], "Type variable differs between tensors: T1"),
    (lambda ins: ins[:1] + [T("bT", (8, 32), "uint8")] + ins[2:], "Rank outside frozen contract: bT"),
    (lambda ins: ins + [T("biasT", (7,))], "biasT must have shape"),
    (lambda ins: ins + [ins[0]], "Duplicate"),
])
def test_contract_violations_are_invalid(mutate, msg):
    with pytest.raises(op.XrmmInvalid, match=msg):
        op.plan(op.Request(MNB, mutate(mnb()), attrs={"N": 8}))


def test_geometry_errors():
    with pytest.raises(op.XrmmInvalid, match="Packed matmul N required"):
        op.plan(op.Request(MNB, mnb(), attrs={}))
    with pytest.raises(op.XrmmInvalid, match="Invalid packed matmul geometry"):
        op.plan(op.Request(MNB, mnb(), attrs={"N": 8, "block_size": 0}))
    with pytest.raises(op.XrmmInvalid, match="bits must be 2, 4 or 8"):
        op.plan(op.Request(MNB, mnb(), attrs={"N": 8, "bits": 3}))
    with pytest.raises(op.XrmmInvalid, match="Unsupported extended operator"):
        op.plan(op.Request("com.microsoft.MatMulBnb4", mnb(), attrs={"N": 8}))


def test_packed_and_float_zero_point_shapes():
    zp_packed = T("zeroPointsT", (8, 1), "uint8")  # kb = 2 blocks, 4-bit: 1 byte per row
    assert op.plan(op.Request(MNB, mnb(extra=(zp_packed,)), attrs={"N": 8}))[0].shape == (2, 3, 8)
    zp_float = T("zeroPointsT", (8, 2), "float32")  # T3 may differ from T1
    assert op.plan(op.Request(MNB, mnb(extra=(zp_float,)), attrs={"N": 8}))[0].shape == (2, 3, 8)
    with pytest.raises(op.XrmmInvalid, match="zeroPointsT must have shape"):
        op.plan(op.Request(MNB, mnb(extra=(T("zeroPointsT", (8, 2), "uint8"),)), attrs={"N": 8}))


def test_requested_outputs_select_storage_and_are_checked():
    want = [op.Tensor("yT", shape=(2, 3, 8), dtype="float16", storage_dtype="float32")]
    outs = op.plan(op.Request(MNB, mnb(), attrs={"N": 8}, requested_outputs=want))
    assert outs[0].storage_dtype == "float32"
    bad = [op.Tensor("yT", shape=(2, 3, 9), dtype="float16")]
    with pytest.raises(op.XrmmInvalid, match="Requested output shape differs from plan"):
        op.plan(op.Request(MNB, mnb(), attrs={"N": 8}, requested_outputs=bad))
    bad = [op.Tensor("yT", shape=(2, 3, 8), dtype="float32")]
    with pytest.raises(op.XrmmInvalid, match="name/type differs"):
        op.plan(op.Request(MNB, mnb(), attrs={"N": 8}, requested_outputs=bad))


def qkv_inputs(K=64, Nq=16, Nkv=8, bs=32):
    kb = K // bs
    ins = [T("aT", (4, K)), T("normScaleT", (K,))]
    for p, n in (("q", Nq), ("k", Nkv), ("v", Nkv)):
        ins += [T(p + "BT", (n, kb, bs // 2), "uint8"), T(p + "ScalesT", (n, kb))]
    return ins


def test_qkv_outputs_and_optional_residual():
    outs = op.plan(op.Request(QKV, qkv_inputs(), attrs={"Nq": 16, "Nkv": 8}))
    assert [(t.name, t.shape) for t in outs] == [("qT", (4, 16)), ("kT", (4, 8)), ("vT", (4, 8))]
    want = [op.Tensor(n, shape=s, dtype="float16") for n, s in
            (("qT", (4, 16)), ("kT", (4, 8)), ("vT", (4, 8)), ("residualT", (4, 64)))]
    outs = op.plan(op.Request(QKV, qkv_inputs(), attrs={"Nq": 16, "Nkv": 8}, requested_outputs=want))
    assert [t.name for t in outs] == ["qT", "kT", "vT", "residualT"]
    with pytest.raises(op.XrmmInvalid, match="Missing required frozen-contract input: normScaleT"):
        op.plan(op.Request(QKV, [t for t in qkv_inputs() if t.name != "normScaleT"], attrs={"Nq": 16, "Nkv": 8}))


def test_mlp_activation_names():
    K, N, bs = 64, 8, 32
    ins = [T("aT", (3, K))] + [T(p + s, sh, dt) for p in ("gate", "up") for s, sh, dt in
                                (("BT", (N, 2, 16), "uint8"), ("ScalesT", (N, 2), "float16"))]
    for act in ("silu", "swish", "gelu", "relu", "tanh", "sigmoid", "identity", "none", "swiglu"):
        assert op.plan(op.Request(MLP, ins, attrs={"N": N, "activation": act}))[0].shape == (3, N)
    with pytest.raises(op.XrmmInvalid, match="Unknown fused activation: mish"):
        op.plan(op.Request(MLP, ins, attrs={"N": N, "activation": "mish"}))


def test_prepare_rejects_byte_count_and_memory_limit_before_touching_a_device():
    req = op.Request(MNB, mnb(), attrs={"N": 8})
    req.inputs[0].data = req.inputs[0].data.reshape(-1)[:-1]  # one element short
    with pytest.raises(op.XrmmInvalid, match="byte count mismatch: aT"):
        op.Operator.prepare("", req)
    with pytest.raises(op.XrmmInvalid, match="memory limit exceeded"):
        op.Operator.prepare("", op.Request(MNB, mnb(), attrs={"N": 8}), op.Options(memory_limit_bytes=64))
    with pytest.raises(op.XrmmInvalid, match="Positive extended runtime limits"):
        op.Operator.prepare("", op.Request(MNB, mnb(), attrs={"N": 8}), op.Options(timeout_ns=0))
