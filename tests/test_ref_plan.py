"""xrmm_plan against the reference's own planner (CPU, no device).

oracle/_ref/libref_plan.so is the reference planner (kernels/_shared/extended/
planner.cpp:67, complex_plan.cpp:117-129, contracts.cpp with contract_data.h)
compiled from its sources by ``make -C oracle ref``, behind a C binding that
takes xrmm_plan's own request structure (oracle/ref_plan_shim.cpp). Every
request below goes to both planners: accepted requests must plan the same
outputs (names, dtypes, storage dtypes, shapes), rejected ones must be
rejected with the reference's message. The deviations are listed and
checked to stay what they are: stricter host checks (tensor shapes the
reference leaves to the device, bits in {2, 4, 8}, positive Nq / Nkv, the
MatMulBnb4 quant_type and absmax count), the packed uint8 zero points this
build adds, and the message for an operation neither build knows.
"""
import ctypes
import os

import pytest

from tests.test_operator_plan import BNB, GBQ, MLP, MNB, QKV, QMOE, SW, T, bnb, gbq_ins, mnb, qkv_inputs, qmoe_ins
from xrgpu_amd import _native as nat
from xrgpu_amd import operator as op

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libref_plan.so")


@pytest.fixture(scope="module")
def ref():
    if not os.path.exists(REF_LIB):
        pytest.skip("oracle/_ref/libref_plan.so is built from the reference checkout (make -C oracle ref)")
    lib = ctypes.CDLL(REF_LIB)
    lib.ref_plan.restype = ctypes.c_int
    lib.ref_plan.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.POINTER(ctypes.c_int32),
                             ctypes.c_char_p, ctypes.c_uint64]
    return lib


def ref_plan(lib, req):
    m = op._Marshal(req)
    descs = (op._CDesc * 8)()
    n = ctypes.c_int32(0)
    msg = ctypes.create_string_buffer(512)
    rc = lib.ref_plan(ctypes.byref(m.req), descs, 8, ctypes.byref(n), msg, 512)
    if rc != 0:
        return None, msg.value.decode()
    return [op._desc_to_tensor(descs[i]) for i in range(n.value)], None


def our_plan(req):
    try:
        return op.plan(req), None
    except nat.XrmmInvalid as e:
        return None, str(e)


def key(outs):
    return [(t.name, t.dtype, t.storage_dtype, tuple(t.shape)) for t in outs]


def mlp_ins(M=3, K=64, N=8, bs=32, extra=()):
    kb = (K + bs - 1) // bs
    return ([T("aT", (M, K))] + [T(p + s, sh, dt) for p in ("gate", "up") for s, sh, dt in
                                 (("BT", (N, kb, bs // 2), "uint8"), ("ScalesT", (N, kb), "float16"))] + list(extra))


def yT(shape, dtype="float16", storage=None, name="yT"):
    return op.Tensor(name, shape=shape, dtype=dtype, storage_dtype=storage)


# (id, request): both planners must agree
AGREE = [
    ("mnb_fp16_rank3", op.Request(MNB, mnb(), attrs={"N": 8, "block_size": 32})),
    ("mnb_K_default", op.Request(MNB, mnb(K=64), attrs={"N": 8})),
    ("mnb_fp32", op.Request(MNB, mnb(dtype="float32"), attrs={"N": 8})),
    ("mnb_K_tail_bs16", op.Request(MNB, mnb(K=20, N=5, bs=16, lead=(3,)), attrs={"N": 5, "block_size": 16, "K": 20})),
    ("mnb_bits8", op.Request(MNB, [T("aT", (2, 64)), T("bT", (8, 2, 32), "uint8"), T("scalesT", (8, 2))],
                             attrs={"N": 8, "bits": 8})),
    ("mnb_bits2", op.Request(MNB, [T("aT", (2, 64)), T("bT", (8, 2, 8), "uint8"), T("scalesT", (8, 2))],
                             attrs={"N": 8, "bits": 2})),
    ("mnb_float_zp_bias", op.Request(MNB, mnb(extra=(T("zeroPointsT", (8, 2), "float32"), T("biasT", (8,)))),
                                     attrs={"N": 8})),
    ("mnb_args_over_attrs", op.Request(MNB, mnb(), attrs={"N": 5}, args={"N": 8})),
    ("mnb_float_integer_N", op.Request(MNB, mnb(), attrs={"N": 8.0})),
    ("mnb_storage_request", op.Request(MNB, mnb(), attrs={"N": 8}, requested_outputs=[yT((2, 3, 8), storage="float32")])),
    ("mnb_missing_bT", op.Request(MNB, mnb()[:1], attrs={"N": 8})),
    ("mnb_unknown_input", op.Request(MNB, mnb() + [T("gammaT", (64,))], attrs={"N": 8})),
    ("mnb_bad_dtype", op.Request(MNB, [T("aT", (2, 3, 64), "int32")] + mnb()[1:], attrs={"N": 8})),
    ("mnb_T1_differs", op.Request(MNB, mnb()[:2] + [T("scalesT", (8, 2), "float32")], attrs={"N": 8})),
    ("mnb_rank", op.Request(MNB, mnb()[:1] + [T("bT", (8, 32), "uint8")] + mnb()[2:], attrs={"N": 8})),
    ("mnb_duplicate", op.Request(MNB, mnb() + [mnb()[0]], attrs={"N": 8})),
    ("mnb_no_N", op.Request(MNB, mnb(), attrs={})),
    ("mnb_bs0", op.Request(MNB, mnb(), attrs={"N": 8, "block_size": 0})),
    ("mnb_fraction_N", op.Request(MNB, mnb(), attrs={"N": 8.5})),
    ("mnb_requested_shape", op.Request(MNB, mnb(), attrs={"N": 8}, requested_outputs=[yT((2, 3, 9))])),
    ("mnb_requested_dtype", op.Request(MNB, mnb(), attrs={"N": 8}, requested_outputs=[yT((2, 3, 8), "float32")])),
    ("qkv", op.Request(QKV, qkv_inputs(), attrs={"Nq": 16, "Nkv": 8})),
    ("qkv_skip", op.Request(QKV, qkv_inputs() + [T("skipT", (4, 64))], attrs={"Nq": 16, "Nkv": 8, "epsilon": 1e-5})),
    ("qkv_residual", op.Request(QKV, qkv_inputs(), attrs={"Nq": 16, "Nkv": 8}, requested_outputs=[
        op.Tensor(n, shape=s, dtype="float16") for n, s in
        (("qT", (4, 16)), ("kT", (4, 8)), ("vT", (4, 8)), ("residualT", (4, 64)))])),
    ("qkv_no_norm", op.Request(QKV, [t for t in qkv_inputs() if t.name != "normScaleT"], attrs={"Nq": 16, "Nkv": 8})),
    ("mlp", op.Request(MLP, mlp_ins(), attrs={"N": 8})),
    ("mlp_all_optional", op.Request(MLP, mlp_ins(extra=(T("skipT", (3, 64)), T("normScaleT", (64,)), T("gateBiasT", (8,)),
                                                        T("upBiasT", (8,)))), attrs={"N": 8, "activation": "gelu"})),
    ("mlp_residual", op.Request(MLP, mlp_ins(extra=(T("skipT", (3, 64)),)), attrs={"N": 8}, requested_outputs=[
        yT((3, 8)), op.Tensor("residualT", shape=(3, 64), dtype="float16")])),
    ("mlp_bad_activation", op.Request(MLP, mlp_ins(), attrs={"N": 8, "activation": "mish"})),
    *[(f"mlp_act_{a}", op.Request(MLP, mlp_ins(), attrs={"N": 8, "activation": a}))
      for a in ("silu", "swish", "relu", "tanh", "sigmoid", "identity", "none", "swiglu", "")],
    ("bnb4", op.Request(BNB, bnb(), attrs={"K": 64, "N": 8, "block_size": 32})),
    ("bnb4_fp32", op.Request(BNB, bnb(dtype="float32"), attrs={"K": 64, "N": 8, "block_size": 32})),
    ("bnb4_no_N", op.Request(BNB, bnb(), attrs={"K": 64})),
    ("bnb4_T1", op.Request(BNB, bnb()[:2] + [T("absmaxT", (16,), "float32")], attrs={"N": 8})),
    ("bnb4_rank", op.Request(BNB, [T("aT", (1, 3, 64))] + bnb()[1:], attrs={"N": 8})),
    ("qmoe_swiglu", op.Request(QMOE, qmoe_ins(), attrs=SW)),
    ("qmoe_blocks", op.Request(QMOE, qmoe_ins(bs=16), attrs=dict(SW, block_size=16))),
    ("qmoe_relu", op.Request(QMOE, qmoe_ins(swiglu=False), attrs={"k": 1, "activation_type": "relu"})),
    ("qmoe_k5", op.Request(QMOE, qmoe_ins(), attrs=dict(SW, k=5))),
    ("qmoe_sparse_mixer", op.Request(QMOE, qmoe_ins(), attrs=dict(SW, use_sparse_mixer=1))),
    ("qmoe_no_fusion", op.Request(QMOE, qmoe_ins(), attrs={"k": 2, "activation_type": "swiglu"})),
    ("qmoe_fusion_relu", op.Request(QMOE, qmoe_ins(swiglu=False), attrs={"k": 1, "swiglu_fusion": 1})),
    ("qmoe_bits8", op.Request(QMOE, qmoe_ins(), attrs=dict(SW, expert_weight_bits=8))),
    ("qmoe_bits2", op.Request(QMOE, qmoe_ins(), attrs=dict(SW, expert_weight_bits=2))),
    ("qmoe_prepacked", op.Request(QMOE, qmoe_ins(), attrs=dict(SW, weights_prepacked=1))),
    ("qmoe_bs24", op.Request(QMOE, qmoe_ins(bs=16), attrs=dict(SW, block_size=24))),
    ("qmoe_scales", op.Request(QMOE, qmoe_ins(bs=16), attrs=SW)),
    ("gbq", op.Request(GBQ, gbq_ins(), attrs={"block_size": 16})),
    ("gbq_zp", op.Request(GBQ, gbq_ins(zp=True), attrs={"block_size": 16})),
    ("gbq_int32", op.Request(GBQ, gbq_ins(idx="int32"), attrs={"block_size": 16})),
    ("gbq_bits8", op.Request(GBQ, gbq_ins(bits=8, pcols=32), attrs={"block_size": 16, "bits": 8})),
]


@pytest.mark.parametrize("name,req", AGREE, ids=[a[0] for a in AGREE])
def test_plan_matches_reference_planner(ref, name, req):
    r_out, r_err = ref_plan(ref, req)
    o_out, o_err = our_plan(req)
    if r_err is None:
        assert o_err is None, f"reference plans {key(r_out)}, xrmm_plan rejects: {o_err}"
        assert key(o_out) == key(r_out)
    else:
        assert o_err is not None, f"reference rejects ({r_err}), xrmm_plan plans {key(o_out)}"
        assert o_err == r_err


# Deliberate deviations: the reference plans these and leaves the malformed
# tensor to the device (a GPU failure code at run time); xrmm_plan rejects
# them on the host with a message naming the tensor.
STRICTER = [
    ("mnb_bT_shape", op.Request(MNB, mnb()[:1] + [T("bT", (8, 2, 15), "uint8")] + mnb()[2:], attrs={"N": 8}),
     "bT must have shape"),
    ("mnb_bias_shape", op.Request(MNB, mnb() + [T("biasT", (7,))], attrs={"N": 8}), "biasT must have shape"),
    ("mnb_args_N", op.Request(MNB, mnb(N=8), attrs={"N": 8}, args={"N": 5}), "bT must have shape"),
    ("mnb_bits3", op.Request(MNB, mnb(), attrs={"N": 8, "bits": 3}), "bits must be 2, 4 or 8"),
    ("qkv_no_Nkv", op.Request(QKV, qkv_inputs(), attrs={"Nq": 16}), "Nq and Nkv must be positive"),
    ("bnb4_quant_type", op.Request(BNB, bnb(), attrs={"N": 8, "quant_type": 2}), "quant_type must be 0"),
    ("bnb4_absmax_short", op.Request(BNB, bnb(bs=32), attrs={"N": 8, "block_size": 16}), "absmaxT holds fewer"),
]


@pytest.mark.parametrize("name,req,msg", STRICTER, ids=[s[0] for s in STRICTER])
def test_documented_stricter_checks(ref, name, req, msg):
    r_out, r_err = ref_plan(ref, req)
    o_out, o_err = our_plan(req)
    assert r_err is None, f"the reference now rejects this request too: {r_err}"
    assert o_err is not None and msg in o_err


def test_unknown_operation_is_rejected_by_both(ref):
    """An operation neither build knows: the reference's contract lookup
    rejects its first input ("Unknown input outside frozen contract: aT"),
    xrmm_plan names the operation ("Unsupported extended operator: ...")."""
    req = op.Request("com.microsoft.MatMulNBitsFp8", mnb(), attrs={"N": 8})
    r_out, r_err = ref_plan(ref, req)
    o_out, o_err = our_plan(req)
    assert r_err == "Unknown input outside frozen contract: aT"
    assert o_err == "Unsupported extended operator: com.microsoft.MatMulNBitsFp8"


def test_packed_zero_points_are_an_extension(ref):
    """uint8 zero points are outside the reference contract (T3 is float); this
    build takes them packed (the ONNX Runtime layout) and plans the same output
    as with float zero points."""
    packed = op.Request(MNB, mnb(extra=(T("zeroPointsT", (8, 1), "uint8"),)), attrs={"N": 8})
    r_out, r_err = ref_plan(ref, packed)
    assert r_err == "Logical dtype outside frozen contract: zeroPointsT"
    floatzp = op.Request(MNB, mnb(extra=(T("zeroPointsT", (8, 2), "float16"),)), attrs={"N": 8})
    r_out, r_err = ref_plan(ref, floatzp)
    assert r_err is None and key(our_plan(packed)[0]) == key(r_out)
    bad = op.Request(MNB, mnb(extra=(T("zeroPointsT", (8, 2), "uint8"),)), attrs={"N": 8})
    assert "zeroPointsT must have shape" in our_plan(bad)[1]
