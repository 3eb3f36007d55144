"""GPU sweep over every MatMulNBitsQkv and MatMulNBitsMlp fixture case of the
reference (kernels/_provenance/upstream/com.microsoft.MatMulNBits{Qkv,Mlp}/
build/webgpu/test.json, extracted into tests/golden/fixtures.json), each with
its own attributes: bits 2/4/8, block sizes 8/16/32, K = 20/21/160/300/301/
2080, epsilon, rank-3 activations, float32 and float16, with and without
skip, normScale, biases and the residual output.

Inputs the fixture holds as data are used as they are; the upstream-only
``fillFloat32`` generator gets seeded stand-ins of the same shape (see
tests/fixture_util.py). Expectations come from the oracle, checked at both
bars: the fixture's own atol + rtol*|ref| (verify_upstream.py:125-151) and
max|d| <= 1e-2*max|Y| (fp16) / 1e-5*max|Y| (fp32). Cases with explicit
outputs (the three pinned Mlp cases) are also compared with those outputs.
float32 cases run a second time converted to float16, which routes the
geometries that allow it through the fast fp16 kernels. The residual output
(A + skip rounded once) must be bit-exact.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests import fixture_util as F

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

QKV = "com.microsoft.MatMulNBitsQkv"
MLP = "com.microsoft.MatMulNBitsMlp"


def dev(x):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).cuda()


def host(t):
    return None if t is None else t.detach().cpu().numpy()


def ops():
    from xrgpu_amd import ops as _ops
    return _ops


def _names(op):
    return [c["name"] for c in F.load_cases() if c["operation"] == op]


def _convert(ins, dtype):
    if dtype is None:
        return ins
    return {k: (v if v.dtype == np.uint8 else v.astype(dtype)) for k, v in ins.items()}


def _check(case, out_name, got, ref, dtype):
    ok, err, lim = O.tolerance_ok(got, ref, dtype)
    assert ok, f"{case['name']}/{out_name}: max|d|={err} > {lim}"
    if np.dtype(dtype) == np.dtype(case["outputs"][out_name]["dtype"]):
        atol, rtol = F.case_tolerance(case, out_name)
        if atol or rtol:
            assert F.reference_compare(got, ref, atol, rtol), f"{case['name']}/{out_name}: fixture tolerance"


def _dtypes(case):
    """The case's own dtype, plus float16 for float32 cases."""
    own = np.dtype(case["inputs"]["aT"]["dtype"])
    return [None] if own == np.float16 else [None, np.float16]


def _qkv_params():
    out = []
    for n in _names(QKV):
        for dt in _dtypes(F.find(QKV, n)):
            out.append(pytest.param(n, dt, id=f"{n}-{'own' if dt is None else 'f16'}"))
    return out


def _mlp_params():
    out = []
    for n in _names(MLP):
        for dt in _dtypes(F.find(MLP, n)):
            out.append(pytest.param(n, dt, id=f"{n}-{'own' if dt is None else 'f16'}"))
    return out


def test_fixture_case_counts():
    # 15 upstream Qkv cases plus the harness KAT; 44 upstream Mlp cases
    assert len(_names(QKV)) == 16 and len(_names(MLP)) == 44


@pytest.mark.parametrize("name,dtype", _qkv_params())
def test_qkv_fixture_case(gpu, name, dtype):
    case = F.find(QKV, name)
    at = case["attrs"]
    ins = _convert(F.case_inputs(case, substitute=True), dtype)
    dt = ins["aT"].dtype
    K, Nq, Nkv = at["K"], at["Nq"], at["Nkv"]
    bits, bs = at.get("bits", 4), at.get("block_size", 32)
    eps = at.get("epsilon", 1e-6)
    want_res = "residualT" in case["outputs"]
    Q, Kk, V, R = ops().matmul_nbits_qkv(
        dev(ins["aT"]), dev(ins["qBT"]), dev(ins["qScalesT"]), dev(ins["kBT"]), dev(ins["kScalesT"]),
        dev(ins["vBT"]), dev(ins["vScalesT"]), norm_scale=dev(ins["normScaleT"]), skip=dev(ins.get("skipT")),
        K=K, Nq=Nq, Nkv=Nkv, bits=bits, block_size=bs, epsilon=eps, want_residual=want_res)
    ref = O.matmul_nbits_qkv(ins["aT"], ins["qBT"], ins["qScalesT"], ins["kBT"], ins["kScalesT"], ins["vBT"],
                             ins["vScalesT"], K=K, Nq=Nq, Nkv=Nkv, norm_scale=ins["normScaleT"],
                             skip=ins.get("skipT"), bits=bits, block_size=bs, epsilon=eps)
    for got, exp, nm in zip((Q, Kk, V), ref[:3], ("qT", "kT", "vT")):
        g = host(got)
        assert g.shape == tuple(case["outputs"][nm]["shape"]) and g.dtype == dt
        _check(case, nm, g, exp, dt)
    if want_res:
        assert np.array_equal(host(R), ref[3])


@pytest.mark.parametrize("name,dtype", _mlp_params())
def test_mlp_fixture_case(gpu, name, dtype):
    case = F.find(MLP, name)
    at = case["attrs"]
    ins = _convert(F.case_inputs(case, substitute=True), dtype)
    dt = ins["aT"].dtype
    K, N = at["K"], at["N"]
    bits, bs = at.get("bits", 4), at.get("block_size", 32)
    eps, act = at.get("epsilon", 1e-5), at.get("activation", "silu")
    want_res = "residualT" in case["outputs"]
    Y, R = ops().matmul_nbits_mlp(
        dev(ins["aT"]), dev(ins["gateBT"]), dev(ins["gateScalesT"]), dev(ins["upBT"]), dev(ins["upScalesT"]),
        skip=dev(ins.get("skipT")), norm_scale=dev(ins.get("normScaleT")), gate_bias=dev(ins.get("gateBiasT")),
        up_bias=dev(ins.get("upBiasT")), K=K, N=N, bits=bits, block_size=bs, epsilon=eps, activation=act,
        want_residual=want_res)
    ref, r = O.matmul_nbits_mlp(ins["aT"], ins["gateBT"], ins["gateScalesT"], ins["upBT"], ins["upScalesT"], K=K, N=N,
                                skip=ins.get("skipT"), norm_scale=ins.get("normScaleT"),
                                gate_bias=ins.get("gateBiasT"), up_bias=ins.get("upBiasT"), bits=bits,
                                block_size=bs, epsilon=eps, activation=act)
    y = host(Y)
    assert y.shape == tuple(case["outputs"]["yT"]["shape"]) and y.dtype == dt
    _check(case, "yT", y, ref, dt)
    if dtype is None and "yT" in case["explicit"]:
        exp = F.materialize(case["outputs"]["yT"])
        assert F.reference_compare(y, exp, *F.case_tolerance(case, "yT"))
    if want_res:
        assert np.array_equal(host(R), r)
        if dtype is None and "residualT" in case["explicit"]:
            assert F.reference_compare(host(R), F.materialize(case["outputs"]["residualT"]),
                                       *F.case_tolerance(case, "residualT"))


@pytest.mark.parametrize("act", ["silu", "gelu", "relu", "tanh", "sigmoid", "identity"])
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_mlp_fixture_geometry_every_activation(gpu, act, dtype):
    """The activation table (complex_plan.cpp:55) on a fixture geometry with
    a K tail (K = 301, block 16), float32 and float16."""
    case = F.find(MLP, "fused_skipsum_multi_trip_odd_k")
    at = case["attrs"]
    ins = _convert(F.case_inputs(case, substitute=True), dtype)
    K, N, bs = at["K"], at["N"], at["block_size"]
    Y, _ = ops().matmul_nbits_mlp(dev(ins["aT"]), dev(ins["gateBT"]), dev(ins["gateScalesT"]), dev(ins["upBT"]),
                                  dev(ins["upScalesT"]), skip=dev(ins["skipT"]), norm_scale=dev(ins["normScaleT"]),
                                  K=K, N=N, block_size=bs, epsilon=at["epsilon"], activation=act)
    ref, _ = O.matmul_nbits_mlp(ins["aT"], ins["gateBT"], ins["gateScalesT"], ins["upBT"], ins["upScalesT"], K=K, N=N,
                                skip=ins["skipT"], norm_scale=ins["normScaleT"], block_size=bs,
                                epsilon=at["epsilon"], activation=act)
    ok, err, lim = O.tolerance_ok(host(Y), ref, dtype)
    assert ok, (act, err, lim)
