"""The kernel-catalog entry of the MatMulNBits family (xrgpu_amd/catalog.py).

The reference's catalog entry (kernels/catalog.json:12080-12130 and
kernels/com.microsoft.MatMulNBits{,Qkv,Mlp}/contract.json, validated by
kernels/catalog.py:85-248) fixes each operator's attribute and IO contract.
The descriptors of this build must keep that portable contract unchanged
(compared with tests/golden/reference_contracts.json, extracted from those
JSON files by tests/golden/extract_contracts.py), declare everything they
accept beyond it under ``extensions``, and describe what the C planner
actually enforces (checked through xrmm_plan, no device needed)."""
import json
import os
import shutil

import numpy as np
import pytest

from xrgpu_amd import catalog
from xrgpu_amd import operator as op

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_contracts.json")
REF = json.load(open(GOLDEN))["operators"]
_NP = {"float16": np.float16, "float32": np.float32, "uint8": np.uint8}


def test_catalog_loads_and_lists_the_family():
    v = catalog.load()
    assert sorted(e["id"] for e in v["entries"]) == sorted(REF)
    assert v["backend"] == "hip" and v["operator_count"] == 3


@pytest.mark.parametrize("identity", list(REF))
def test_portable_contract_equals_the_reference(identity):
    ours, ref = catalog.contract(identity), REF[identity]["contract"]
    for key in catalog.PORTABLE + ("limits", "domain", "name", "since_version"):
        assert ours[key] == ref[key], key
    # the reference's catalog also rejects anything else (kernels/catalog.py:162-167)
    assert ref["capabilities"]["cpu_fallback"] is False and ours["capabilities"]["cpu_fallback"] is False
    assert ours["capabilities"]["silent_type_conversion"] is False
    assert ours["backend"] == "hip" and ref["backend"] == "vulkan"
    assert REF[identity]["catalog_entry"]["native"]["api"] == "extended"


@pytest.mark.parametrize("identity", list(REF))
def test_extensions_only_widen(identity):
    ours = catalog.contract(identity)
    merged = catalog.merged_contract(ours)
    ref = REF[identity]["contract"]
    for port, spec in ref["inputs"].items():
        assert merged["inputs"][port] == spec
    for port in set(merged["inputs"]) - set(ref["inputs"]):
        assert merged["inputs"][port].get("optional") is True, port
    for var, types in ref["type_constraints"].items():
        assert set(types) <= set(merged["type_constraints"][var])
    for name, rule in ref["attribute_constraints"].items():
        m = merged["attribute_constraints"][name]
        if isinstance(rule.get("values"), list) and isinstance(m.get("values"), list):
            assert set(rule["values"]) <= set(m["values"]), name
    assert merged["outputs"] == ref["outputs"]


def _tensor(name, shape, dtype):
    return op.Tensor(name, np.zeros(shape, _NP[dtype]))


def _request(identity, dtype="float16", drop=(), add=(), swap=None, K=64, N=8, bs=32):
    """A minimal valid request of the operator from its contract ports."""
    kb = K // bs
    shapes = {"aT": (2, K), "skipT": (2, K), "normScaleT": (K,)}
    ins = []
    c = catalog.contract(identity)
    for port, spec in c["inputs"].items():
        if (spec.get("optional") and port not in add) or port in drop:
            continue
        if port.endswith("BT") or port == "bT":
            t = _tensor(port, (N, kb, bs // 2), "uint8")
        elif port.endswith("ScalesT") or port == "scalesT":
            t = _tensor(port, (N, kb), dtype)
        elif port.endswith("BiasT") or port == "biasT":
            t = _tensor(port, (N,), dtype)
        elif "ZeroPoints" in port or port == "zeroPointsT":
            t = _tensor(port, (N, kb), dtype)
        else:
            t = _tensor(port, shapes[port], dtype)
        ins.append(swap(t) if swap else t)
    attrs = {"K": K, "block_size": bs}
    attrs.update({"Nq": N, "Nkv": N} if identity.endswith("Qkv") else {"N": N})
    return op.Request(identity, ins, attrs=attrs)


@pytest.mark.parametrize("dtype", ["float16", "float32"])
@pytest.mark.parametrize("identity", list(REF))
def test_planner_follows_the_contract(identity, dtype):
    c = catalog.contract(identity)
    outs = op.plan(_request(identity, dtype))
    required_outs = [n for n, s in c["outputs"].items() if not s.get("optional")]
    assert sorted(t.name for t in outs) == sorted(required_outs)
    assert all(t.dtype == dtype for t in outs)
    # every optional input of the merged contract is accepted
    merged = catalog.merged_contract(c)
    optional = [p for p, s in merged["inputs"].items() if s.get("optional")]
    op.plan(_request(identity, dtype, add=optional))
    # every required input is required, with the reference planner's message
    for port, spec in c["inputs"].items():
        if not spec.get("optional"):
            with pytest.raises(op.XrmmInvalid, match="Missing required frozen-contract input: " + port):
                op.plan(_request(identity, dtype, drop=(port,)))


@pytest.mark.parametrize("identity", list(REF))
def test_planner_rejects_types_outside_the_contract(identity):
    def to_int32(t):
        return _tensor(t.name, t.shape, "float16") if t.name != "aT" else op.Tensor("aT", np.zeros(t.shape, np.int32))
    with pytest.raises(op.XrmmInvalid, match="Logical dtype outside frozen contract: aT"):
        op.plan(_request(identity, swap=to_int32))
    req = _request(identity)
    req.inputs.append(_tensor("notAPortT", (4,), "float16"))
    with pytest.raises(op.XrmmInvalid, match="Unknown input outside frozen contract: notAPortT"):
        op.plan(req)


@pytest.mark.parametrize("identity", list(REF))
def test_bind_resolves_the_native_and_python_entry_points(identity):
    b = catalog.bind(identity)
    assert b.c_entry == catalog.contract(identity)["native"]["zero_copy"]
    assert callable(b.zero_copy) and b.plan is op.plan
    outs = b.plan(b.request(_request(identity).inputs, _request(identity).attrs))
    assert outs


def test_tampered_descriptor_is_rejected(tmp_path):
    root = tmp_path / "kernels"
    shutil.copytree(catalog.ROOT, root)
    catalog.load(str(root))
    p = root / "com.microsoft.MatMulNBits" / "contract.json"
    d = json.load(open(p))
    d["capabilities"]["cpu_fallback"] = True
    json.dump(d, open(p, "w"))
    with pytest.raises(ValueError, match="checksum"):
        catalog.load(str(root))
    idx = json.load(open(root / "catalog.json"))
    idx["backend"] = "vulkan"
    json.dump(idx, open(root / "catalog.json", "w"))
    with pytest.raises(ValueError, match="identity mismatch"):
        catalog.load(str(root))
