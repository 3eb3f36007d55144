"""Kernel-catalog entry of the MatMulNBits family on the HIP backend.

The reference registers each native operator in ``kernels/catalog.json``
(entries such as ``kernels/catalog.json:12080-12130``) next to a descriptor
``kernels/<id>/contract.json`` that fixes the operator's attribute and IO
contract, and ``kernels/catalog.py:85-248`` (``load``) validates the catalog
before anything binds to it. This module is the same entry for this
library: ``xrgpu_amd/kernels/catalog.json`` lists the three operators
(MatMulNBits, MatMulNBitsQkv, MatMulNBitsMlp) with ``"backend": "hip"``, each
descriptor keeps the reference's portable contract (attributes and defaults,
attribute constraints, type constraints, ports with their ONNX names,
limits) unchanged and declares what this build accepts beyond it under
``extensions``; ``load`` validates them the way the reference's loader
validates its own (identity, descriptor digests, no CPU fallback, no silent
type conversion), and :func:`bind` returns the callables the entry names:
the request lifecycle of :mod:`xrgpu_amd.operator` and the zero-copy torch
front end of :mod:`xrgpu_amd.ops`, both over libxrmm.so's C ABI.

``python -m xrgpu_amd.catalog --write`` refreshes the index after a
descriptor changes.
"""
from __future__ import annotations

import argparse
import hashlib
import importlib
import json
import os
from dataclasses import dataclass

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.join(HERE, "kernels")
INDEX = os.path.join(ROOT, "catalog.json")
OPERATORS = ("com.microsoft.MatMulNBits", "com.microsoft.MatMulNBitsQkv", "com.microsoft.MatMulNBitsMlp")
BACKEND, TARGET = "hip", "linux-x86_64-gfx950"
# the descriptor fields the reference's catalog loader compares with the
# upstream manifest (kernels/catalog.py:183-193): a drop-in keeps them
PORTABLE = ("inputs", "outputs", "type_constraints", "attributes", "attribute_constraints")


def _sha_file(path: str) -> str:
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def _digest(value) -> str:
    return hashlib.sha256(json.dumps(value, sort_keys=True, separators=(",", ":")).encode()).hexdigest()


def _contract_path(identity: str) -> str:
    return os.path.join(ROOT, identity, "contract.json")


def _entry(identity: str) -> dict:
    contract = json.load(open(_contract_path(identity)))
    return {"id": identity, "path": identity, "contract": identity + "/contract.json",
            "descriptor_digests": {"contract": _sha_file(_contract_path(identity))},
            "native": contract["native"], "status": contract["status"]}


def write_index() -> dict:
    """Rebuild catalog.json from the descriptors (maintainer step)."""
    value = {"schema_version": 1, "kind": "xrgpu.native-kernel-catalog", "backend": BACKEND, "target": TARGET,
             "operator_count": len(OPERATORS), "entries": [_entry(i) for i in OPERATORS]}
    value["catalog_sha256"] = _digest(value)
    with open(INDEX, "w") as f:
        json.dump(value, f, indent=1, sort_keys=True)
        f.write("\n")
    return value


def merged_contract(contract: dict) -> dict:
    """The contract with its declared extensions applied: extra optional
    input ports, widened type variables and attribute value sets."""
    out = {k: json.loads(json.dumps(contract[k])) for k in PORTABLE}
    ext = contract.get("extensions", {})
    out["inputs"].update(ext.get("inputs", {}))
    for var, types in ext.get("type_constraints", {}).items():
        have = out["type_constraints"].setdefault(var, [])
        have.extend(t for t in types if t not in have)
    for name, rule in ext.get("attribute_constraints", {}).items():
        out["attribute_constraints"].setdefault(name, {}).update(rule)
    return out


def load(root: str = ROOT) -> dict:
    """Validate the catalog and its descriptors; returns the index.

    Raises ValueError on any mismatch, as the reference's loader does."""
    index = os.path.join(root, "catalog.json")
    value = json.load(open(index))
    if value.get("schema_version") != 1 or value.get("kind") != "xrgpu.native-kernel-catalog":
        raise ValueError("Unsupported native catalog")
    if _digest({k: v for k, v in value.items() if k != "catalog_sha256"}) != value.get("catalog_sha256"):
        raise ValueError("Native catalog identity mismatch")
    if (value.get("backend"), value.get("target")) != (BACKEND, TARGET):
        raise ValueError("Unsupported native catalog target")
    entries = value.get("entries", [])
    ids = [e["id"] for e in entries]
    if tuple(ids) != OPERATORS or value.get("operator_count") != len(OPERATORS):
        raise ValueError("Native catalog requires exactly the MatMulNBits family")
    for e in entries:
        identity = e["id"]
        if e["path"] != identity or e["contract"] != identity + "/contract.json":
            raise ValueError("Native operator descriptor path mismatch")
        path = os.path.join(root, e["contract"])
        if _sha_file(path) != e["descriptor_digests"]["contract"]:
            raise ValueError("Native descriptor checksum mismatch: " + e["contract"])
        contract = json.load(open(path))
        if (contract.get("kind") != "xrgpu.native-operator" or contract.get("id") != identity
                or contract.get("backend") != BACKEND):
            raise ValueError("Native descriptor target/identity mismatch")
        for key in ("native", "status"):
            if contract[key] != e[key]:
                raise ValueError("Native catalog and contract differ: " + identity + " " + key)
        caps = contract.get("capabilities", {})
        if caps.get("cpu_fallback") is not False or caps.get("silent_type_conversion") is not False:
            raise ValueError("Native contract must reject unsupported execution")
        ext = contract.get("extensions", {})
        for port, spec in ext.get("inputs", {}).items():
            if port in contract["inputs"] or not spec.get("optional"):
                raise ValueError("Extension ports must be new and optional: " + port)
    return value


def contract(identity: str) -> dict:
    """The validated descriptor of one operator."""
    load()
    if identity not in OPERATORS:
        raise KeyError(identity)
    return json.load(open(_contract_path(identity)))


@dataclass
class Binding:
    """What a catalog entry binds to: the request lifecycle (plan, Operator)
    and the zero-copy device call, both over libxrmm.so."""
    identity: str
    contract: dict
    plan: object
    Operator: object
    Request: object
    zero_copy: object
    c_entry: str

    def request(self, inputs, attrs=None, args=None, requested_outputs=()):
        return self.Request(self.identity, list(inputs), attrs=dict(attrs or {}), args=dict(args or {}),
                            requested_outputs=list(requested_outputs))


def bind(identity: str) -> Binding:
    """Resolve an entry's native and Python bindings (loads libxrmm.so; the
    zero-copy front end also imports torch)."""
    c = contract(identity)
    from . import _native, operator
    lib = _native.lib()
    names = [c["native"]["zero_copy"], c["native"]["select_kernel"], *c["native"]["lifecycle"]]
    missing = [n for n in names if not hasattr(lib, n)]
    if missing:
        raise RuntimeError("libxrmm.so lacks " + ", ".join(missing))
    mod, fn = c["python"]["zero_copy"].split(":")
    zero_copy = getattr(importlib.import_module(mod), fn)
    return Binding(identity, c, operator.plan, operator.Operator, operator.Request, zero_copy, c["native"]["zero_copy"])


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--write", action="store_true", help="rebuild kernels/catalog.json from the descriptors")
    a = ap.parse_args()
    if a.write:
        write_index()
    v = load()
    print(f"catalog ok: {v['operator_count']} operators, backend {v['backend']}, target {v['target']}")


if __name__ == "__main__":
    main()
