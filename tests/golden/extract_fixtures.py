"""Extract golden vectors from the reference's fixture JSON: the MatMulNBits
family and the next operators built on the same dequantisation (QMoE,
GatherBlockQuantized, MatMulBnb4).

Run in a container that has the reference checkout:

    python tests/golden/extract_fixtures.py /root/reference

It reads only data files (the frozen upstream ``test.json`` of those operators) and writes ``tests/golden/fixtures.json``: every case whose inputs
use the generators the reference's own harness can materialise
(``values``/``constant``/``cycle``/``linspace``, kernels/_shared/verify_upstream.py:90-122)
with their explicit expected outputs and tolerances, plus the structural
metadata (name, attrs, input specs) of every other case so parity tests can
reuse their shapes with seeded inputs. ``fixtureArrays`` references are
resolved inline. It also records the Qkv known-answer case that
kernels/_shared/extended/complex_reference.py:251-272 builds, as data.
"""
from __future__ import annotations

import json
import os
import sys

OPS = ("com.microsoft.MatMulNBits", "com.microsoft.MatMulNBitsQkv", "com.microsoft.MatMulNBitsMlp",
       "com.microsoft.QMoE", "com.microsoft.GatherBlockQuantized", "com.microsoft.MatMulBnb4")
MATERIALIZABLE = {"values", "constant", "cycle", "linspace"}


def _resolve(value, doc):
    if isinstance(value, dict) and "$ref" in value:
        ref = value["$ref"]
        assert ref.startswith("#/fixtureArrays/")
        return doc["fixtureArrays"][ref.split("/")[-1]]
    return value


def _spec(spec, doc):
    out = {k: v for k, v in spec.items() if k != "data"}
    data = spec.get("data")
    if isinstance(data, dict):
        d = dict(data)
        if "values" in d:
            d["values"] = _resolve(d["values"], doc)
        out["data"] = d
    return out


def main(reference: str) -> None:
    cases = []
    for op in OPS:
        path = os.path.join(reference, "kernels/_provenance/upstream", op, "build/webgpu/test.json")
        doc = json.load(open(path))
        for case in doc["cases"]:
            inputs = {n: _spec(s, doc) for n, s in case["inputs"].items()}
            outputs = {n: _spec(s, doc) for n, s in case["outputs"].items()}
            kinds = {n: (s.get("data") or {}).get("kind") for n, s in inputs.items()}
            cases.append(dict(
                operation=op,
                name=case["name"],
                source=os.path.relpath(path, reference),
                attrs=case.get("attrs", {}),
                inputs=inputs,
                outputs=outputs,
                materializable=all(k in MATERIALIZABLE for k in kinds.values()),
                explicit=[n for n, s in outputs.items() if "data" in s],
                tolerance=case.get("tolerance"),
                relTolerance=case.get("relTolerance"),
            ))
    # kernels/_shared/extended/complex_reference.py:251-272, restated as data:
    # bytes 152/168/184 = codes (8, 9)/(8, 10)/(8, 11) -> weights [0, 1|2|3, 0, 1|2|3] * 0.5
    cases.append(dict(
        operation="com.microsoft.MatMulNBitsQkv",
        name="independent_nonzero_reference_qkv_kat",
        source="kernels/_shared/extended/complex_reference.py:251-272",
        attrs={"K": 4, "Nq": 2, "Nkv": 2, "block_size": 16},
        inputs={
            "aT": {"dtype": "float32", "shape": [1, 4], "data": {"kind": "values", "values": [1, 2, -1, 0.5]}},
            "skipT": {"dtype": "float32", "shape": [1, 4], "data": {"kind": "values", "values": [0.5, -0.5, 0.25, 1]}},
            "normScaleT": {"dtype": "float32", "shape": [4], "data": {"kind": "values", "values": [1, 0.5, 2, 1]}},
            **{f"{p}BT": {"dtype": "uint8", "shape": [2, 1, 8], "data": {"kind": "constant", "value": byte}}
               for p, byte in (("q", 152), ("k", 168), ("v", 184))},
            **{f"{p}ScalesT": {"dtype": "float32", "shape": [2, 1], "data": {"kind": "constant", "value": 0.5}}
               for p in "qkv"},
        },
        outputs={"qT": {"dtype": "float32", "shape": [1, 2]}, "kT": {"dtype": "float32", "shape": [1, 2]},
                 "vT": {"dtype": "float32", "shape": [1, 2]}, "residualT": {"dtype": "float32", "shape": [1, 4]}},
        materializable=True, explicit=[], tolerance=0.0002, relTolerance=0.0002,
        kat={"weights_code_high_nibble": {"q": 9, "k": 10, "v": 11}, "scale": 0.5, "epsilon": 1e-6},
    ))
    here = os.path.dirname(os.path.abspath(__file__))
    with open(os.path.join(here, "fixtures.json"), "w") as f:
        json.dump({"generated_by": "tests/golden/extract_fixtures.py", "cases": cases}, f, indent=0)
    print(len(cases), "cases;", sum(c["materializable"] for c in cases), "materializable;",
          sum(bool(c["explicit"]) for c in cases), "with explicit outputs")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
