"""Extract the portable operator contract of the MatMulNBits family from the
reference's kernel descriptors, as data.

Run in a container that has the reference checkout:

    python tests/golden/extract_contracts.py /root/reference

It reads only the JSON descriptors
``kernels/com.microsoft.MatMulNBits{,Qkv,Mlp}/contract.json`` and the
matching ``kernels/catalog.json`` entries, and writes
``tests/golden/reference_contracts.json``: per operator the fields a catalog
entry must keep for a drop-in (attributes and defaults, attribute
constraints, type constraints, input and output ports with their ONNX names,
capabilities, limits), plus the catalog entry's id, path and status. The
catalog test compares this build's descriptors with them.
"""
from __future__ import annotations

import json
import os
import sys

OPS = ("com.microsoft.MatMulNBits", "com.microsoft.MatMulNBitsQkv", "com.microsoft.MatMulNBitsMlp")
KEEP = ("id", "domain", "name", "since_version", "kind", "schema_version", "attributes", "attribute_constraints",
        "type_constraints", "inputs", "outputs", "capabilities", "limits", "backend", "status")


def main(ref: str) -> None:
    kernels = os.path.join(ref, "kernels")
    catalog = json.load(open(os.path.join(kernels, "catalog.json")))
    entries = {e["id"]: e for e in catalog["entries"]}
    out = {"source": "kernels/<id>/contract.json and kernels/catalog.json of the reference checkout", "operators": {}}
    for op in OPS:
        contract = json.load(open(os.path.join(kernels, op, "contract.json")))
        e = entries[op]
        out["operators"][op] = {
            "contract": {k: contract[k] for k in KEEP if k in contract},
            "catalog_entry": {"id": e["id"], "path": e["path"], "contract": e["contract"], "status": e["status"],
                              "native": e["native"]},
        }
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_contracts.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")
    print("wrote", path)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
