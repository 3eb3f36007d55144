"""Materialise the golden fixture cases (tests/golden/fixtures.json) as NumPy arrays.

Generators follow the rules of the reference harness
(kernels/_shared/verify_upstream.py:90-122): ``values``, ``constant``,
``cycle`` (np.resize of the list) and ``linspace`` (float64 inclusive then one
cast). The upstream ``fillFloat32`` generator is not in the reference either
(tests/test_upstream_operator_fixtures.py:52-58 treats it as unsupported);
when ``substitute`` is set, such inputs get seeded ``offset + scale*U(-1,1)``
values (the generator's own offset and scale) so the case's shape, attributes
and other inputs are still exercised (those cases carry no explicit outputs,
so the oracle supplies the expectation).
"""
from __future__ import annotations

import json
import os
import zlib

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_CACHE = None


def load_cases():
    global _CACHE
    if _CACHE is None:
        with open(os.path.join(HERE, "golden", "fixtures.json")) as f:
            _CACHE = json.load(f)["cases"]
    return _CACHE


def find(operation: str, name: str):
    for c in load_cases():
        if c["operation"] == operation and c["name"] == name:
            return c
    raise KeyError(name)


def materialize(spec, seed_key: str = "", substitute: bool = False):
    dtype = np.dtype(spec["dtype"])
    shape = tuple(spec["shape"])
    count = int(np.prod(shape)) if shape else 1
    data = spec.get("data") or {}
    kind = data.get("kind")
    if kind == "values":
        arr = np.asarray(data["values"], dtype=dtype)
        assert arr.size == count
    elif kind == "constant":
        arr = np.full(count, data["value"], dtype=dtype)
    elif kind == "cycle":
        arr = np.resize(np.asarray(data["values"], dtype=dtype), count)
    elif kind == "linspace":
        arr = np.linspace(data["start"], data["end"], count, dtype=np.float64).astype(dtype)
    elif substitute:
        rng = np.random.default_rng(zlib.crc32(seed_key.encode()))
        if dtype == np.uint8:
            arr = rng.integers(0, 256, count, dtype=np.uint8)
        else:
            # bounded like the upstream sin/cos product it stands in for:
            # offset + scale * u with |u| <= 1
            u = rng.uniform(-1.0, 1.0, count)
            arr = (float(data.get("offset", 0.0)) + float(data.get("scale", 1.0)) * u).astype(dtype)
    else:
        raise ValueError("unsupported generator " + str(kind))
    return arr.reshape(shape)


MATERIALIZABLE = ("values", "constant", "cycle", "linspace")


def materializable(case) -> bool:
    """True when every input of ``case`` is given by data the fixture holds."""
    return all((s.get("data") or {}).get("kind") in MATERIALIZABLE for s in case["inputs"].values())


def case_inputs(case, substitute: bool = False):
    return {n: materialize(s, case["name"] + "/" + n, substitute) for n, s in case["inputs"].items()}


def case_tolerance(case, out_name):
    spec = case["outputs"][out_name]
    atol = spec.get("tolerance", case.get("tolerance") or 0)
    rtol = spec.get("relTolerance", case.get("relTolerance") or 0)
    return float(atol or 0), float(rtol or 0)


def reference_compare(actual, expected, atol, rtol) -> bool:
    """``compare`` of kernels/_shared/verify_upstream.py:137-151 (atol + rtol*|ref|)."""
    a = np.asarray(actual).astype(np.float64)
    e = np.asarray(expected).astype(np.float64)
    if a.shape != e.shape:
        return False
    fin = np.isfinite(a) & np.isfinite(e)
    special = (a == e) & ~fin
    if not np.all(fin | special):
        return False
    err = np.abs(a[fin] - e[fin])
    return bool(np.all(err <= atol + rtol * np.abs(e[fin])))
