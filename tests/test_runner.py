"""The job-JSON runner (xrgpu_amd/lib/xrmm_execute) on the CPU: the wire format
of kernels/_shared/extended/tests/execute.cpp:14-35 in plan-only mode (no
device), literal and file tensors, and its error reporting (a JSON object on
stderr, exit status 1)."""
import json
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# XRMM_EXECUTE selects another build of the runner (the host-sanitizer build)
RUNNER = os.environ.get("XRMM_EXECUTE") or os.path.join(ROOT, "xrgpu_amd", "lib", "xrmm_execute")


def run_job(tmp_path, job, name="job.json"):
    if not os.path.exists(RUNNER):
        pytest.fail("xrmm_execute is not built (python -m xrgpu_amd.build)")
    path = tmp_path / name
    path.write_text(json.dumps(job))
    r = subprocess.run([RUNNER, str(path)], capture_output=True, text=True, timeout=60)
    return r.returncode, r.stdout, r.stderr


def lit(name, arr, dtype=None, storage=None):
    arr = np.asarray(arr)
    t = {"name": name, "dtype": dtype or str(arr.dtype), "shape": list(arr.shape), "values": arr.tolist()}
    if storage:
        t["storage_dtype"] = storage
    return t


def mnb_job(M=2, K=64, N=8, bs=32):
    kb = K // bs
    return {"operation": "com.microsoft.MatMulNBits", "package": "",
            "inputs": [lit("aT", np.zeros((M, K), np.float32), "float16", "float32"),
                       lit("bT", np.zeros((N, kb, bs // 2), np.uint8)),
                       lit("scalesT", np.ones((N, kb), np.float32), "float16", "float32"), None],
            "attrs": {"K": K, "N": N, "block_size": bs}, "plan_only": True}


def test_plan_only_literals(tmp_path):
    rc, out, err = run_job(tmp_path, mnb_job())
    assert rc == 0, err
    ans = json.loads(out)
    assert ans["planned_outputs"] == [{"name": "yT", "dtype": "float16", "storage_dtype": "float16", "shape": [2, 8],
                                       "layout": "contiguous"}]
    assert ans["outputs"] == ans["planned_outputs"]
    assert ans["info"]["backend"] == "host_shape_plan" and ans["info"]["test_only"] is True
    assert ans["info"]["physical_qualification"] is False and ans["info"]["operation"] == "com.microsoft.MatMulNBits"


def test_plan_only_files_args_and_requested_storage(tmp_path):
    T_, H, I, E = 3, 64, 32, 4
    arrays = {"inputT": np.zeros((T_, H), np.float32), "routerT": np.zeros((T_, E), np.float32),
              "fc1T": np.zeros((E, I, H // 2), np.uint8), "fc1ScalesT": np.zeros((E, I), np.float32),
              "fc2T": np.zeros((E, H, I // 2), np.uint8), "fc2ScalesT": np.zeros((E, H), np.float32)}
    inputs = []
    for n, a in arrays.items():
        a.tofile(tmp_path / f"{n}.bin")
        inputs.append({"name": n, "dtype": str(a.dtype), "shape": list(a.shape), "file": f"{n}.bin"})
    job = {"operation": "com.microsoft.QMoE", "package": "", "inputs": inputs, "plan_only": True,
           "attrs": {"k": 1, "activation_type": "relu"}, "args": {"k": 2},
           "outputs": [{"name": "outputT", "dtype": "float32", "shape": [T_, H]}]}
    rc, out, err = run_job(tmp_path, job)
    assert rc == 0, err
    assert json.loads(out)["planned_outputs"][0]["shape"] == [T_, H]
    job["args"] = {"k": 5}  # args override attrs, and k > E fails the planner
    rc, out, err = run_job(tmp_path, job)
    assert rc == 1 and json.loads(err) == {"error": "Invalid MoE input or routing geometry", "physical_qualification": False}


@pytest.mark.parametrize("mutate,msg", [
    (lambda j: j.pop("operation"), "Missing JSON key: operation"),
    (lambda j: j["attrs"].update(bits=3), "bits must be 2, 4 or 8"),
    (lambda j: j["inputs"][1].update(values=[1, 2, 3]), "Literal tensor value count mismatch"),
    (lambda j: j["inputs"][1].update(dtype="complex64"), "Unsupported dtype: complex64"),
    (lambda j: j["attrs"].update(extra=[1, 2]), "Unsupported native attribute encoding: extra"),
    (lambda j: j["inputs"][1].update(values=None, file="missing.bin"), "Tensor file byte count mismatch"),
])
def test_errors_are_json_on_stderr(tmp_path, mutate, msg):
    job = mnb_job()
    mutate(job)
    if job.get("inputs") and job["inputs"][1].get("values") is None:
        job["inputs"][1].pop("values", None)
    rc, out, err = run_job(tmp_path, job)
    assert rc == 1 and out == ""
    e = json.loads(err)
    assert msg in e["error"] and e["physical_qualification"] is False


def test_malformed_json(tmp_path):
    path = tmp_path / "bad.json"
    path.write_text('{"operation": "x", ')
    r = subprocess.run([RUNNER, str(path)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "Invalid invocation JSON" in json.loads(r.stderr)["error"]
    r = subprocess.run([RUNNER], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "Usage" in json.loads(r.stderr)["error"]


def _fuzz_cases():
    """Seeded malformed job files: every truncation point of a valid job (every
    7th byte), single-byte substitutions with JSON-significant characters,
    and hand-picked hostile inputs (deep nesting, huge numbers, bad escapes,
    bytes that are not UTF-8, oversized shapes)."""
    base = json.dumps(mnb_job(M=1, K=32, N=2, bs=32)).encode()
    rng = np.random.default_rng(20261202)
    cases = [base[:n] for n in range(0, len(base), 7)]
    subs = b'{}[]",:\\0-eE.+ \x00\xff'
    for _ in range(60):
        b = bytearray(base)
        i = int(rng.integers(len(b)))
        b[i] = subs[int(rng.integers(len(subs)))]
        cases.append(bytes(b))
    cases += [
        b"[" * 200000, b"{\"a\":" * 100000, b"\"" + b"\\" * 99999, b"1e99999", b"-", b"-0e-99999",
        b"{\"operation\": \"\\ud800\"}", b"{\"operation\": \"\\u00zz\"}", b"{\"operation\": \"\x80\xfe\"}",
        b"{\"operation\": 1e400, \"inputs\": [], \"attrs\": {}}",
        base.replace(b"[1, 64]", b"[4294967297, 4294967297]").replace(b"\"shape\": [1, 32]",
                                                                       b"\"shape\": [9223372036854775807, 3]"),
        base.replace(b"\"N\": 2", b"\"N\": -1"), base.replace(b"\"N\": 2", b"\"N\": 1.5e300"),
        base.replace(b"\"block_size\": 32", b"\"block_size\": 0"),
        base + b" trailing", b"\xef\xbb\xbf" + base, b"",
    ]
    return cases


def test_parser_fuzz_never_crashes(tmp_path):
    """The runner reads untrusted job files: every malformed input ends in exit
    status 0 or 1 with a JSON error object, never in a signal (the same test
    runs against the AddressSanitizer / UBSan build of the runner)."""
    if not os.path.exists(RUNNER):
        pytest.fail("xrmm_execute is not built (python -m xrgpu_amd.build)")
    path = tmp_path / "fuzz.json"
    for i, data in enumerate(_fuzz_cases()):
        path.write_bytes(data)
        r = subprocess.run([RUNNER, str(path)], capture_output=True, timeout=60)
        assert r.returncode in (0, 1), (i, data[:80], r.returncode, r.stderr[-400:])
        if r.returncode == 1:
            assert "error" in json.loads(r.stderr.decode("utf-8", "replace")), (i, r.stderr[-200:])
