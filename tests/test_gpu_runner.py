"""GPU: full jobs through the job-JSON runner (xrgpu_amd/lib/xrmm_execute, the
wire format of kernels/_shared/extended/tests/execute.cpp:14-35): inputs as
raw files and as literals (float16 literals converted once from double),
repeat, profiling, output files read back and checked against the oracle."""
import json
import os
import subprocess

import numpy as np
import pytest

from oracle import moe as QM
from oracle import oracle as O
from oracle import quant as Q

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RUNNER = os.path.join(ROOT, "xrgpu_amd", "lib", "xrmm_execute")


def file_tensor(tmp, name, arr, dtype=None):
    arr = np.ascontiguousarray(arr)
    arr.tofile(tmp / f"{name}.bin")
    return {"name": name, "dtype": dtype or str(arr.dtype), "shape": list(arr.shape), "file": f"{name}.bin"}


def run(tmp, job):
    job = dict(job, package="", output_directory="out")
    (tmp / "job.json").write_text(json.dumps(job))
    r = subprocess.run([RUNNER, str(tmp / "job.json")], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    ans = json.loads(r.stdout)
    outs = []
    for d in ans["outputs"]:
        outs.append(np.fromfile(d["file"], dtype=np.dtype(d["storage_dtype"])).reshape(d["shape"]))
    return ans, outs


def test_matmul_nbits_literals_fp16(gpu, tmp_path):
    rng = np.random.default_rng(1)
    M, K, N, bs = 2, 128, 16, 32
    a = rng.standard_normal((M, K))
    b = rng.integers(0, 256, (N, K // bs, bs // 2), dtype=np.uint8)
    s = rng.uniform(0.01, 0.05, (N, K // bs))
    job = {"operation": "com.microsoft.MatMulNBits",
           "inputs": [{"name": "aT", "dtype": "float16", "shape": [M, K], "values": a.tolist()},
                      file_tensor(tmp_path, "bT", b),
                      {"name": "scalesT", "dtype": "float16", "shape": [N, K // bs], "values": s.tolist()}],
           "attrs": {"K": K, "N": N, "block_size": bs}, "repeat": 3, "profiling": True}
    ans, (y,) = run(tmp_path, job)
    assert ans["info"]["backend"] == "hip" and ans["info"]["gpu_ms"] > 0 and ans["info"]["executed"] is True
    ref = O.matmul_nbits(a.astype(np.float16), b, s.astype(np.float16), K=K, N=N, block_size=bs)
    ok, err, lim = O.tolerance_ok(y, ref, np.float16)
    assert y.dtype == np.float16 and ok, (err, lim)


def test_qmoe_files(gpu, tmp_path):
    rng = np.random.default_rng(2)
    T_, H, I, E = 4, 128, 64, 4
    ins = dict(inputT=rng.standard_normal((T_, H)).astype(np.float32),
               routerT=rng.standard_normal((T_, E)).astype(np.float32),
               fc1T=rng.integers(0, 256, (E, 2 * I, H // 2), dtype=np.uint8),
               fc1ScalesT=rng.uniform(0.01, 0.05, (E, 2 * I)).astype(np.float32),
               fc2T=rng.integers(0, 256, (E, H, I // 2), dtype=np.uint8),
               fc2ScalesT=rng.uniform(0.01, 0.05, (E, H)).astype(np.float32))
    job = {"operation": "com.microsoft.QMoE", "inputs": [file_tensor(tmp_path, n, a) for n, a in ins.items()],
           "attrs": {"k": 2, "activation_type": "swiglu", "swiglu_fusion": 1}}
    ans, (y,) = run(tmp_path, job)
    ref = QM.qmoe(*ins.values(), k=2, activation="swiglu", swiglu_fusion=1)
    ok, err, lim = O.tolerance_ok(y, ref, np.float32)
    assert ok, (err, lim)


def test_gbq_and_bnb4_files(gpu, tmp_path):
    rng = np.random.default_rng(3)
    data = rng.integers(0, 256, (20, 32), dtype=np.uint8)
    scales = rng.uniform(-1, 1, (20, 4)).astype(np.float32)
    idx = np.array([19, 0, 7], np.int64)
    job = {"operation": "com.microsoft.GatherBlockQuantized",
           "inputs": [file_tensor(tmp_path, "dataT", data), file_tensor(tmp_path, "indicesT", idx),
                      file_tensor(tmp_path, "scalesT", scales)], "attrs": {"bits": 4, "block_size": 16}}
    _, (y,) = run(tmp_path, job)
    assert np.array_equal(y, Q.gather_block_quantized(data, idx, scales, bits=4, block_size=16))
    M, K, N, bs = 3, 256, 40, 64
    a = rng.standard_normal((M, K)).astype(np.float32)
    b = rng.integers(0, 256, N * K // 2, dtype=np.uint8)
    am = rng.uniform(0.1, 1, N * K // bs).astype(np.float32)
    job = {"operation": "com.microsoft.MatMulBnb4",
           "inputs": [file_tensor(tmp_path, "aT", a), file_tensor(tmp_path, "bT", b),
                      file_tensor(tmp_path, "absmaxT", am)], "attrs": {"K": K, "N": N, "block_size": bs}}
    _, (y,) = run(tmp_path, job)
    ok, err, lim = O.tolerance_ok(y, Q.matmul_bnb4(a, b, am, K=K, N=N, block_size=bs), np.float32)
    assert ok, (err, lim)
