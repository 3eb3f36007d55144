"""Build libxrmm.so for gfx950 in-tree with hipcc.

``python -m xrgpu_amd.build`` compiles ``xrgpu_amd/csrc`` into
``xrgpu_amd/lib/libxrmm.so``. Translation units compile in parallel (the GEMV
family once per zero-point kind) into ``xrgpu_amd/_build`` and are linked into
one shared library. It cross-compiles without a GPU.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ_DIR = os.path.join(HERE, "_build")
LIB_DIR = os.path.join(HERE, "lib")
LIB = os.path.join(LIB_DIR, "libxrmm.so")
RUNNER = os.path.join(LIB_DIR, "xrmm_execute")  # job-JSON runner over the C ABI
ARCH = os.environ.get("XRMM_OFFLOAD_ARCH", "gfx950")

# (source, extra defines, object name)
UNITS = [
    ("xrmm_kernels.hip", [], "kernels.o"),
    ("xrmm_gemv_zp.hip", ["-DXRMM_ZPK=0"], "gemv_zp0.o"),
    ("xrmm_gemv_zp.hip", ["-DXRMM_ZPK=1"], "gemv_zp1.o"),
    ("xrmm_gemv_zp.hip", ["-DXRMM_ZPK=2"], "gemv_zp2.o"),
    ("xrmm_gemv_dot_zp.hip", ["-DXRMM_ZPK=0"], "dot_zp0.o"),
    ("xrmm_gemv_dot_zp.hip", ["-DXRMM_ZPK=1"], "dot_zp1.o"),
    ("xrmm_gemv_dot_zp.hip", ["-DXRMM_ZPK=2"], "dot_zp2.o"),
    ("xrmm_gemv_mq_zp.hip", ["-DXRMM_ZPK=0"], "mq_zp0.o"),
    ("xrmm_gemv_mq_zp.hip", ["-DXRMM_ZPK=2"], "mq_zp2.o"),
    ("xrmm_gemv_f32_zp.hip", ["-DXRMM_ZPK=0"], "f32_zp0.o"),
    ("xrmm_gemv_f32_zp.hip", ["-DXRMM_ZPK=1"], "f32_zp1.o"),
    ("xrmm_gemv_f32_zp.hip", ["-DXRMM_ZPK=2"], "f32_zp2.o"),
    ("xrmm_gemv_sk_zp.hip", ["-DXRMM_ZPK=0"], "sk_zp0.o"),
    ("xrmm_gemv_sk_zp.hip", ["-DXRMM_ZPK=1"], "sk_zp1.o"),
    ("xrmm_gemv_sk_zp.hip", ["-DXRMM_ZPK=2"], "sk_zp2.o"),
    ("xrmm_gemm_zp.hip", ["-DXRMM_ZPK=0"], "gemm_zp0.o"),
    ("xrmm_gemm_zp.hip", ["-DXRMM_ZPK=1"], "gemm_zp1.o"),
    ("xrmm_gemm_zp.hip", ["-DXRMM_ZPK=2"], "gemm_zp2.o"),
    ("xrmm_gemm_fused_zp.hip", ["-DXRMM_ZPK=0"], "fused_zp0.o"),
    ("xrmm_gemm_fused_zp.hip", ["-DXRMM_ZPK=1"], "fused_zp1.o"),
    ("xrmm_gemm_fused_zp.hip", ["-DXRMM_ZPK=2"], "fused_zp2.o"),
    ("xrmm_gemm_f32x.hip", [], "gemm_f32x.o"),
    ("xrmm_gemm_f32x_h.hip", [], "gemm_f32x_h.o"),
    ("xrmm_f32_split.hip", [], "f32_split.o"),
    ("xrmm_moe.hip", [], "moe.o"),
    ("xrmm_quant.hip", [], "quant.o"),
    ("xrmm_int8a.hip", [], "int8a.o"),
    ("xrmm_probe.hip", [], "probe.o"),
    ("xrmm_api.cpp", [], "api.o"),
    ("xrmm_operator.cpp", [], "operator.o"),
]

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # keep packed-fp32 VALU forms out of the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed: " + " ".join(cmd[-3:]))
    noise = [ln for ln in res.stderr.splitlines() if ln.strip() and "packed-fp32-ops" not in ln]
    if verbose and noise:
        sys.stderr.write("\n".join(noise) + "\n")


def build(verbose: bool = False, jobs: int | None = None) -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    os.makedirs(OBJ_DIR, exist_ok=True)
    cc = hipcc()
    inc = ["-I", os.path.join(ROOT, "include"), "-I", CSRC]
    units = [(os.path.join(CSRC, src), defs, os.path.join(OBJ_DIR, obj)) for src, defs, obj in UNITS
             if os.path.exists(os.path.join(CSRC, src))]
    cmds = [[cc, *FLAGS, *inc, *defs, "-c", src, "-o", obj] for src, defs, obj in units]
    jobs = jobs or min(len(cmds), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB + ".tmp"
    _run([cc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *[obj for _, _, obj in units], "-o", tmp], verbose)
    os.replace(tmp, LIB)
    # the runner is host code only: the system C++ compiler, linked to the
    # library beside it
    cxx = shutil.which("g++") or shutil.which("c++") or cc
    _run([cxx, "-O2", "-std=c++17", "-Wall", "-I", os.path.join(ROOT, "include"), os.path.join(CSRC, "xrmm_execute.cpp"),
          "-L", LIB_DIR, "-lxrmm", "-Wl,-rpath,$ORIGIN", "-o", RUNNER + ".tmp"], verbose)
    os.replace(RUNNER + ".tmp", RUNNER)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
